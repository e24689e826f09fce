"""GPU parity of the q8 producers (bq_norm_q8, bq_add_norm_q8, bq_resid_q8,
bq_gate_norm_q8, bq_silu_mul_norm_q8): the reference's norm kernels that emit
the GEMV's q8 activations (bruce.cu:541-641, 1110-1228, 1427-1572).

- fp32 rows: within TOL_F32 of the float64 oracle, normwise per row (the
  reference's fast __expf is replaced by expf, and the sums of squares are
  reduced in a different order, so agreement is to rounding).
- q8 rows: bit-exact with the oracle quantizer applied to the emitted fp32 row.
  This is the "stays bit-identical to the standalone quantizer" requirement.
- dst = NULL gives the same q8 rows.
"""
import numpy as np
import pytest

from helpers import dev, host

pytestmark = pytest.mark.gpu
TOL_F32 = 2e-6


def inputs(oracle, op, rows, n, seed):
    g = lambda s, r, mean=0.0, std=1.0: oracle.gaussian(seed * 10 + s, r * n, mean, std).reshape(r, n)
    a = g(1, rows)
    if op == "norm":
        return [a]
    if op == "add":
        return [a, g(2, rows)]
    if op == "resid":
        return [a, g(2, rows, 0.0, 3.0), oracle.gaussian(seed * 10 + 3, n, 0.5, 0.3)]
    if op == "gate":
        return [a, g(2, rows, 0.0, 2.0), oracle.gaussian(seed * 10 + 3, n, 1.0, 0.3)]
    return [g(1, rows, 0.0, 2.0), a, oracle.gaussian(seed * 10 + 3, n, 1.0, 0.3),
            oracle.gaussian(seed * 10 + 4, n, 1.0, 0.3)]


def run(bq, op, ins, rows, n, with_out=True):
    import torch
    d = [dev(t) for t in ins]
    out = None
    if op in ("add", "resid"):
        out = d[0]                      # in place
    elif with_out:
        out = torch.full((rows, n), float("nan"), device="cuda")
    args = dict(out=out, a=d[0])
    for k, t in zip("bcd", d[1:]):
        args[k] = t
    r, (xq, xd, xs) = bq.norm_q8(op, rows, n, **args)
    assert r == bq.BQ_OK
    torch.cuda.synchronize()
    return (host(out) if out is not None else None), host(xq), host(xd), host(xs)


CASES = [(1, 32), (1, 2560), (1, 3072), (1, 4096), (1, 7168), (1, 9216), (3, 20480), (8, 3072), (5, 32768),
         (64, 9216)]


@pytest.mark.parametrize("op", ["norm", "add", "resid", "gate", "silu"])
@pytest.mark.parametrize("rows,n", CASES)
def test_norm_q8(bq, oracle, op, rows, n):
    print(f"norm_q8 {op} rows={rows} n={n}", flush=True)
    ins = inputs(oracle, op, rows, n, rows + n)
    out, xq, xd, xs = run(bq, op, ins, rows, n)
    ref = oracle.norm_rows(op, *ins)
    assert oracle.normwise_err(out, ref) < TOL_F32
    rq, rd, rs = oracle.q8_rows(out)
    assert np.array_equal(xq, rq)
    assert np.array_equal(xd.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(xs, rs)
    if op in ("norm", "gate", "silu"):
        _, xq2, xd2, xs2 = run(bq, op, ins, rows, n, with_out=False)
        assert np.array_equal(xq2, xq) and np.array_equal(xd2, xd) and np.array_equal(xs2, xs)


def test_norm_q8_prefill_rows(bq, oracle):
    """2048 rows x 3072 (a prompt batch): sampled rows against the oracle."""
    rows, n = 2048, 3072
    ins = inputs(oracle, "resid", rows, n, 77)
    out, xq, xd, xs = run(bq, "resid", ins, rows, n)
    idx = np.array([0, 1, 777, 2046, 2047])
    ref = oracle.norm_rows("resid", ins[0][idx], ins[1][idx], ins[2])
    assert oracle.normwise_err(out[idx], ref) < TOL_F32
    rq, _, _ = oracle.q8_rows(out)
    assert np.array_equal(xq, rq)


def test_norm_q8_zero_row(bq, oracle):
    """An all-zero row stays zero (eps keeps the scale finite); q8 is all zero."""
    out, xq, xd, xs = run(bq, "norm", [np.zeros((1, 256), np.float32)], 1, 256)
    assert np.all(out == 0) and np.all(xq == 0) and np.all(xd == 0) and np.all(xs == 0)


def test_norm_q8_rejects(bq):
    import torch
    a = torch.zeros((1, 32800), device="cuda")
    xq = torch.zeros((1, 32800), dtype=torch.int8, device="cuda")
    xd = torch.zeros((1, 32800 // 32), device="cuda")
    xs = torch.zeros((1, 32800 // 32), dtype=torch.int32, device="cuda")
    q8 = (xq, xd, xs)
    with pytest.raises(bq.BqError):
        bq.norm_q8("norm", 1, 48, out=a, a=a, q8=q8)           # n % 32
    assert bq.norm_q8("norm", 1, 32800, out=a, a=a, q8=q8)[0] == bq.BQ_UNSUPPORTED
    with pytest.raises(bq.BqError):
        bq.norm_q8("resid", 1, 64, a=a, b=a, q8=q8)            # alpha missing
