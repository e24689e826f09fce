"""GPU parity of bq_gemv_norm_fused: a q8 producer (norm / add / resid / gate /
silu*mul, then the row L2 norm and q8) and the GEMV of its row in one launch.

Reference: the two launches it replaces -- the standalone producer
(bq_*_q8, pinned against the oracle in test_gpu_norm.py) followed by
bq_gemv_q8_fused on the producer's fp32 row.  The emitted fp32 row and its q8
row must be bit-identical to that pair; the GEMV outputs agree to fp32
summation order (normwise < 1e-6: the K split may differ) and are checked
against the oracle on the q8 codes (normwise < 1e-4).
"""
import numpy as np
import pytest

from helpers import dev, host, weights

pytestmark = pytest.mark.gpu

# (op, weight format, K, N per part, parts)
CASES = [
    ("resid", "q5k", 3072, 9216, 2),    # gate+up after the attention residual
    ("gate", "q5k", 4096, 3072, 1),     # O projection after the attention gate
    ("silu", "q6k", 9216, 3072, 1),     # down projection
    ("norm", "q6k_rep", 3072, 4096, 1), # final norm + head-like GEMV, W160 repack
    ("add", "q5k", 256, 64, 1),
    ("resid", "q5k", 5120, 512, 1),     # 5 chunks: a 16-wave workgroup
    ("silu", "q6k", 16384, 256, 1),     # the largest row
    ("norm", "q5k", 1280, 640, 3),
    ("resid", "q5k", 2560, 7168, 2),    # gate+up at the reference model's hidden size (3 chunks, the last half full)
    ("resid", "q5k", 2560, 4096, 3),    # q / k / gate parts at that size
]


def _inputs(oracle, op, K, seed):
    g = lambda s, m, sd: oracle.gaussian(seed + s, K, m, sd).astype(np.float32)
    a = g(0, 0.0, 1.0)
    b = g(1, 0.0, 2.0)
    if op == "resid":
        c = np.random.default_rng(seed).uniform(0.0, 1.0, K).astype(np.float32)
    else:
        c = g(2, 1.0, 0.3)
    d = g(3, 1.0, 0.3)
    used = {"norm": 1, "add": 2, "resid": 3, "gate": 3, "silu": 4}[op]
    return [a, b, c, d][:used]


def _weights(bq, oracle, fmt, K, N, seed):
    import torch
    raw = weights(seed, N, K, "q5k" if fmt == "q5k" else "q6k")
    draw = dev(raw)
    if fmt == "q5k":
        return raw, bq.make_weight(draw, bq.TYPE_Q5_K, K, N)
    if fmt == "q6k":
        return raw, bq.make_weight(draw, bq.TYPE_Q6_K, K, N)
    rep = bq.repack_q6k(draw, K, N)
    return raw, bq.make_weight(draw, bq.TYPE_Q6_K, K, N, rep=rep)


@pytest.mark.parametrize("op,fmt,K,N,parts", CASES)
def test_producer_gemv_matches_two_launches(bq, oracle, op, fmt, K, N, parts):
    import torch
    print(f"producer {op} {fmt} K={K} N={N} parts={parts}", flush=True)
    seed = 300 + K // 256 + parts
    ins = _inputs(oracle, op, K, seed)
    W = [_weights(bq, oracle, fmt, K, N, seed + 10 + p) for p in range(parts)]
    ws = [w for _, w in W]
    dins = [dev(v) for v in ins]
    # --- two launches: producer, then the fused-quantize GEMV on its fp32 row
    q8a = (torch.empty(K, dtype=torch.int8, device="cuda"), torch.empty(K // 32, device="cuda"),
           torch.empty(K // 32, dtype=torch.int32, device="cuda"))
    args = dict(zip("abcd", [t.view(1, K) for t in dins]))
    if op in ("add", "resid"):
        xin = dins[0].clone()
        args["a"] = xin.view(1, K)
        bq.norm_q8(op, 1, K, q8=q8a, **args)
        row1 = xin
    else:
        row1 = torch.empty(K, device="cuda")
        bq.norm_q8(op, 1, K, out=row1.view(1, K), q8=q8a, **args)
    y1 = [torch.empty(N, device="cuda") for _ in range(parts)]
    assert bq.gemv_q8_fused(y1, ws, row1) == bq.BQ_OK
    # --- one launch
    out = torch.full((K,), float("nan"), device="cuda")
    q8b = (torch.empty(K, dtype=torch.int8, device="cuda"), torch.empty(K // 32, device="cuda"),
           torch.empty(K // 32, dtype=torch.int32, device="cuda"))
    y2 = [torch.full((N,), float("nan"), device="cuda") for _ in range(parts)]
    pad = dins + [None] * (4 - len(dins))
    assert bq.gemv_norm_fused(y2, ws, op, pad[0], pad[1], pad[2], pad[3], out=out, q8=q8b) == bq.BQ_OK
    torch.cuda.synchronize()
    assert np.array_equal(host(out).view(np.uint32), host(row1).view(np.uint32))
    for u, v in zip(q8a, q8b):
        assert np.array_equal(host(u), host(v))
    # the GEMV may split K differently from bq_gemv_q8_fused (the producer
    # path keeps the fewest workgroups): same terms, fp32 summation order
    for p in range(parts):
        assert oracle.normwise_err(host(y2[p])[None], host(y1[p])[None]) < 1e-6, p
    # --- oracle on the q8 codes
    xq, xd, xs = (host(t).reshape(1, -1) for t in q8b)
    for p, (raw, _) in enumerate(W):
        ref = oracle.gemm_q5k(raw, xq, xd, xs) if fmt == "q5k" else oracle.gemm_q6k(raw, xq, xd)
        assert oracle.normwise_err(host(y2[p])[None], ref) < 1e-4


def test_producer_gemv_without_outputs(bq, oracle):
    """out and the q8 row are optional; the GEMV result does not depend on them."""
    import torch
    K, N = 3072, 1024
    ins = [dev(v) for v in _inputs(oracle, "silu", K, 5)]
    raw, w = _weights(bq, oracle, "q5k", K, N, 6)
    y1, y2 = torch.empty(N, device="cuda"), torch.empty(N, device="cuda")
    out = torch.empty(K, device="cuda")
    assert bq.gemv_norm_fused([y1], [w], "silu", *ins, out=out) == bq.BQ_OK
    assert bq.gemv_norm_fused([y2], [w], "silu", *ins) == bq.BQ_OK
    torch.cuda.synchronize()
    assert np.array_equal(host(y1), host(y2))


def test_producer_gemv_rejects(bq, oracle):
    import torch
    K = 256
    a, b, c = (dev(v) for v in _inputs(oracle, "resid", K, 7))
    _, w = _weights(bq, oracle, "q5k", K, 64, 8)
    y = torch.empty(64, device="cuda")
    with pytest.raises(bq.BqError):
        bq.gemv_norm_fused([y], [w], "resid", a, b, c, out=a)       # out aliases an input
    with pytest.raises(bq.BqError):
        bq.gemv_norm_fused([y], [w], "add", a)                      # add without h
    big = torch.zeros(16640 // 256 * 176 * 4, dtype=torch.uint8, device="cuda")
    wb = bq.make_weight(big, bq.TYPE_Q5_K, 16640, 4)
    xb = torch.zeros(16640, device="cuda")
    assert bq.gemv_norm_fused([torch.empty(4, device="cuda")], [wb], "norm", xb) == bq.BQ_UNSUPPORTED
