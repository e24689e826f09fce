"""Seeded random shapes through the prefill dispatchers, against the oracle.

The hand-picked cases elsewhere pin each tier at chosen shapes; this sweep
draws (weight format, parts, K, N per part, rows) from a fixed-seed generator
so that shapes nobody picked cross every dispatch boundary of bq_gemm_b /
bq_gemm_b_fused (engine/src/bruce.cu:7423-7426 launch_gemm_b_fused, 7429
launch_gemm_b):
  * rows 1..8: the multi-row GEMV, in 8-row chunks above;
  * rows > 8 and every N a multiple of 128: the MMQ tile (Q5_K, both tiers)
    or the W160 GEMM (Q6_K prepacked);
  * rows > 8 with some N off the 128 grid: bq_gemm_b per part (the GEMV
    chunks for the parts off the grid, the tile for the others);
  * prepacked Q5_K with K not a multiple of 512: the raw tier, not W144.
The decode-side fused entries get the same treatment: bq_gemv_q8_fused at
random K (up to 20480), ragged N per part and 1..4 parts (q8 row bit-exact
with the oracle quantizer, y against the oracle GEMV), and the producer fold
bq_gemv_norm_fused at random op, format, K and N (its checks are
test_gpu_producer's: the pair it replaces, then the oracle).
The expected tier is derived from the shape here and the oracle of that tier
is the reference (the W144 tier's fp16 min term, bruce.cu:6604-6792, is
evaluated by oracle.gemm_q5k_144).  Tolerance: helpers.check (normwise 1e-4,
elementwise 1e-3 with a 1e-2 floor).
"""
import numpy as np
import pytest

from helpers import acts, check, dev, host, weights

pytestmark = pytest.mark.gpu

N_CASES = 64
N_DECODE = 32


def _draw(i):
    """Case i's shape, a pure function of i."""
    r = np.random.default_rng(90210 + i)
    fmt = ["q5k", "q5k_rep", "q6k", "q6k_rep"][i % 4]
    K = 256 * int(r.integers(1, 13))
    cls = int(r.integers(0, 3))
    rows = int(r.integers(1, 9)) if cls == 0 else int(r.integers(9, 97)) if cls == 1 else int(r.integers(97, 301))
    nparts = int(r.integers(1, 5)) if fmt.startswith("q5k") else 1
    on_grid = r.random() < 0.7
    Ns = [128 * int(r.integers(1, 4)) if on_grid else 16 * int(r.integers(1, 25)) for _ in range(nparts)]
    return fmt, K, Ns, rows


CASES = [_draw(i) for i in range(N_CASES)]


@pytest.mark.parametrize("fmt,K,Ns,rows", CASES, ids=[f"{c[0]}-K{c[1]}-N{'_'.join(map(str, c[2]))}-r{c[3]}"
                                                     for c in CASES])
def test_dispatch_sweep(bq, oracle, fmt, K, Ns, rows):
    import torch
    print(f"sweep {fmt} K={K} Ns={Ns} rows={rows}", flush=True)
    q5 = fmt.startswith("q5k")
    rep = fmt.endswith("_rep")
    seed = 5000 + K + 7 * rows + sum(Ns)
    raws = [weights(seed + p, n, K, "q5k" if q5 else "q6k") for p, n in enumerate(Ns)]
    _, (xq, xd, xs) = acts(seed + 99, rows, K)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        if q5:
            if rep:
                w144, dm = bq.repack_q5k(g, K, n)
                ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n, rep=w144, rep_min=dm))
            else:
                ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q6_K, K, n, rep=bq.repack_q6k(g, K, n) if rep else None))
    ys = [torch.full((rows, n), float("nan"), device="cuda") for n in Ns]
    if len(ws) > 1:
        bq.gemm_b_fused(ys, ws, rows, gq, gd, gs, xdh)
    else:
        bq.gemm_b(ys[0], ws[0], rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    for r, n, y in zip(raws, Ns, ys):
        # per part: a fused call with any N off the grid falls back to
        # bq_gemm_b per part, which takes the tile for the parts on the grid
        w144_tier = q5 and rep and rows > 8 and K % 512 == 0 and n % 128 == 0
        if not q5:
            ref = oracle.gemm_q6k(r, xq, xd)
        elif w144_tier:
            r144, rdm = oracle.repack_q5k_144(r, K)
            ref = oracle.gemm_q5k_144(r144, rdm, xq, xd, oracle.fill_xdh(xd, xs), n)
        else:
            ref = oracle.gemm_q5k(r, xq, xd, xs)
        yh = host(y)
        assert np.isfinite(yh).all(), "unwritten outputs"
        check(oracle, yh, ref, what=f"N={n} w144={w144_tier}")


def _draw_decode(i):
    r = np.random.default_rng(31337 + i)
    fmt = ["q5k", "q6k", "q6k_rep"][i % 3]
    K = 256 * int(r.integers(1, 81))
    nparts = int(r.integers(1, 5))
    Ns = [16 * int(r.integers(1, 65)) for _ in range(nparts)]
    return fmt, K, Ns


DECODE = [_draw_decode(i) for i in range(N_DECODE)]


@pytest.mark.parametrize("fmt,K,Ns", DECODE, ids=[f"{c[0]}-K{c[1]}-N{'_'.join(map(str, c[2]))}" for c in DECODE])
def test_gemv_q8_fused_sweep(bq, oracle, fmt, K, Ns):
    import torch
    print(f"sweep gemv_q8_fused {fmt} K={K} Ns={Ns}", flush=True)
    seed = 7000 + K + sum(Ns)
    x, (xq, xd, xs) = acts(seed, 1, K)
    q5 = fmt == "q5k"
    raws = [weights(seed + 1 + p, n, K, "q5k" if q5 else "q6k") for p, n in enumerate(Ns)]
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        if q5:
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q6_K, K, n, rep=bq.repack_q6k(g, K, n) if fmt.endswith("rep") else None))
    ys = [torch.full((n,), float("nan"), device="cuda") for n in Ns]
    gq = torch.full((1, K), 99, dtype=torch.int8, device="cuda")
    gd = torch.full((1, K // 32), float("nan"), device="cuda")
    gs = torch.full((1, K // 32), -7, dtype=torch.int32, device="cuda")
    assert bq.gemv_q8_fused(ys, ws, dev(x), gq, gd, gs) == bq.BQ_OK
    torch.cuda.synchronize()
    assert np.array_equal(host(gq), xq)
    assert np.array_equal(host(gd).view(np.uint32), xd.view(np.uint32))
    assert np.array_equal(host(gs), xs)
    for r, n, y in zip(raws, Ns, ys):
        ref = oracle.gemm_q5k(r, xq, xd, xs) if q5 else oracle.gemm_q6k(r, xq, xd)
        check(oracle, host(y)[None], ref, what=f"N={n}")


def _draw_producer(i):
    r = np.random.default_rng(4242 + i)
    op = ["norm", "add", "resid", "gate", "silu"][i % 5]
    fmt = ["q5k", "q6k", "q6k_rep"][int(r.integers(0, 3))]
    return op, fmt, 256 * int(r.integers(1, 65)), 16 * int(r.integers(1, 65)), int(r.integers(1, 5))


PRODUCER = [_draw_producer(i) for i in range(20)]


@pytest.mark.parametrize("op,fmt,K,N,parts", PRODUCER)
def test_producer_sweep(bq, oracle, op, fmt, K, N, parts):
    from test_gpu_producer import test_producer_gemv_matches_two_launches as producer_case
    producer_case(bq, oracle, op, fmt, K, N, parts)
