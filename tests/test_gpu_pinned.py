"""GPU parity of the timed kernel instances and the reference model's shapes.

Every instance the benchmark times is checked here at the shape it is timed
at, and the shapes of the reference's own model (hidden 2560, FF 7168,
engine/src/bruce.cu:43-49, with its K = 2560 / 7168 Q6_K kernels
:4515-4581, :7307) are checked through every entry point that serves them.
The reference's GPU-side known-answer checks run through the production
GEMMs: "y = K" (tools/mmq_test.cu:311-334) and the unpacked-tile check
(:363-384), restated as one-hot activations that make the GEMM output the
transposed code tile.

Tolerance: bit-exact for codes and integer results; fp32 outputs against the
oracle (double precision) within max relative error 1e-4 normwise per
activation row, and, printed beside it, elementwise with a floor of 1e-2 x
the row's largest output within 1e-3, the reference's per-output bar
(helpers.check).
"""
import numpy as np
import pytest

from helpers import acts, check, dev, host, kat_q5k, kat_q6k, np_codes_q5k, np_codes_q6k, weights

pytestmark = pytest.mark.gpu


def _q8(oracle, x):
    xq, xd, xs = oracle.q8_rows(x)
    return (xq, xd, xs), (dev(xq), dev(xd), dev(xs))


def _nan(*shape):
    import torch
    return torch.full(shape, float("nan"), device="cuda")


# ---------------------------------------------------------------- timed decode instances
def test_headline_gate_up_fused(bq, oracle):
    """The headline launch: fused quantize + gate+up GEMV over 2 x 9216 x 3072
    Q5_K (the compile-time-K instance with three steps per wave, selected from
    20M weight values), as bench.py times it."""
    import torch
    K, N = 3072, 9216
    print("headline gate+up fused 2x9216x3072", flush=True)
    raws = [weights(2000 + i, N, K, "q5k") for i in range(2)]
    x, _ = acts(2002, 1, K)
    xq, xd, xs = oracle.q8_rows(x)
    ws = [bq.make_weight(dev(r), bq.TYPE_Q5_K, K, N) for r in raws]
    ys = [_nan(N), _nan(N)]
    gq = torch.full((1, K), 99, dtype=torch.int8, device="cuda")
    gd = _nan(1, K // 32)
    gs = torch.full((1, K // 32), -7, dtype=torch.int32, device="cuda")
    assert bq.gemv_q8_fused(ys, ws, dev(x), gq, gd, gs) == bq.BQ_OK
    torch.cuda.synchronize()
    assert np.array_equal(host(gq), xq)
    assert np.array_equal(host(gd).view(np.uint32), xd.view(np.uint32))
    assert np.array_equal(host(gs), xs)
    for i, (r, y) in enumerate(zip(raws, ys)):
        check(oracle, host(y)[None], oracle.gemm_q5k(r, xq, xd, xs), what=f"part {i}")


@pytest.mark.parametrize("rows", [1, 2, 4, 8])
def test_gate_up_verify(bq, oracle, rows):
    """bq_verify_fused over the 2 x 9216 x 3072 gate+up pair (q8 input): rows 1
    and 2 run the three-steps-per-wave instance (40M weight values), 4 the
    dot4 one, 8 the matrix-core one."""
    K, N = 3072, 9216
    print(f"gate+up verify rows={rows}", flush=True)
    raws = [weights(2010 + i, N, K, "q5k") for i in range(2)]
    x, _ = acts(2012 + rows, rows, K)
    (xq, xd, xs), g = _q8(oracle, x)
    ws = [bq.make_weight(dev(r), bq.TYPE_Q5_K, K, N) for r in raws]
    ys = [_nan(rows, N), _nan(rows, N)]
    assert bq.verify_fused(ys, ws, rows, *g) == bq.BQ_OK
    import torch
    torch.cuda.synchronize()
    for i, (r, y) in enumerate(zip(raws, ys)):
        check(oracle, host(y), oracle.gemm_q5k(r, xq, xd, xs), what=f"part {i}")


# ---------------------------------------------------------------- config 4 at M = 512 / 8192
@pytest.mark.parametrize("M", [512, 8192])
def test_config4_m(bq, oracle, M):
    """Config 4 (Q5_K 9216 x 3072) at M = 512 and 8192 through both tiers;
    64 token rows x 256 weight rows of the output are checked (the tokens
    spread over the whole range, including the last tile)."""
    import torch
    K, N = 3072, 9216
    print(f"config4 M={M}", flush=True)
    raw = weights(2100, N, K, "q5k")
    x, _ = acts(2101 + M, M, K)
    (xq, xd, xs), g = _q8(oracle, x)
    gr = dev(raw)
    w144, dm = bq.repack_q5k(gr, K, N)
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    rng = np.random.default_rng(M)
    mi = np.unique(np.concatenate([rng.choice(M, 62, replace=False), [0, M - 1]]))
    ni = np.unique(np.concatenate([rng.choice(N, 254, replace=False), [0, N - 1]]))
    sub = raw[ni]
    for prepacked in (False, True):
        w = bq.make_weight(gr, bq.TYPE_Q5_K, K, N, rep=w144 if prepacked else None,
                           rep_min=dm if prepacked else None)
        y = _nan(M, N)
        assert bq.try_mmq([y], [w], M, *g, xdh) == bq.BQ_OK
        torch.cuda.synchronize()
        yh = host(y)
        assert np.isfinite(yh).all()
        if prepacked:
            r144, rdm = oracle.repack_q5k_144(sub, K)
            ref = oracle.gemm_q5k_144(r144, rdm, xq[mi], xd[mi], oracle.fill_xdh(xd[mi], xs[mi]), len(ni))
        else:
            ref = oracle.gemm_q5k(sub, xq[mi], xd[mi], xs[mi])
        check(oracle, yh[np.ix_(mi, ni)], ref, what=f"prepacked={prepacked}")
        del y


# ---------------------------------------------------------------- Q6_K GEMM, both token-tile heights
@pytest.mark.parametrize("M", [96, 768, 1024])
def test_q6_gemm_tiles(bq, oracle, M):
    """The Q6_K GEMM over W160 at the down projection's shape (3072 x 9216)
    for row counts whose work estimate picks the 32-token tile (96, 1024) and
    the 128-token tile (768); 64 token rows x 256 weight rows checked."""
    import torch
    K, N = 9216, 3072
    print(f"q6 gemm M={M}", flush=True)
    raw = weights(2200, N, K, "q6k")
    x, _ = acts(2201 + M, M, K)
    (xq, xd, xs), g = _q8(oracle, x)
    gr = dev(raw)
    w = bq.make_weight(gr, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(gr, K, N))
    rng = np.random.default_rng(M + 1)
    mi = np.unique(np.concatenate([rng.choice(M, 62, replace=False), [0, M - 1]]))
    ni = np.unique(np.concatenate([rng.choice(N, 254, replace=False), [0, N - 1]]))
    y = _nan(M, N)
    bq.gemm_q6k_mma(y, w, M, g[0], g[1])
    torch.cuda.synchronize()
    yh = host(y)
    assert np.isfinite(yh).all()
    check(oracle, yh[np.ix_(mi, ni)], oracle.gemm_q6k(raw[ni], xq[mi], xd[mi]), what=f"M={M}")


# ---------------------------------------------------------------- the reference model's shapes
REF_SHAPES = [("q5k", 7168, 2560), ("q5k", 2560, 7168), ("q6k", 2560, 7168)]


@pytest.mark.parametrize("qt,N,K", REF_SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 6, 8])
def test_ref_shapes_gemv(bq, oracle, qt, N, K, rows):
    """Hidden 2560 / FF 7168: Q5_K gate/up (7168 x 2560), Q5_K and Q6_K down
    (2560 x 7168; raw blocks and W160), decode and verify row counts."""
    import torch
    print(f"ref shape {qt} {N}x{K} rows={rows}", flush=True)
    raw = weights(2200 + K + rows, N, K, qt)
    x, _ = acts(2201 + rows, rows, K)
    (xq, xd, xs), g = _q8(oracle, x)
    gr = dev(raw)
    if qt == "q5k":
        y = _nan(rows, N)
        assert bq.verify_fused([y], [bq.make_weight(gr, bq.TYPE_Q5_K, K, N)], rows, *g) == bq.BQ_OK
        torch.cuda.synchronize()
        check(oracle, host(y), oracle.gemm_q5k(raw, xq, xd, xs), what="verify")
    else:
        ref = oracle.gemm_q6k(raw, xq, xd)
        y = _nan(rows, N)
        bq.gemm_q6k_raw(y, bq.make_weight(gr, bq.TYPE_Q6_K, K, N), rows, g[0], g[1])
        torch.cuda.synchronize()
        check(oracle, host(y), ref, what="raw")
        y2 = _nan(rows, N)
        bq.gemm_q6k_dp(y2, bq.make_weight(gr, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(gr, K, N)), rows, g[0], g[1])
        torch.cuda.synchronize()
        check(oracle, host(y2), ref, what="W160")
    if rows == 1:
        # the fused quantize + GEMV form of the decode step
        tp = bq.TYPE_Q5_K if qt == "q5k" else bq.TYPE_Q6_K
        yf = _nan(N)
        assert bq.gemv_q8_fused([yf], [bq.make_weight(gr, tp, K, N)], dev(x[0])) == bq.BQ_OK
        torch.cuda.synchronize()
        ref = oracle.gemm_q5k(raw, xq, xd, xs) if qt == "q5k" else oracle.gemm_q6k(raw, xq, xd)
        check(oracle, host(yf)[None], ref, what="fused")


@pytest.mark.parametrize("qt,N,K", REF_SHAPES)
def test_ref_shapes_mmq(bq, oracle, qt, N, K):
    """The prefill GEMMs at the reference's shapes, M = 512 (all tiers), 64
    token rows x 256 weight rows checked."""
    import torch
    M = 512
    print(f"ref shape mmq {qt} {N}x{K}", flush=True)
    raw = weights(2300 + K, N, K, qt)
    x, _ = acts(2301 + K, M, K)
    (xq, xd, xs), g = _q8(oracle, x)
    gr = dev(raw)
    rng = np.random.default_rng(K)
    mi = np.sort(rng.choice(M, 64, replace=False))
    ni = np.sort(rng.choice(N, 256, replace=False))
    sub = raw[ni]
    if qt == "q6k":
        y = _nan(M, N)
        bq.gemm_q6k_mma(y, bq.make_weight(gr, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(gr, K, N)), M, g[0], g[1])
        torch.cuda.synchronize()
        check(oracle, host(y)[np.ix_(mi, ni)], oracle.gemm_q6k(sub, xq[mi], xd[mi]), what="q6k")
        return
    w144, dm = bq.repack_q5k(gr, K, N)
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    for prepacked in (False, True):
        w = bq.make_weight(gr, bq.TYPE_Q5_K, K, N, rep=w144 if prepacked else None,
                           rep_min=dm if prepacked else None)
        y = _nan(M, N)
        assert bq.try_mmq([y], [w], M, *g, xdh) == bq.BQ_OK
        torch.cuda.synchronize()
        if prepacked:
            r144, rdm = oracle.repack_q5k_144(sub, K)
            ref = oracle.gemm_q5k_144(r144, rdm, xq[mi], xd[mi], oracle.fill_xdh(xd[mi], xs[mi]), len(ni))
        else:
            ref = oracle.gemm_q5k(sub, xq[mi], xd[mi], xs[mi])
        check(oracle, host(y)[np.ix_(mi, ni)], ref, what=f"prepacked={prepacked}")


# ---------------------------------------------------------------- the reference's KATs on the GPU
def test_kat_y_equals_K_gemms(bq, oracle):
    """tools/mmq_test.cu:311-334 ("simple == 3"): every code 1, d = 1, dmin =
    0, unit scales, x = 1, xd = 1, xsum = 0, so every output is exactly K --
    through the raw-tier and W144 GEMMs (one and several token tiles, with
    and without the K split), the Q6_K GEMM (its own KAT block: q - 32 = 1)
    and every multi-row GEMV row count."""
    import torch
    K, N = 1024, 256
    r5, r6 = kat_q5k(N, K), kat_q6k(N, K)
    g5, g6 = dev(r5), dev(r6)
    w144, dm = bq.repack_q5k(g5, K, N)
    W5 = bq.make_weight(g5, bq.TYPE_Q5_K, K, N)
    W144 = bq.make_weight(g5, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm)
    W6 = bq.make_weight(g6, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g6, K, N))
    W6r = bq.make_weight(g6, bq.TYPE_Q6_K, K, N)
    for M in (96, 128, 300):
        xq = torch.ones((M, K), dtype=torch.int8, device="cuda")
        xd = torch.ones((M, K // 32), device="cuda")
        xs = torch.zeros((M, K // 32), dtype=torch.int32, device="cuda")
        xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
        for w in (W5, W144):
            for work in ("auto", None):
                y = _nan(M, N)
                assert bq.try_mmq([y], [w], M, xq, xd, xs, xdh, work=work) == bq.BQ_OK
                torch.cuda.synchronize()
                assert np.all(host(y) == K), (M, w is W144, work)
        for work in ("auto", None):
            y = _nan(M, N)
            bq.gemm_q6k_mma(y, W6, M, xq, xd, work=work)
            torch.cuda.synchronize()
            assert np.all(host(y) == K), (M, "q6k", work)
    xq = torch.ones((8, K), dtype=torch.int8, device="cuda")
    xd = torch.ones((8, K // 32), device="cuda")
    xs = torch.zeros((8, K // 32), dtype=torch.int32, device="cuda")
    for rows in range(1, 9):
        y = _nan(rows, N)
        assert bq.verify_fused([y], [W5], rows, xq, xd, xs) == bq.BQ_OK
        y6, y6r = _nan(rows, N), _nan(rows, N)
        bq.gemm_q6k_dp(y6, W6, rows, xq, xd)
        bq.gemm_q6k_raw(y6r, W6r, rows, xq, xd)
        torch.cuda.synchronize()
        for t in (y, y6, y6r):
            assert np.all(host(t) == K), rows


def _tile_weights(qt, N, K, seed):
    """Random codes under the KAT header (d = 1, dmin = 0, unit scales), so
    that a one-hot activation row selects one code exactly."""
    raw = weights(seed, N, K, qt)
    kat = kat_q5k(N, K) if qt == "q5k" else kat_q6k(N, K)
    b = raw.reshape(N, K // 256, -1).copy()
    k = kat.reshape(N, K // 256, -1)
    if qt == "q5k":
        b[:, :, 0:16] = k[:, :, 0:16]             # d, dmin, scales
    else:
        b[:, :, 192:210] = k[:, :, 192:210]       # scales, d
    return b.reshape(N, -1)


def test_unpacked_tile_bitexact(bq, oracle):
    """tools/mmq_test.cu:363-384 checks the kernel's unpacked int8 tile against
    host-decoded codes.  Restated through the production GEMMs: activation row
    m is one-hot at k = m with xd = 1 (xsum irrelevant with dmin = 0), weights
    have unit scales, so Y[m][n] is exactly the code of weight n at k = m --
    the whole unpacked (raw tier, in-kernel), repacked (W144) and Q6_K (W160)
    code matrix, transposed, bit for bit against the numpy decoders."""
    import torch
    K, N = 512, 256
    M = K
    r5 = _tile_weights("q5k", N, K, 2400)
    r6 = _tile_weights("q6k", N, K, 2401)
    c5 = np_codes_q5k(r5, K).T.astype(np.float32)
    c6 = (np_codes_q6k(r6, K) - 32).T.astype(np.float32)
    xq = torch.eye(M, K, dtype=torch.int8, device="cuda")
    xd = torch.ones((M, K // 32), device="cuda")
    xs = torch.zeros((M, K // 32), dtype=torch.int32, device="cuda")
    for g in range(K // 32):
        xs[32 * g:32 * g + 32, g] = 1
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    g5, g6 = dev(r5), dev(r6)
    w144, dm = bq.repack_q5k(g5, K, N)
    for w in (bq.make_weight(g5, bq.TYPE_Q5_K, K, N), bq.make_weight(g5, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm)):
        y = _nan(M, N)
        assert bq.try_mmq([y], [w], M, xq, xd, xs, xdh) == bq.BQ_OK
        torch.cuda.synchronize()
        assert np.array_equal(host(y), c5)
    y = _nan(M, N)
    bq.gemm_q6k_mma(y, bq.make_weight(g6, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g6, K, N)), M, xq, xd)
    torch.cuda.synchronize()
    assert np.array_equal(host(y), c6)
