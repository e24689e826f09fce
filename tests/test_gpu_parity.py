"""GPU parity of libbq (through its C ABI) against the CPU oracle.

Tolerance (stated by BASELINE's north star): integer dots, codes and repacked
layouts bit-exact; fp32 outputs within max relative error 1e-4, measured
normwise per activation row (max |y - ref| / max |ref| over the row), against
the oracle evaluated in double precision.
"""
import numpy as np
import pytest

from helpers import acts, check, dev, host, weights

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _xq_dev(xq, xd, xs):
    return dev(xq), dev(xd), dev(xs)


# ---------------------------------------------------------------- quantizer
@pytest.mark.parametrize("M,K", [(1, 3072), (3, 9216), (2048, 3072), (5, 32)])
def test_quantizer_bitexact(bq, oracle, M, K):
    import torch
    x, (xq, xd, xs) = acts(100 + M, M, K)
    x[0, :32] = 0.0                       # an all-zero group
    if K > 64:
        x[0, 32:64] = 0.0
        x[0, 40] = 1e-30                  # a lone tiny value
    if K > 96:
        # 0 < amax < 127 * 2^-128: d denormal, id = inf; zeros -> 0 (NaN under
        # cvt.rni), every other value -> +-127
        x[-1, 64:96] = 1e-38
        x[-1, [66, 70, 95]] = 0.0
        x[-1, 80] = -3e-39
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs, gh = bq.quantize_q8(dev(x), with_xdh=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(gq), xq)
    assert np.array_equal(host(gd).view(np.uint32), xd.view(np.uint32))
    assert np.array_equal(host(gs), xs)
    assert np.array_equal(host(gh).view(np.uint16), oracle.fill_xdh(xd, xs))
    gh2 = bq.fill_xdh(gd, gs)
    assert np.array_equal(host(gh2).view(np.uint16), oracle.fill_xdh(xd, xs))


# ---------------------------------------------------------------- repacks
@pytest.mark.parametrize("N,K", [(128, 512), (300, 3072)])
def test_repack_bitexact(bq, oracle, N, K):
    import torch
    raw5 = weights(200 + N, N, K, "q5k")
    raw6 = weights(300 + N, N, K, "q6k")
    w144, dm = bq.repack_q5k(dev(raw5), K, N)
    w160 = bq.repack_q6k(dev(raw6), K, N)
    torch.cuda.synchronize()
    r144, rdm = oracle.repack_q5k_144(raw5, K)
    r160 = oracle.repack_q6k_160(raw6, K)
    assert np.array_equal(host(w144), r144)
    assert np.array_equal(host(dm).view(np.uint16), rdm)
    assert np.array_equal(host(w160), r160)


# ---------------------------------------------------------------- integer dots (KAT)
def test_q5k_int_dots_bitexact(bq, oracle):
    """d = 1, dmin = 0 and a single nonzero 6-bit scale (=1) in group n % (K/32):
    with xd = 1 the kernel output is exactly that group's integer dot."""
    import torch
    K, N = 1024, 256
    raw = weights(401, N, K, "q5k").reshape(N, K // 256, 176).copy()
    raw[:, :, 0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    raw[:, :, 2:4] = 0
    raw[:, :, 4:16] = 0
    for n in range(N):
        g = n % (K // 32)
        sb, j = g // 8, g % 8
        if j < 4:
            raw[n, sb, 4 + j] = 1
        else:
            raw[n, sb, 8 + j] = 1  # low nibble of scales[j + 4]
    raw = raw.reshape(N, -1)
    _, (xq, xd, xs) = acts(402, 1, K)
    xd = np.ones_like(xd)
    y = torch.empty(N, device="cuda")
    w = bq.make_weight(dev(raw), bq.TYPE_Q5_K, K, N)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    bq.gemv(y, w, gq, gd, gs)
    torch.cuda.synchronize()
    dots = oracle.dots_q5k(raw, xq)[0]
    want = np.array([dots[n, n % (K // 32)] for n in range(N)], np.float32)
    assert np.array_equal(host(y), want)


def test_q6k_int_dots_bitexact(bq, oracle):
    import torch
    K, N = 1024, 256
    raw = weights(403, N, K, "q6k").reshape(N, K // 256, 210).copy()
    raw[:, :, 208:210] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    raw[:, :, 192:208] = 0
    for n in range(N):
        g16 = n % (K // 16)
        raw[n, g16 // 16, 192 + g16 % 16] = 1
    raw = raw.reshape(N, -1)
    _, (xq, xd, xs) = acts(404, 1, K)
    xd = np.ones_like(xd)
    dots = oracle.dots16_q6k(raw, xq)[0]
    want = np.array([dots[n, n % (K // 16)] for n in range(N)], np.float32)
    gq, gd = dev(xq), dev(xd)
    y = torch.empty(N, device="cuda")
    bq.gemm_q6k_raw(y, bq.make_weight(dev(raw), bq.TYPE_Q6_K, K, N), 1, gq, gd)
    torch.cuda.synchronize()
    assert np.array_equal(host(y), want)
    rep = bq.repack_q6k(dev(raw), K, N)
    y2 = torch.empty(N, device="cuda")
    bq.gemm_q6k_dp(y2, bq.make_weight(None, bq.TYPE_Q6_K, K, N, rep=rep), 1, gq, gd)
    torch.cuda.synchronize()
    assert np.array_equal(host(y2), want)


# ---------------------------------------------------------------- GEMV Q5_K
@pytest.mark.parametrize("N,K", [(256, 1024), (3072, 3072), (400, 4096), (64, 2560)])
def test_gemv_q5k(bq, oracle, N, K):
    import torch
    raw = weights(500 + N, N, K, "q5k")
    _, (xq, xd, xs) = acts(501, 1, K)
    ref = oracle.gemm_q5k(raw, xq, xd, xs)
    y = torch.full((N,), float("nan"), device="cuda")
    bq.gemv(y, bq.make_weight(dev(raw), bq.TYPE_Q5_K, K, N), *_xq_dev(xq, xd, xs))
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), ref) < TOL


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
def test_verify_fused_parts(bq, oracle, rows):
    """Config-2/5 style fused parts (gate+up, q/k/gate/v) and 2..8 verify rows."""
    import torch
    K = 3072
    Ns = [512, 128, 1024, 256]
    raws = [weights(600 + i, n, K, "q5k") for i, n in enumerate(Ns)]
    _, (xq, xd, xs) = acts(610 + rows, rows + 1, K)
    ws = [bq.make_weight(dev(r), bq.TYPE_Q5_K, K, n) for r, n in zip(raws, Ns)]
    ys = [torch.full((rows, n), float("nan"), device="cuda") for n in Ns]
    gq, gd, gs = _xq_dev(xq, xd, xs)
    assert bq.verify_fused(ys, ws, rows, gq, gd, gs, xoff=1) == bq.BQ_OK
    torch.cuda.synchronize()
    for r, y in zip(raws, ys):
        ref = oracle.gemm_q5k(r, xq[1:], xd[1:], xs[1:])
        assert oracle.normwise_err(host(y), ref) < TOL


def test_verify_config3_full(bq, oracle):
    """Config 3: Q5_K 9216x3072, rows 1/2/4/8 sharing one weight stream."""
    import torch
    K, N = 3072, 9216
    raw = weights(700, N, K, "q5k")
    _, (xq, xd, xs) = acts(701, 8, K)
    ref = oracle.gemm_q5k(raw, xq, xd, xs)
    w = bq.make_weight(dev(raw), bq.TYPE_Q5_K, K, N)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    for rows in (1, 2, 4, 8):
        y = torch.full((rows, N), float("nan"), device="cuda")
        assert bq.verify_fused([y], [w], rows, gq, gd, gs) == bq.BQ_OK
        torch.cuda.synchronize()
        assert oracle.normwise_err(host(y), ref[:rows]) < TOL, rows


def test_verify_unsupported(bq):
    import torch
    K = 512
    raw = torch.zeros((24, K // 256 * 176), dtype=torch.uint8, device="cuda")
    w = bq.make_weight(raw, bq.TYPE_Q5_K, K, 24)     # N % 16 != 0
    y = torch.zeros((1, 24), device="cuda")
    xq = torch.zeros((9, K), dtype=torch.int8, device="cuda")
    xd = torch.zeros((9, K // 32), device="cuda")
    xs = torch.zeros((9, K // 32), dtype=torch.int32, device="cuda")
    assert bq.verify_fused([y], [w], 1, xq, xd, xs) == bq.BQ_UNSUPPORTED
    w2 = bq.make_weight(raw[:16], bq.TYPE_Q5_K, K, 16)
    assert bq.verify_fused([y], [w2], 9, xq, xd, xs) == bq.BQ_UNSUPPORTED   # rows > 8
    w6 = bq.make_weight(raw[:16], bq.TYPE_Q6_K, K, 16)
    assert bq.verify_fused([y], [w6], 1, xq, xd, xs) == bq.BQ_UNSUPPORTED   # not Q5_K


# ---------------------------------------------------------------- Q6_K GEMV
@pytest.mark.parametrize("N,K,rows", [(3072, 9216, 1), (256, 3072, 3), (512, 1024, 8), (130, 768, 2)])
def test_q6k_gemv(bq, oracle, N, K, rows):
    import torch
    raw = weights(800 + N, N, K, "q6k")
    _, (xq, xd, xs) = acts(801, rows, K)
    ref = oracle.gemm_q6k(raw, xq, xd)
    graw = dev(raw)
    gq, gd = dev(xq), dev(xd)
    y = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_q6k_raw(y, bq.make_weight(graw, bq.TYPE_Q6_K, K, N), rows, gq, gd)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), ref) < TOL
    rep = bq.repack_q6k(graw, K, N)
    y2 = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_q6k_dp(y2, bq.make_weight(graw, bq.TYPE_Q6_K, K, N, rep=rep), rows, gq, gd)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y2), ref) < TOL
    if rows == 1:
        y3 = torch.full((N,), float("nan"), device="cuda")
        bq.gemv(y3, bq.make_weight(graw, bq.TYPE_Q6_K, K, N, rep=rep), gq, gd, None)
        torch.cuda.synchronize()
        assert oracle.normwise_err(host(y3), ref) < TOL


@pytest.mark.parametrize("fmt", ["q5k", "q5k_k4096", "q5k_n6912", "q6k_raw", "q6k_rep"])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 6, 7, 8])
def test_multirow_every_row_count(bq, oracle, fmt, rows):
    """Every multi-row instance (dot4 below, matrix-core dot products from 6
    rows for Q5_K and from 3 for Q6_K, partial last set of four rows
    included) against the oracle.  The Q5_K shapes reach the compile-time-K
    instances with one (small N), two (rows 5, N*K >= 20M) and three steps per
    wave, at K = 3072 and 4096."""
    import torch
    print(f"multirow {fmt} rows={rows}", flush=True)
    K, N = {"q5k": (3072, 528), "q5k_k4096": (4096, 528), "q5k_n6912": (3072, 6912)}.get(fmt, (9216, 132))
    q5 = fmt.startswith("q5k")
    raw = weights(1000 + rows, N, K, "q5k" if q5 else "q6k")
    _, (xq, xd, xs) = acts(1010 + rows, rows, K)
    g = dev(raw)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    y = torch.full((rows, N), float("nan"), device="cuda")
    if q5:
        assert bq.verify_fused([y], [bq.make_weight(g, bq.TYPE_Q5_K, K, N)], rows, gq, gd, gs) == bq.BQ_OK
        ref = oracle.gemm_q5k(raw, xq, xd, xs)
    elif fmt == "q6k_raw":
        bq.gemm_q6k_raw(y, bq.make_weight(g, bq.TYPE_Q6_K, K, N), rows, gq, gd)
        ref = oracle.gemm_q6k(raw, xq, xd)
    else:
        w = bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g, K, N))
        bq.gemm_q6k_dp(y, w, rows, gq, gd)
        ref = oracle.gemm_q6k(raw, xq, xd)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), ref) < TOL


def test_q6_verify_fused(bq, oracle):
    import torch
    K = 1024
    Ns = [256, 128]
    raws = [weights(900 + i, n, K, "q6k") for i, n in enumerate(Ns)]
    _, (xq, xd, xs) = acts(902, 6, K)
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        ws.append(bq.make_weight(g, bq.TYPE_Q6_K, K, n, rep=bq.repack_q6k(g, K, n)))
    ys = [torch.full((6, n), float("nan"), device="cuda") for n in Ns]
    assert bq.q6_verify_fused(ys, ws, 6, dev(xq), dev(xd)) == bq.BQ_OK
    torch.cuda.synchronize()
    for r, y in zip(raws, ys):
        assert oracle.normwise_err(host(y), oracle.gemm_q6k(r, xq, xd)) < TOL


# ---------------------------------------------------------------- fused quantize + GEMV
@pytest.mark.parametrize("qtype,K,Ns,rep", [
    ("q5k", 3072, [512, 1024], False),     # config-2 gate+up shape class
    ("q5k", 256, [48], False),
    ("q5k", 12288, [64, 32, 16, 80], False),  # 4 parts
    ("q5k", 49152, [32], False),           # largest fused K (16 waves, 3 chunks each)
    ("q6k", 9216, [3072], False),          # config-2 down projection
    ("q6k", 1024, [130], True),
    ("q5k", 2560, [40, 24], False),        # partial last chunk / block group
    ("q5k", 5120, [40], False),            # 5 K slices
    ("q6k", 20480, [64], False),           # 16-wave workgroups, 2 chunks per wave
    ("q6k", 12288, [48], True),
])
def test_gemv_q8_fused(bq, oracle, qtype, K, Ns, rep):
    """One launch quantizes x and runs the GEMV: q8 outputs bit-exact with the
    oracle quantizer, y within TOL of the oracle and within 1e-6 of the
    unfused pair (the same per-group arithmetic once the codes are in LDS; the
    two paths may split K differently, which reorders the slice sums)."""
    import torch
    x, _ = acts(1000 + K, 1, K)
    x[0, :32] = 0.0                                  # an all-zero group
    xq, xd, xs = oracle.q8_rows(x)
    raws = [weights(1010 + i, n, K, qtype) for i, n in enumerate(Ns)]
    tp = bq.TYPE_Q5_K if qtype == "q5k" else bq.TYPE_Q6_K
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        ws.append(bq.make_weight(g, tp, K, n, rep=bq.repack_q6k(g, K, n) if rep else None))
    ys = [torch.full((n,), float("nan"), device="cuda") for n in Ns]
    gx = dev(x)
    gq = torch.full((1, K), 99, dtype=torch.int8, device="cuda")
    gd = torch.full((1, K // 32), float("nan"), device="cuda")
    gs = torch.full((1, K // 32), -7, dtype=torch.int32, device="cuda")
    assert bq.gemv_q8_fused(ys, ws, gx, gq, gd, gs) == bq.BQ_OK
    torch.cuda.synchronize()
    assert np.array_equal(host(gq), xq)
    assert np.array_equal(host(gd).view(np.uint32), xd.view(np.uint32))
    assert np.array_equal(host(gs), xs)
    for r, y, w in zip(raws, ys, ws):
        ref = oracle.gemm_q5k(r, xq, xd, xs) if qtype == "q5k" else oracle.gemm_q6k(r, xq, xd)
        assert oracle.normwise_err(host(y)[None], ref) < TOL
        # the two-launch pair: the same per-group arithmetic; the K split (and
        # so the order in which slice sums are added) may differ per path
        y2 = torch.full_like(y, float("nan"))
        bq.gemv(y2, w, gq, gd, gs)
        torch.cuda.synchronize()
        assert oracle.normwise_err(host(y2)[None], host(y).astype(np.float64)[None]) < 1e-6
    ys3 = [torch.full((n,), float("nan"), device="cuda") for n in Ns]   # without q8 outputs
    assert bq.gemv_q8_fused(ys3, ws, gx) == bq.BQ_OK
    torch.cuda.synchronize()
    for y, y3 in zip(ys, ys3):
        assert np.array_equal(host(y3).view(np.uint32), host(y).view(np.uint32))


def test_config5_shapes(bq, oracle):
    """BASELINE config 5 layer shapes through the fused entry: QKV Q5_K 5120x3072,
    O Q5_K 3072x4096 (two K slices), and the Q6_K lm_head 131072x3072 built, as
    in the benchmark, from 16 copies of one 8192-row block: rows with identical
    bytes must give bit-identical outputs wherever they sit, and the first and
    last 1024 rows must match the oracle."""
    import torch
    for qt, N, K in (("q5k", 5120, 3072), ("q5k", 3072, 4096)):
        raw = weights(1100 + K, N, K, qt)
        x, _ = acts(1101 + K, 1, K)
        xq, xd, xs = oracle.q8_rows(x)
        y = torch.full((N,), float("nan"), device="cuda")
        assert bq.gemv_q8_fused([y], [bq.make_weight(dev(raw), bq.TYPE_Q5_K, K, N)], dev(x)) == bq.BQ_OK
        torch.cuda.synchronize()
        assert oracle.normwise_err(host(y)[None], oracle.gemm_q5k(raw, xq, xd, xs)) < TOL, (N, K)
    K, blk = 3072, 8192
    raw = weights(1200, blk, K, "q6k")
    lm = dev(raw).repeat(16, 1).contiguous()
    x, _ = acts(1201, 1, K)
    xq, xd, xs = oracle.q8_rows(x)
    y = torch.full((16 * blk,), float("nan"), device="cuda")
    assert bq.gemv_q8_fused([y], [bq.make_weight(lm, bq.TYPE_Q6_K, K, 16 * blk)], dev(x)) == bq.BQ_OK
    torch.cuda.synchronize()
    yh = host(y).reshape(16, blk)
    assert all(np.array_equal(yh[0].view(np.uint32), yh[i].view(np.uint32)) for i in range(1, 16))
    for rows in (slice(0, 1024), slice(blk - 1024, blk)):
        ref = oracle.gemm_q6k(np.ascontiguousarray(raw[rows]), xq, xd)
        assert oracle.normwise_err(yh[15][rows][None], ref) < TOL


def test_gemv_q8_fused_rejects(bq):
    import torch
    K = 512
    raw5 = torch.zeros((16, K // 256 * 176), dtype=torch.uint8, device="cuda")
    raw6 = torch.zeros((16, K // 256 * 210), dtype=torch.uint8, device="cuda")
    w5 = bq.make_weight(raw5, bq.TYPE_Q5_K, K, 16)
    w6 = bq.make_weight(raw6, bq.TYPE_Q6_K, K, 16)
    w5b = bq.make_weight(raw5, bq.TYPE_Q5_K, 256, 32)
    y = torch.zeros(16, device="cuda")
    x = torch.zeros(K, device="cuda")
    assert bq.gemv_q8_fused([y, y], [w5, w6], x) == bq.BQ_UNSUPPORTED   # mixed types
    assert bq.gemv_q8_fused([y, y], [w5, w5b], x) == bq.BQ_UNSUPPORTED  # mismatched K
    assert bq.gemv_q8_fused([y] * 5, [w5] * 5, x) == bq.BQ_UNSUPPORTED  # > 4 parts
    Kbig = 49408                                                       # above the GEMV K limit
    rawb = torch.zeros((16, Kbig // 256 * 176), dtype=torch.uint8, device="cuda")
    wb = bq.make_weight(rawb, bq.TYPE_Q5_K, Kbig, 16)
    xb = torch.zeros(Kbig, device="cuda")
    assert bq.gemv_q8_fused([y], [wb], xb) == bq.BQ_UNSUPPORTED
    assert bq.verify_fused([y.view(1, 16)], [wb], 1, xb.to(torch.int8).view(1, -1),
                           torch.zeros(1, Kbig // 32, device="cuda"),
                           torch.zeros(1, Kbig // 32, dtype=torch.int32, device="cuda")) == bq.BQ_UNSUPPORTED
    xq = torch.zeros(K, dtype=torch.int8, device="cuda")
    with pytest.raises(bq.BqError):                                    # xq without xd/xsum
        bq.gemv_q8_fused([y], [w5], x, xq)


# ---------------------------------------------------------------- prefill GEMM
def _mmq_case(bq, oracle, seed, M, Ns, K, prepacked):
    import torch
    raws = [weights(seed + i, n, K, "q5k") for i, n in enumerate(Ns)]
    _, (xq, xd, xs) = acts(seed + 50, M, K)
    ws, keep = [], []
    for r, n in zip(raws, Ns):
        g = dev(r)
        if prepacked:
            w144, dm = bq.repack_q5k(g, K, n)
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n, rep=w144, rep_min=dm))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
    ys = [torch.full((M, n), float("nan"), device="cuda") for n in Ns]
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    gq, gd, gs = _xq_dev(xq, xd, xs)
    assert bq.try_mmq(ys, ws, M, gq, gd, gs, xdh) == bq.BQ_OK
    torch.cuda.synchronize()
    for r, n, y in zip(raws, Ns, ys):
        if prepacked:
            w144, dm = oracle.repack_q5k_144(r, K)
            ref = oracle.gemm_q5k_144(w144, dm, xq, xd, oracle.fill_xdh(xd, xs), n)
        else:
            ref = oracle.gemm_q5k(r, xq, xd, xs)
        assert oracle.normwise_err(host(y), ref) < TOL


@pytest.mark.parametrize("prepacked", [False, True])
def test_mmq_q5k(bq, oracle, prepacked):
    _mmq_case(bq, oracle, 1000, 256, [256], 1024, prepacked)


@pytest.mark.parametrize("prepacked", [False, True])
def test_mmq_q5k_ragged_parts(bq, oracle, prepacked):
    # 200 rows (not a multiple of the 128 tile), three parts
    _mmq_case(bq, oracle, 1100, 200, [128, 256, 128], 1536, prepacked)


# Row counts that are not multiples of either token tile, multi-part launches
# with unequal N, and K-split classes: each case's tile height and split come
# from the launch's work estimate (both heights occur below).
@pytest.mark.parametrize("prepacked", [False, True])
@pytest.mark.parametrize("M,Ns,K", [(97, [256, 128], 1024), (129, [128, 384], 1536), (300, [256, 128, 128], 1024),
                                    (1000, [384], 512)])
def test_mmq_tile_heights(bq, oracle, prepacked, M, Ns, K):
    import torch
    print(f"mmq tiles M={M} Ns={Ns} K={K} prepacked={prepacked}", flush=True)
    raws = [weights(1200 + i + M, n, K, "q5k") for i, n in enumerate(Ns)]
    _, (xq, xd, xs) = acts(1250 + M, M, K)
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        if prepacked:
            w144, dm = bq.repack_q5k(g, K, n)
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n, rep=w144, rep_min=dm))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
    ys = [torch.full((M, n), float("nan"), device="cuda") for n in Ns]
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    gq, gd, gs = _xq_dev(xq, xd, xs)
    assert bq.try_mmq(ys, ws, M, gq, gd, gs, xdh) == bq.BQ_OK
    torch.cuda.synchronize()
    for r, n, y in zip(raws, Ns, ys):
        if prepacked:
            w144, dm = oracle.repack_q5k_144(r, K)
            ref = oracle.gemm_q5k_144(w144, dm, xq, xd, oracle.fill_xdh(xd, xs), n)
        else:
            ref = oracle.gemm_q5k(r, xq, xd, xs)
        check(oracle, host(y), ref, what=f"N={n}")


@pytest.mark.parametrize("M", [9, 33, 100, 257])
def test_q6k_mma_rows(bq, oracle, M):
    """The Q6_K GEMM over W160 at row counts off both token tiles (N 384,
    K 2048: the K split is taken at every one of them)."""
    import torch
    K, N = 2048, 384
    raw = weights(1300 + M, N, K, "q6k")
    _, (xq, xd, xs) = acts(1350 + M, M, K)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    g = dev(raw)
    y = torch.full((M, N), float("nan"), device="cuda")
    bq.gemm_q6k_mma(y, bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g, K, N)), M, gq, gd)
    torch.cuda.synchronize()
    check(oracle, host(y), oracle.gemm_q6k(raw, xq, xd), what=f"M={M}")


def test_mmq_unsupported(bq):
    import torch
    K = 512
    raw = torch.zeros((128, K // 256 * 176), dtype=torch.uint8, device="cuda")
    w = bq.make_weight(raw, bq.TYPE_Q5_K, K, 128)
    y = torch.zeros((64, 128), device="cuda")
    xq = torch.zeros((64, K), dtype=torch.int8, device="cuda")
    xd = torch.zeros((64, K // 32), device="cuda")
    xs = torch.zeros((64, K // 32), dtype=torch.int32, device="cuda")
    assert bq.try_mmq([y], [w], 64, xq, xd, xs) == bq.BQ_UNSUPPORTED  # rows < 96


@pytest.mark.parametrize("K,N,M", [(1024, 256, 160), (256, 128, 1), (256, 384, 300), (9216, 128, 140),
                                   (3072, 256, 257)])
def test_mmq_q6k(bq, oracle, K, N, M):
    """Q6_K GEMM over W160: the shortest K (one stage pair), a single token,
    token counts that leave a partial tile, the down projection's K = 9216."""
    import torch
    print(f"mmq q6k K={K} N={N} M={M}", flush=True)
    raw = weights(1200 + K // 128 + M, N, K, "q6k")
    _, (xq, xd, xs) = acts(1201 + M, M, K)
    g = dev(raw)
    w = bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g, K, N))
    y = torch.full((M, N), float("nan"), device="cuda")
    bq.gemm_q6k_mma(y, w, M, dev(xq), dev(xd))
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), oracle.gemm_q6k(raw, xq, xd)) < TOL


def test_mmq_config4_full_slices(bq, oracle):
    """Config 4 at full size (M = 2048, N = 9216, K = 3072, both tiers); the
    oracle checks a sample of 48 token rows x 192 weight rows of the output."""
    import torch
    K, N, M = 3072, 9216, 2048
    raw = weights(1300, N, K, "q5k")
    _, (xq, xd, xs) = acts(1301, M, K)
    g = dev(raw)
    w144, dm = bq.repack_q5k(g, K, N)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    rng = np.random.default_rng(7)
    mi = np.sort(rng.choice(M, 48, replace=False))
    ni = np.sort(rng.choice(N, 192, replace=False))
    for prepacked in (False, True):
        w = bq.make_weight(g, bq.TYPE_Q5_K, K, N, rep=w144 if prepacked else None,
                           rep_min=dm if prepacked else None)
        y = torch.full((M, N), float("nan"), device="cuda")
        assert bq.try_mmq([y], [w], M, gq, gd, gs, xdh) == bq.BQ_OK
        torch.cuda.synchronize()
        yh = host(y)
        assert np.isfinite(yh).all()
        sub = raw[ni]
        if prepacked:
            r144, rdm = oracle.repack_q5k_144(sub, K)
            ref = oracle.gemm_q5k_144(r144, rdm, xq[mi], xd[mi], oracle.fill_xdh(xd[mi], xs[mi]), len(ni))
        else:
            ref = oracle.gemm_q5k(sub, xq[mi], xd[mi], xs[mi])
        assert oracle.normwise_err(yh[np.ix_(mi, ni)], ref) < TOL, prepacked


@pytest.mark.parametrize("rows", [17, 100, 128])
def test_mmq_w144_ksplit(bq, oracle, rows):
    """The W144 GEMM over one token tile split into 8 K slices (3072 / 256 = 12
    stage pairs; 8 weight-row tiles): against the oracle, and bit-identical
    between two calls (the slices are summed in a fixed order)."""
    import torch
    K, N = 3072, 1024
    print(f"mmq w144 k-split rows={rows}", flush=True)
    raw = weights(1500 + rows, N, K, "q5k")
    _, (xq, xd, xs) = acts(1501 + rows, rows, K)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    g = dev(raw)
    w144, dm = bq.repack_q5k(g, K, N)
    w = bq.make_weight(g, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm)
    y1 = torch.full((rows, N), float("nan"), device="cuda")
    y2 = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_b(y1, w, rows, gq, gd, gs, xdh)
    bq.gemm_b(y2, w, rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    assert np.array_equal(host(y1).view(np.uint32), host(y2).view(np.uint32))
    r144, rdm = oracle.repack_q5k_144(raw, K)
    ref = oracle.gemm_q5k_144(r144, rdm, xq, xd, oracle.fill_xdh(xd, xs), N)
    assert oracle.normwise_err(host(y1), ref) < TOL


@pytest.mark.parametrize("rows", [9, 33, 96, 128, 129, 300])
def test_w144_min_term_xdh(bq, oracle, rows):
    """The W144 tier's fp16 min term alone (every super-block's d = 0, so
    y = sum_g f16(Dm[n][g]) * f16(xdh[m][g])), through bq_gemm_b: up to 64
    rows the 32-token tile forms xdh = half(xd * xsum) itself, above it
    k_fill_xdh fills it first (bruce.cu:6598-6602).  Against the product of
    the oracle's Dm and xdh in float64, at 2e-6 of the output's largest
    value: one xdh value rounded the other way (2^-11 of its term) fails it."""
    import torch
    K, N = 1024, 256
    raw = weights(1450 + rows, N, K, "q5k").copy()
    raw.reshape(N, K // 256, 176)[:, :, 0:2] = 0          # d = 0: no sc*q term
    _, (xq, xd, xs) = acts(1451 + rows, rows, K)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    g5 = dev(raw)
    w144, dm = bq.repack_q5k(g5, K, N)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    y = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_b(y, bq.make_weight(g5, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm), rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    _, rdm = oracle.repack_q5k_144(raw, K)
    hx = oracle.fill_xdh(xd, xs).view(np.float16).astype(np.float64).reshape(rows, K // 32)
    hd = np.asarray(rdm).view(np.float16).astype(np.float64).reshape(N, K // 32)
    ref = hx @ hd.T
    yh = host(y).astype(np.float64)
    assert np.isfinite(yh).all()
    assert np.abs(yh - ref).max() <= 2e-6 * np.abs(ref).max()


# ---------------------------------------------------------------- dispatcher
@pytest.mark.parametrize("rows", [3, 8, 9, 12, 16, 17, 20, 27, 28, 43, 60, 130, 1536, 1537])
def test_gemm_b_dispatch(bq, oracle, rows):
    """bq_gemm_b: 8-row GEMV chunks up to 8 rows, the MMQ tile above (the 32-
    or 128-token tile by the launch's work estimate; K-split while the tiles
    leave workgroup slots empty); bq_try_mmq keeps the reference's
    rows >= 96."""
    import torch
    K, N = 1024, 256
    raw5 = weights(1400, N, K, "q5k")
    raw6 = weights(1401, N, K, "q6k")
    _, (xq, xd, xs) = acts(1402, rows, K)
    gq, gd, gs = _xq_dev(xq, xd, xs)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    g5 = dev(raw5)
    y = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_b(y, bq.make_weight(g5, bq.TYPE_Q5_K, K, N), rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), oracle.gemm_q5k(raw5, xq, xd, xs)) < TOL
    # prepacked: the W144 tile (fp16 min term) above 8 rows
    w144, dm = bq.repack_q5k(g5, K, N)
    yp = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_b(yp, bq.make_weight(g5, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm), rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    if rows > 8:
        r144, rdm = oracle.repack_q5k_144(raw5, K)
        ref = oracle.gemm_q5k_144(r144, rdm, xq, xd, oracle.fill_xdh(xd, xs), N)
    else:
        ref = oracle.gemm_q5k(raw5, xq, xd, xs)
    assert oracle.normwise_err(host(yp), ref) < TOL
    if rows < 96:
        yt = torch.empty((rows, N), device="cuda")
        assert bq.try_mmq([yt], [bq.make_weight(g5, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm)], rows,
                          gq, gd, gs, xdh) == bq.BQ_UNSUPPORTED
    g6 = dev(raw6)
    y6 = torch.full((rows, N), float("nan"), device="cuda")
    bq.gemm_b(y6, bq.make_weight(g6, bq.TYPE_Q6_K, K, N, rep=bq.repack_q6k(g6, K, N)), rows, gq, gd, gs, xdh)
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y6), oracle.gemm_q6k(raw6, xq, xd)) < TOL
