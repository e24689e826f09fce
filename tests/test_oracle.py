"""CPU checks that pin the oracle (oracle/bq_oracle.c) independently of itself.

Each check is chosen so that a plausible mistake (wrong bit of the 6-bit scale
layout, swapped nibble, dropped min term, wrong rounding) fails it: IEEE fp16
against numpy, hand-built known-answer blocks from the published GGUF layout,
the mmq_test.cu "y = K" KAT (tools/mmq_test.cu:311-334), brute-force integer
dots, linearity, and the repack index maps rebuilt with numpy.
"""
import numpy as np
import pytest

from helpers import acts, kat_q5k as kat_weights, kat_q6k, np_codes_q5k, np_codes_q6k, weights


# ---------------------------------------------------------------- fp16
def test_h2f_exhaustive(oracle):
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_h2f(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_f2h_rn_matches_numpy(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 4000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                  5.960464477539063e-08, 6.103515625e-05, -6.1e-05], np.float32),
        # exact ties between two halves (normal and denormal ranges)
        (np.arange(1, 200, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        (np.float32(1.0) + np.arange(0, 64, dtype=np.float32) * np.float32(2.0 ** -11)),
    ])
    got = np.array([L.orc_f2h_rn(float(v)) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- quantizer
def test_q8_invariants(oracle):
    x, (xq, xd, xs) = acts(11, 3, 1024)
    g = xq.reshape(3, 32, 32).astype(np.int32)
    assert np.all(np.abs(g) <= 127)
    assert np.array_equal(xs, g.sum(-1))
    # the largest-magnitude value of every group lands on +-127
    assert np.all(np.abs(g).max(-1) == 127)
    # round to nearest: |v - q*d| <= d/2 (+ float slack)
    err = np.abs(x.reshape(3, 32, 32) - g * xd[..., None].astype(np.float64))
    assert np.all(err <= xd[..., None] * (0.5 + 1e-5))
    # numpy float32 restatement (amax * (1/127), IEEE 1/d, round-half-even)
    amax = np.abs(x.reshape(3, 32, 32)).max(-1).astype(np.float32)
    d = amax * np.float32(1.0 / 127.0)
    assert np.array_equal(d.view(np.uint32), xd.view(np.uint32))
    idv = np.float32(1.0) / d
    q = np.clip(np.rint(x.reshape(3, 32, 32).astype(np.float32) * idv[..., None]), -127, 127)
    assert np.array_equal(q.astype(np.int32), g)


def test_q8_special_cases(oracle):
    x = np.zeros((1, 128), np.float32)
    x[0, 32 + 7] = -3.25       # single negative value
    x[0, 64:96] = 2.0          # constant group
    x[0, 96] = 1e-30           # tiny positive value alone
    xq, xd, xs = oracle.q8_rows(x)
    assert xd[0, 0] == 0 and np.all(xq[0, :32] == 0) and xs[0, 0] == 0
    assert xq[0, 39] == -127 and xs[0, 1] == -127 and np.count_nonzero(xq[0, 32:64]) == 1
    assert np.all(xq[0, 64:96] == 127) and xs[0, 2] == 127 * 32
    assert xq[0, 96] == 127 and xd[0, 3] > 0
    # 0 < amax < 127 * 2^-128: d is denormal, id = 1/d = inf.  The
    # reference's __float2int_rn (PTX cvt.rni: NaN -> 0, +-inf saturates)
    # gives 0 for v = 0 (0 * inf = NaN) and +-127 for every other value.
    x = np.zeros((1, 64), np.float32)
    x[0, :32] = 1e-38
    x[0, [3, 9, 31]] = 0.0
    x[0, 5] = -1e-38
    x[0, 7] = -0.0
    x[0, 40] = 2e-39                         # alone: d denormal as well
    xq, xd, xs = oracle.q8_rows(x)
    assert 0 < xd[0, 0] < np.float32(2.0 ** -126) and np.isinf(np.float32(1) / xd[0, 0])
    want = np.where(x[0, :32] > 0, 127, np.where(x[0, :32] < 0, -127, 0))
    assert np.array_equal(xq[0, :32], want) and xs[0, 0] == want.sum()
    assert xq[0, 40] == 127 and np.count_nonzero(xq[0, 32:]) == 1 and xs[0, 1] == 127
    # ties round half to even: amax = 127 -> d = 1 exactly, v = k + 0.5
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]
    xq, xd, _ = oracle.q8_rows(x)
    assert xd[0, 0] == np.float32(127.0) * np.float32(1 / 127)
    if xd[0, 0] == 1.0:
        assert list(xq[0, 1:6]) == [0, 2, 2, 0, -2]


# ---------------------------------------------------------------- format decode KATs
SCALES = np.array([0xC1, 0x42, 0x03, 0x84, 0x45, 0x86, 0xC7, 0x08, 0x9A, 0xBC, 0xDE, 0xF0], np.uint8)
# hand-decoded from the GGUF Q5_K/Q4_K 12-byte scale layout
SC_EXPECT = [1, 2, 3, 4, 58, 28, 14, 32]
M_EXPECT = [5, 6, 7, 8, 25, 43, 61, 15]


def test_q5k_scale_kat(oracle):
    for j in range(8):
        assert oracle.q5k_scale(SCALES, j) == (SC_EXPECT[j], M_EXPECT[j]), j


def test_q5k_code_kat(oracle):
    blk = np.zeros(176, np.uint8)
    blk[48 + 32 * 1 + 5] = 0xA3   # sub-block pair 1 (j = 2, 3), position 5
    blk[16 + 5] = 0b00001000      # high bit for j = 3 at position 5
    L = oracle.lib()
    codes = np.array([L.orc_q5k_code(blk.ctypes.data, k) for k in range(256)])
    want = np.zeros(256, int)
    want[32 * 2 + 5] = 3
    want[32 * 3 + 5] = 10 + 16
    assert np.array_equal(codes, want)


def test_q6k_code_kat(oracle):
    blk = np.zeros(210, np.uint8)
    blk[64 * 1 + 32 * 1 + 7] = 0x5C   # half 1, quarters 1 (low) and 3 (high), l = 7
    blk[128 + 32 * 1 + 7] = 0b11000100
    blk[192:208] = np.arange(16, dtype=np.int8).view(np.uint8) - 8
    L = oracle.lib()
    codes = np.array([L.orc_q6k_code(blk.ctypes.data, k) for k in range(256)])
    want = np.zeros(256, int)
    want[128 + 32 + 7] = 0xC + (1 << 4)
    want[128 + 96 + 7] = 5 + (3 << 4)
    assert np.array_equal(codes, want)
    scs = [L.orc_q6k_sc(blk.ctypes.data, k) for k in range(256)]
    assert scs == [k // 16 - 8 for k in range(256)]


# ---------------------------------------------------------------- encoders
@pytest.mark.parametrize("qtype,tol", [("q5k", 0.06), ("q6k", 0.03)])
def test_encoder_roundtrip(oracle, qtype, tol):
    w = oracle.gaussian(3, 32 * 1024, 0, 0.02).reshape(32, 1024)
    raw = oracle.quantize_q5k(w) if qtype == "q5k" else oracle.quantize_q6k(w)
    deq = oracle.dequant_q5k(raw, 1024) if qtype == "q5k" else oracle.dequant_q6k(raw, 1024)
    rel = np.sqrt(((deq - w) ** 2).mean()) / w.std()
    assert rel < tol
    # deterministic
    raw2 = oracle.quantize_q5k(w) if qtype == "q5k" else oracle.quantize_q6k(w)
    assert np.array_equal(raw, raw2)


def test_dots_vs_numpy(oracle):
    raw5 = weights(21, 24, 512, "q5k")
    raw6 = weights(22, 24, 512, "q6k")
    _, (xq, xd, xs) = acts(23, 2, 512)
    c5 = np_codes_q5k(raw5, 512)
    c6 = np_codes_q6k(raw6, 512) - 32
    x = xq.astype(np.int64)
    d5 = np.einsum("ngl,mgl->mng", c5.reshape(24, 16, 32), x.reshape(2, 16, 32))
    d6 = np.einsum("ngl,mgl->mng", c6.reshape(24, 32, 16), x.reshape(2, 32, 16))
    assert np.array_equal(oracle.dots_q5k(raw5, xq), d5)
    assert np.array_equal(oracle.dots16_q6k(raw6, xq), d6)


def test_gemm_vs_dequant_matmul(oracle):
    raw5 = weights(31, 40, 768, "q5k")
    raw6 = weights(32, 40, 768, "q6k")
    _, (xq, xd, xs) = acts(33, 3, 768)
    xr = (xq.reshape(3, 24, 32) * xd[..., None].astype(np.float64)).reshape(3, 768)
    # the dequantized weight times the dequantized activation is the same sum
    # (xsum carries the min term): sum_k (ds*u - dm) * xd*q
    y5 = xr @ oracle.dequant_q5k(raw5, 768).astype(np.float64).T
    y6 = xr @ oracle.dequant_q6k(raw6, 768).astype(np.float64).T
    assert oracle.normwise_err(oracle.gemm_q5k(raw5, xq, xd, xs), y5) < 1e-6
    assert oracle.normwise_err(oracle.gemm_q6k(raw6, xq, xd), y6) < 1e-6
    # the reference's serial fp32 order stays within 1e-5 of the double result
    assert oracle.normwise_err(oracle.gemm_q5k_f32(raw5, xq, xd, xs), oracle.gemm_q5k(raw5, xq, xd, xs)) < 1e-5
    assert oracle.normwise_err(oracle.gemm_q6k_f32(raw6, xq, xd), oracle.gemm_q6k(raw6, xq, xd)) < 1e-5


def test_kat_y_equals_K(oracle):
    K, N, M = 1024, 8, 2
    raw = kat_weights(N, K)
    xq = np.ones((M, K), np.int8)
    xd = np.ones((M, K // 32), np.float32)
    xs = np.zeros((M, K // 32), np.int32)
    assert np.all(oracle.gemm_q5k(raw, xq, xd, xs) == K)
    assert np.all(oracle.gemm_q5k_f32(raw, xq, xd, xs) == K)


def test_kat_q6k_y_equals_K(oracle):
    K, N, M = 512, 4, 2
    raw = kat_q6k(N, K)
    assert np.all(np_codes_q6k(raw, K) == 33)
    xq = np.ones((M, K), np.int8)
    xd = np.ones((M, K // 32), np.float32)
    assert np.all(oracle.gemm_q6k(raw, xq, xd) == K)
    assert np.all(oracle.gemm_q6k_f32(raw, xq, xd) == K)
    assert np.all(np_codes_q5k(kat_weights(N, K), K) == 1)


def test_linearity_and_min_term(oracle):
    raw = weights(41, 16, 512, "q5k")
    _, (xq, xd, xs) = acts(42, 2, 512)
    y = oracle.gemm_q5k(raw, xq, xd, xs)
    assert np.array_equal(oracle.gemm_q5k(raw, xq, xd * np.float32(2), xs), 2 * y)
    # dmin = 0 removes exactly the min term: y0 = sum xd*ds*dot
    raw0 = raw.reshape(16, 2, 176).copy()
    raw0[:, :, 2:4] = 0
    raw0 = raw0.reshape(16, -1)
    dots = oracle.dots_q5k(raw0, xq).astype(np.float64)
    ds = np.zeros((16, 16))
    L = oracle.lib()
    for n in range(16):
        for g in range(16):
            b = raw0.reshape(16, 2, 176)[n, g // 8]
            sc, _ = oracle.q5k_scale(b[4:16], g % 8)
            ds[n, g] = float(np.float32(L.orc_h2f(int(b[0]) | int(b[1]) << 8)) * np.float32(sc))
    want = np.einsum("mng,ng,mg->mn", dots, ds, xd.astype(np.float64))
    assert np.allclose(oracle.gemm_q5k(raw0, xq, xd, xs), want, rtol=1e-12, atol=0)


# ---------------------------------------------------------------- repacks
def test_repack_q5k_144_map(oracle):
    K, N = 512, 8
    raw = weights(51, N, K, "q5k")
    w144, dm = oracle.repack_q5k_144(raw, K)
    codes = np_codes_q5k(raw, K)
    assert np.array_equal(w144[:, :, :128].transpose(1, 0, 2).reshape(N, K), codes)
    # ds / dm from the hand-checked scale decoder
    L = oracle.lib()
    b = raw.reshape(N, K // 256, 176)
    for n in range(N):
        for sb in range(K // 256):
            d = np.float32(L.orc_h2f(int(b[n, sb, 0]) | int(b[n, sb, 1]) << 8))
            dmin = np.float32(L.orc_h2f(int(b[n, sb, 2]) | int(b[n, sb, 3]) << 8))
            for j in range(8):
                sc, m = oracle.q5k_scale(b[n, sb, 4:16], j)
                st = w144[sb * 2 + j // 4, n]
                assert st[128 + 4 * (j % 4):132 + 4 * (j % 4)].view(np.float32)[0] == d * np.float32(sc)
                assert dm[n, sb * 8 + j] == np.float16(-(dmin * np.float32(m))).view(np.uint16)


def test_repack_q6k_160_map(oracle):
    K, N = 512, 8
    raw = weights(52, N, K, "q6k")
    rep = oracle.repack_q6k_160(raw, K)
    codes = np_codes_q6k(raw, K) - 32
    assert np.array_equal(rep[:, :, :128].view(np.int8).reshape(N, K), codes)
    b = raw.reshape(N, K // 256, 210)
    d = b[:, :, 208:210].copy().view(np.float16).astype(np.float32)[..., 0]
    sc = b[:, :, 192:208].view(np.int8).astype(np.float32)
    want = (d[:, :, None] * sc).reshape(N, K // 128, 8)
    assert np.array_equal(rep[:, :, 128:].copy().view(np.float32), want)


def test_gemm_144_vs_exact(oracle):
    K, N = 1024, 16
    raw = weights(61, N, K, "q5k")
    _, (xq, xd, xs) = acts(62, 3, K)
    w144, dm = oracle.repack_q5k_144(raw, K)
    xdh = oracle.fill_xdh(xd, xs)
    y = oracle.gemm_q5k(raw, xq, xd, xs)
    y144 = oracle.gemm_q5k_144(w144, dm, xq, xd, xdh, N)
    # the two differ only by the fp16 rounding of Dm and xdh: bound it term by term
    L = oracle.lib()
    dmf = np.vectorize(lambda h: L.orc_h2f(int(h)))(dm).astype(np.float64)
    xdhf = np.vectorize(lambda h: L.orc_h2f(int(h)))(xdh).astype(np.float64)
    exact_min = -np.zeros((3, N))
    b = raw.reshape(N, K // 256, 176)
    dm_exact = np.zeros((N, K // 32))
    for n in range(N):
        for g in range(K // 32):
            blk = b[n, g // 8]
            _, m = oracle.q5k_scale(blk[4:16], g % 8)
            dm_exact[n, g] = -float(np.float32(L.orc_h2f(int(blk[2]) | int(blk[3]) << 8)) * np.float32(m))
    exact_min = (xd.astype(np.float64) * xs) @ dm_exact.T
    approx_min = xdhf @ dmf.T
    assert np.allclose(y144 - approx_min, y - exact_min, rtol=1e-12, atol=1e-9)
