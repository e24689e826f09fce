"""CPU checks that pin the Q8_0 logits-head restatement in the oracle
(orc_quantize_q8s: bruce.cu:4843-4867, orc_gemv_q8s: bruce.cu:4409-4449).

- The BF16 -> Q8S conversion is the activation quantizer's arithmetic applied
  to widened bf16 values. That quantizer is pinned separately by its closed-form
  checks. The codes must therefore equal orc_q8_rows bit for bit, and each scale
  must be numpy's float16 rounding of xd.
- A hand-built matrix pins the 272-byte block layout: where each scale and each
  code lives.
- The GEMV is checked against a float64 matmul of the dequantized operands. That
  matmul is built with numpy reshapes of the block layout, not the oracle's
  loops. It is also checked against the "y = K" known answer and exact scaling
  in rs.
"""
import numpy as np
import pytest

from helpers import acts


def split_q8s(oracle, w, K):
    """Q8S [N, K/256*272] -> (scales f32 [N, K/32], codes int8 [N, K]) via reshapes."""
    N = w.shape[0]
    b = w.reshape(N, K // 256, 272)
    sc = np.ascontiguousarray(b[:, :, :16]).view(np.float16).astype(np.float32).reshape(N, K // 32)
    codes = np.ascontiguousarray(b[:, :, 16:]).view(np.int8).reshape(N, K)
    return sc, codes


def test_bf16_helper_matches_torch(oracle):
    import torch
    x = oracle.gaussian(3, 4096, 0.0, 1.0) * np.float32(10.0) ** np.repeat(np.arange(-4, 4), 512).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(x), ref)
    assert np.array_equal(oracle.bf16_to_f32(ref), torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("N,K", [(3, 256), (17, 2560), (5, 3072)])
def test_q8s_equals_q8_rows(oracle, N, K):
    w = oracle.f32_to_bf16(oracle.gaussian(40 + K, N * K, 0.0, 0.02).reshape(N, K))
    w[0, :32] = 0                                       # all-zero group
    w[1 % N, 40] = oracle.f32_to_bf16(np.array([-3.0], np.float32))[0]  # one large value
    q = oracle.quantize_q8s(w)
    assert q.shape == (N, K // 256 * 272)
    sc, codes = split_q8s(oracle, q, K)
    xq, xd, _ = oracle.q8_rows(oracle.bf16_to_f32(w))
    assert np.array_equal(codes, xq)
    assert np.array_equal(sc.astype(np.float16).view(np.uint16), xd.astype(np.float16).view(np.uint16))
    # round trip: |v - s*q| <= d/2 + 127*|s - d| with the fp16-rounded scale s
    v = oracle.bf16_to_f32(w).astype(np.float64).reshape(N, K // 32, 32)
    deq = sc.astype(np.float64)[..., None] * codes.reshape(N, K // 32, 32)
    bound = xd[..., None] * 0.5 + 127 * np.abs(sc - xd)[..., None] + 1e-12
    assert np.all(np.abs(v - deq) <= bound * (1 + 1e-6))


def test_q8s_layout_kat(oracle):
    """Group g of super-block s in row r holds one value +-(1 + 8s + g) at lane
    (r + 3g + s) % 32: its code must be +-127 at byte 16 + 32g + lane of block s,
    the scale half_rn(amax * (1/127)) at bytes 2g..2g+1, every other code 0."""
    N, K = 3, 768
    w = np.zeros((N, K), np.float32)
    for r in range(N):
        for s in range(K // 256):
            for g in range(8):
                sign = -1.0 if (r + g) % 2 else 1.0
                w[r, 256 * s + 32 * g + (r + 3 * g + s) % 32] = sign * (1 + 8 * s + g)
    q = oracle.quantize_q8s(oracle.f32_to_bf16(w)).reshape(N, K // 256, 272)
    for r in range(N):
        for s in range(K // 256):
            blk = q[r, s]
            for g in range(8):
                a = np.float32(1 + 8 * s + g)
                d = a * np.float32(1.0 / 127.0)
                assert blk[2 * g:2 * g + 2].view(np.uint16)[0] == np.float16(d).view(np.uint16)
                lane = (r + 3 * g + s) % 32
                codes = blk[16 + 32 * g:16 + 32 * g + 32].view(np.int8)
                sign = -1 if (r + g) % 2 else 1
                assert codes[lane] == 127 * sign
                assert np.count_nonzero(codes) == 1


def make_q8s(oracle, seed, N, K):
    w = oracle.f32_to_bf16(oracle.gaussian(seed, N * K, 0.0, 0.02).reshape(N, K))
    return oracle.quantize_q8s(w)


@pytest.mark.parametrize("M,N,K", [(1, 33, 256), (3, 20, 2560), (8, 7, 3072)])
def test_gemv_q8s_vs_dequant_matmul(oracle, M, N, K):
    w = make_q8s(oracle, 7 + M, N, K)
    _, (xq, xd, _) = acts(70 + M, M, K)
    rs = oracle.gaussian(9, N, 1.0, 0.1)
    got = oracle.gemv_q8s(w, K, xq, xd, rs)
    sc, codes = split_q8s(oracle, w, K)
    wdeq = (sc.astype(np.float64)[..., None] * codes.reshape(N, K // 32, 32)).reshape(N, K)
    xdeq = (xd.astype(np.float64)[..., None] * xq.reshape(M, K // 32, 32)).reshape(M, K)
    ref = (xdeq @ wdeq.T) * rs.astype(np.float64)[None]
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    # no rs == rs of ones
    assert np.array_equal(oracle.gemv_q8s(w, K, xq, xd), oracle.gemv_q8s(w, K, xq, xd, np.ones(N, np.float32)))


def test_gemv_q8s_kat_y_equals_K(oracle):
    """All scales 1.0, all codes 1, xq = 1, xd = 1: every output is K (then * rs)."""
    N, K = 5, 1024
    blk = np.zeros(272, np.uint8)
    blk[:16] = np.full(8, 1.0, np.float16).view(np.uint8)
    blk[16:] = 1
    w = np.tile(blk, (N, K // 256))
    xq = np.ones((2, K), np.int8)
    xd = np.ones((2, K // 32), np.float32)
    assert np.all(oracle.gemv_q8s(w, K, xq, xd) == K)
    rs = np.arange(1, N + 1, dtype=np.float32)
    assert np.array_equal(oracle.gemv_q8s(w, K, xq, xd, rs), np.tile(K * rs.astype(np.float64), (2, 1)))


def test_q8s_tiny_groups(oracle):
    """amax = 1e-38 (an fp32 denormal): d = amax/127 underflows the half scale
    to 0 and 1/d overflows to inf, so every nonzero code saturates to +-127 and
    zeros stay 0 (0 * inf = NaN -> 0) -- what the reference's device conversion
    (__float2int_rn, PTX cvt.rni) produces.  amax = 1e-30:
    finite id, ordinary codes, half scale 0."""
    K = 256
    w = np.zeros((1, K), np.float32)
    w[0, :32] = 1e-38
    w[0, 5] = -1e-38
    w[0, 11] = 0.0                               # 0 * inf = NaN -> 0 (cvt.rni)
    w[0, 32:64] = np.linspace(-1e-30, 1e-30, 32)
    b = oracle.f32_to_bf16(w)
    sc, codes = split_q8s(oracle, oracle.quantize_q8s(b), K)
    assert sc[0, 0] == 0 and sc[0, 1] == 0
    i = np.arange(32)
    assert np.all(codes[0, :32] == np.where(i == 5, -127, np.where(i == 11, 0, 127)))
    assert codes[0, 32] == -127 and codes[0, 63] == 127
    xq, _, _ = oracle.q8_rows(oracle.bf16_to_f32(b)[:, 32:64])
    assert np.array_equal(codes[0, 32:64], xq[0])
