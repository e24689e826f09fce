"""Synthetic k-quant weights and activations for benchmarks (numpy, vectorised).

The reference engine only reads llama.cpp-encoded GGUF files; it has no
encoder.  Benchmarks need Gaussian weights encoded to GGUF Q5_K / Q6_K, so this
module provides a deterministic encoder.  Blocks follow the GGUF layouts:

  Q5_K  176 B / 256 values: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
        value k = 32j + l: u = nibble (j & 1) of qs[32(j>>1) + l] | bit j of qh[l] << 4
        w = d*sc_j*u - dmin*m_j, 6-bit sc_j / m_j packed as in GGUF (j >= 4 split
        into a low nibble in scales[8 + j - 4] and two top bits in scales[j - 4] / scales[j])
  Q6_K  210 B / 256 values: ql[128] | qh[64] | sc int8[16] | d f16
        value k = 128h + 32u + l: q = nibble (u >> 1) of ql[64h + 32(u & 1) + l]
        | 2 bits (2u) of qh[32h + l] << 4;  w = d*sc[k/16]*(q - 32)

All arithmetic is float32 in a fixed order, so the bytes are reproducible.
"""
import numpy as np

QK = 256


def gaussian(seed, shape, std=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def _f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _f16_val(bits):
    return bits.view(np.float16).astype(np.float32)


def quantize_q5k(w):
    """float32 [N, K] (K % 256 == 0) -> uint8 [N, K/256*176]."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    nsb = K // QK
    v = w.reshape(N, nsb, 8, 32)
    lo = v.min(-1)
    hi = v.max(-1)
    mn = np.where(lo < 0, -lo, np.float32(0)).astype(np.float32)
    scf = ((hi + mn) / np.float32(31)).astype(np.float32)
    dh = _f16_bits(scf.max(-1) / np.float32(63))
    mh = _f16_bits(mn.max(-1) / np.float32(63))
    d = _f16_val(dh)[..., None]
    dmin = _f16_val(mh)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d > 0, np.clip(np.ceil(scf / d), 0, 63), 0).astype(np.int32)
        m = np.where(dmin > 0, np.clip(np.ceil(mn / dmin), 0, 63), 0).astype(np.int32)
        ds = (d * sc.astype(np.float32)).astype(np.float32)
        dm = (dmin * m.astype(np.float32)).astype(np.float32)
        u = np.where(ds[..., None] > 0, np.rint((v + dm[..., None]) / ds[..., None]), 0)
    u = np.clip(u, 0, 31).astype(np.uint8)                      # [N, nsb, 8, 32]
    out = np.zeros((N, nsb, 176), np.uint8)
    out[:, :, 0:2] = dh[..., None].view(np.uint8).reshape(N, nsb, 2)
    out[:, :, 2:4] = mh[..., None].view(np.uint8).reshape(N, nsb, 2)
    s = np.zeros((N, nsb, 12), np.int32)
    s[:, :, 0:4] = (sc[:, :, 0:4] & 63) | ((sc[:, :, 4:8] >> 4) << 6)
    s[:, :, 4:8] = (m[:, :, 0:4] & 63) | ((m[:, :, 4:8] >> 4) << 6)
    s[:, :, 8:12] = (sc[:, :, 4:8] & 0xF) | ((m[:, :, 4:8] & 0xF) << 4)
    out[:, :, 4:16] = s.astype(np.uint8)
    qh = np.zeros((N, nsb, 32), np.uint8)
    for j in range(8):
        qh |= ((u[:, :, j, :] >> 4) & 1) << j
    out[:, :, 16:48] = qh
    qs = (u[:, :, 0::2, :] & 0xF) | ((u[:, :, 1::2, :] & 0xF) << 4)  # [N, nsb, 4, 32]
    out[:, :, 48:176] = qs.reshape(N, nsb, 128)
    return out.reshape(N, nsb * 176)


def quantize_q6k(w):
    """float32 [N, K] (K % 256 == 0) -> uint8 [N, K/256*210]."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    nsb = K // QK
    v = w.reshape(N, nsb, 16, 16)
    a = np.abs(v)
    idx = a.argmax(-1)
    amax = np.take_along_axis(a, idx[..., None], -1)[..., 0]
    vmax = np.take_along_axis(v, idx[..., None], -1)[..., 0]
    sf = (np.where(vmax < 0, -amax, amax) / np.float32(31)).astype(np.float32)
    dh = _f16_bits((amax / np.float32(31)).max(-1) / np.float32(127))
    d = _f16_val(dh)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        r = (sf / d).astype(np.float32)
        sc = np.where(d > 0, np.clip(np.where(r < 0, np.floor(r), np.ceil(r)), -127, 127), 0).astype(np.int32)
        scale = (d * sc.astype(np.float32)).astype(np.float32)
        q = np.where(scale[..., None] != 0, np.rint(v / scale[..., None]), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(N, nsb, 2, 4, 32)  # [h][u][l]
    out = np.zeros((N, nsb, 210), np.uint8)
    ql = np.zeros((N, nsb, 2, 2, 32), np.uint8)
    for u in range(4):
        ql[:, :, :, u & 1, :] |= (q[:, :, :, u, :] & 0xF) << (4 * (u >> 1))
    out[:, :, 0:128] = ql.reshape(N, nsb, 128)
    qh = np.zeros((N, nsb, 2, 32), np.uint8)
    for u in range(4):
        qh |= ((q[:, :, :, u, :] >> 4) & 3) << (2 * u)
    out[:, :, 128:192] = qh.reshape(N, nsb, 64)
    out[:, :, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, :, 208:210] = dh[..., None].view(np.uint8).reshape(N, nsb, 2)
    return out.reshape(N, nsb * 210)


def q5k_bytes(N, K):
    return N * (K // QK) * 176


def q6k_bytes(N, K):
    return N * (K // QK) * 210
