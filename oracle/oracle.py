"""numpy front end of the C oracle (oracle/bq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libbq_oracle.so")

QK = 256
Q5K_BYTES = 176
Q6K_BYTES = 210


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        S = ctypes.c_size_t
        sig = {
            "orc_gaussian": (None, [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, P, S]),
            "orc_h2f": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f2h_rn": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_q8_rows": (None, [P, I, I, P, P, P]),
            "orc_fill_xdh": (None, [P, P, S, P]),
            "orc_quantize_q5k": (None, [P, I, I, P]),
            "orc_quantize_q6k": (None, [P, I, I, P]),
            "orc_q5k_scale": (None, [P, I, P, P]),
            "orc_q5k_code": (I, [P, I]),
            "orc_q6k_code": (I, [P, I]),
            "orc_q6k_sc": (I, [P, I]),
            "orc_dequant_q5k": (None, [P, I, I, P]),
            "orc_dequant_q6k": (None, [P, I, I, P]),
            "orc_dots_q5k": (None, [P, P, I, I, I, P]),
            "orc_dots16_q6k": (None, [P, P, I, I, I, P]),
            "orc_gemm_q5k": (None, [P, P, P, P, I, I, I, P]),
            "orc_gemm_q5k_f32": (None, [P, P, P, P, I, I, I, P]),
            "orc_gemm_q6k": (None, [P, P, P, I, I, I, P]),
            "orc_gemm_q6k_f32": (None, [P, P, P, I, I, I, P]),
            "orc_gemm_q5k_144": (None, [P, P, P, P, P, I, I, I, P]),
            "orc_repack_q5k_144": (None, [P, I, I, P, P]),
            "orc_repack_q6k_160": (None, [P, I, I, P]),
            "orc_quantize_q8s": (None, [P, I, I, P]),
            "orc_gemv_q8s": (None, [P, I, I, I, P, P, P, P]),
            "orc_norm_rows": (None, [I, P, P, P, P, I, I, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- data
def gaussian(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    lib().orc_gaussian(seed, mean, std, _p(out), n)
    return out


def q8_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    xq = np.empty((M, K), np.int8)
    xd = np.empty((M, K // 32), np.float32)
    xs = np.empty((M, K // 32), np.int32)
    lib().orc_q8_rows(_p(x), M, K, _p(xq), _p(xd), _p(xs))
    return xq, xd, xs


def fill_xdh(xd, xsum):
    xd = np.ascontiguousarray(xd, np.float32)
    xsum = np.ascontiguousarray(xsum, np.int32)
    out = np.empty(xd.shape, np.uint16)
    lib().orc_fill_xdh(_p(xd), _p(xsum), xd.size, _p(out))
    return out


def quantize_q5k(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty((N, K // QK * Q5K_BYTES), np.uint8)
    lib().orc_quantize_q5k(_p(w), N, K, _p(out))
    return out


def quantize_q6k(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty((N, K // QK * Q6K_BYTES), np.uint8)
    lib().orc_quantize_q6k(_p(w), N, K, _p(out))
    return out


def dequant_q5k(raw, K):
    N = raw.shape[0]
    out = np.empty((N, K), np.float32)
    lib().orc_dequant_q5k(_p(raw), N, K, _p(out))
    return out


def dequant_q6k(raw, K):
    N = raw.shape[0]
    out = np.empty((N, K), np.float32)
    lib().orc_dequant_q6k(_p(raw), N, K, _p(out))
    return out


def dots_q5k(raw, xq):
    M, K = xq.shape
    N = raw.shape[0]
    out = np.empty((M, N, K // 32), np.int32)
    lib().orc_dots_q5k(_p(raw), _p(xq), M, N, K, _p(out))
    return out


def dots16_q6k(raw, xq):
    M, K = xq.shape
    N = raw.shape[0]
    out = np.empty((M, N, K // 16), np.int32)
    lib().orc_dots16_q6k(_p(raw), _p(xq), M, N, K, _p(out))
    return out


def gemm_q5k(raw, xq, xd, xs):
    M, K = xq.shape
    N = raw.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_gemm_q5k(_p(raw), _p(xq), _p(xd), _p(xs), M, N, K, _p(y))
    return y


def gemm_q5k_f32(raw, xq, xd, xs):
    M, K = xq.shape
    N = raw.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_gemm_q5k_f32(_p(raw), _p(xq), _p(xd), _p(xs), M, N, K, _p(y))
    return y


def gemm_q6k(raw, xq, xd):
    M, K = xq.shape
    N = raw.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_gemm_q6k(_p(raw), _p(xq), _p(xd), M, N, K, _p(y))
    return y


def gemm_q6k_f32(raw, xq, xd):
    M, K = xq.shape
    N = raw.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_gemm_q6k_f32(_p(raw), _p(xq), _p(xd), M, N, K, _p(y))
    return y


def gemm_q5k_144(w144, dm, xq, xd, xdh, N):
    M, K = xq.shape
    y = np.empty((M, N), np.float64)
    lib().orc_gemm_q5k_144(_p(w144), _p(dm), _p(xq), _p(xd), _p(xdh), M, N, K, _p(y))
    return y


def repack_q5k_144(raw, K):
    N = raw.shape[0]
    w144 = np.empty((K // 128, N, 144), np.uint8)
    dm = np.empty((N, K // 32), np.uint16)
    lib().orc_repack_q5k_144(_p(raw), K, N, _p(w144), _p(dm))
    return w144, dm


def repack_q6k_160(raw, K):
    N = raw.shape[0]
    out = np.empty((N, K // 128, 160), np.uint8)
    lib().orc_repack_q6k_160(_p(raw), K, N, _p(out))
    return out


Q8S_BYTES = 272  # Q8_0 logits head: 8 fp16 scales + 256 int8 per (row, 256 values)


def quantize_q8s(w_bf16):
    """bf16 bit patterns uint16 [N, K] -> Q8S uint8 [N, K/256*272]."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    N, K = w.shape
    out = np.empty((N, K // QK * Q8S_BYTES), np.uint8)
    lib().orc_quantize_q8s(_p(w), K, N, _p(out))
    return out


def gemv_q8s(w, K, xq, xd, rs=None):
    """Q8S [N, K/256*272] x q8 rows -> float64 [M, N]."""
    N = w.shape[0]
    xq = np.ascontiguousarray(xq, np.int8).reshape(-1, K)
    M = xq.shape[0]
    xd = np.ascontiguousarray(xd, np.float32)
    y = np.empty((M, N), np.float64)
    rsa = None if rs is None else np.ascontiguousarray(rs, np.float32)
    lib().orc_gemv_q8s(_p(w), K, N, M, _p(xq), _p(xd), None if rsa is None else _p(rsa), _p(y))
    return y


NORM_OPS = {"norm": 0, "add": 1, "resid": 2, "gate": 3, "silu": 4}


def norm_rows(op, a, b=None, c=None, d=None):
    """float64 rows v of the reference's norm kernels (see orc_norm_rows)."""
    a = np.ascontiguousarray(a, np.float32)
    rows, n = a.shape
    arr = [None if t is None else np.ascontiguousarray(t, np.float32) for t in (b, c, d)]
    out = np.empty((rows, n), np.float64)
    lib().orc_norm_rows(NORM_OPS[op], _p(a), *[None if t is None else _p(t) for t in arr], rows, n, _p(out))
    return out


def f32_to_bf16(x):
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def q5k_scale(scales12, js):
    s = np.ascontiguousarray(scales12, np.uint8)
    sc = ctypes.c_int()
    m = ctypes.c_int()
    lib().orc_q5k_scale(_p(s), js, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


# ---------------------------------------------------------------- helpers
def normwise_err(y, ref):
    """max |y - ref| over each row / max |ref| of that row (rows = activation rows)."""
    y = np.asarray(y, np.float64).reshape(ref.shape)
    ref = np.asarray(ref, np.float64)
    if ref.ndim == 1:
        ref = ref[None]
        y = y[None]
    num = np.abs(y - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-30)
    return float((num / den).max())


def elementwise_err(y, ref, floor=1e-2):
    """max over elements of |y - ref| / max(|ref|, floor * max |ref| of its row):
    the relative error of each output, with outputs smaller than `floor` times
    the row's largest measured against that floor (an output near zero is a
    cancellation of large terms, whose fp32 rounding scales with the terms,
    not with the output)."""
    y = np.asarray(y, np.float64).reshape(np.shape(ref))
    ref = np.asarray(ref, np.float64)
    if ref.ndim == 1:
        ref = ref[None]
        y = y[None]
    fl = np.maximum(floor * np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
    return float((np.abs(y - ref) / np.maximum(np.abs(ref), fl)).max())
