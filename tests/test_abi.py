"""CPU checks of the C ABI: libbq.so loads, exports every function that
include/bq.h declares, and its host-only entry points match the oracle."""
import ctypes
import os
import re

import numpy as np

from helpers import weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "bq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bq_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_exports():
    import bq
    L = bq.load()
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(L, n), n
    assert sorted(names) == sorted(bq.EXPORTS)


def test_library_is_gfx950_hip():
    import bq
    data = open(bq.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert bq.load().bq_version().decode().startswith("bq ")


def test_strerror():
    import bq
    assert bq.strerror(0) == "ok"
    assert "unsupported" in bq.strerror(1)


def test_repack_q6k_host_matches_oracle(oracle):
    import bq
    for N, K in [(4, 256), (17, 1024)]:
        raw = weights(77 + N, N, K, "q6k")
        got = bq.repack_q6k_host(raw, K, N)
        assert np.array_equal(got, oracle.repack_q6k_160(raw, K))


def test_repack_sizes():
    import bq
    L = bq.load()
    assert L.bq_repack_q5k_bytes(3072, 9216) == 31850496
    assert L.bq_repack_q5k_min_bytes(3072, 9216) == 1769472
    assert L.bq_repack_q6k_bytes(9216, 3072) == 35389440


def test_host_repack_rejects_bad_shape():
    import bq
    L = bq.load()
    buf = (ctypes.c_uint8 * 1024)()
    assert L.bq_repack_q6k_host(buf, 100, 1, buf) == bq.BQ_EINVAL
    assert L.bq_repack_q6k_host(None, 256, 1, buf) == bq.BQ_EINVAL


def test_quantize_q8s_host_matches_oracle(oracle):
    """bq_quantize_q8s_host (q8k_quant_host, bruce.cu:4843-4867) on the CPU."""
    import bq
    for N, K in [(3, 256), (11, 2560)]:
        w = oracle.f32_to_bf16(oracle.gaussian(500 + N, N * K, 0.0, 0.02).reshape(N, K))
        w[0, :32] = 0
        w[0, 32:64] = oracle.f32_to_bf16(np.full(32, 1e-38, np.float32))   # tiny (denormal half scale)
        w[0, [33, 60]] = 0                                                  # id = inf: zeros stay 0
        w[1, 64:96] = oracle.f32_to_bf16(np.linspace(-3e4, 3e4, 32).astype(np.float32))
        got = bq.quantize_q8s_host(w, K, N)
        assert np.array_equal(got, oracle.quantize_q8s(w))


def test_q8s_sizes_and_rejects():
    import bq
    L = bq.load()
    assert L.bq_q8s_bytes(2560, 131072) == 356515840      # the reference's 356.5 MB logits head
    assert L.bq_q8s_bytes(3072, 131072) == 427819008
    buf = (ctypes.c_uint8 * 1024)()
    assert L.bq_quantize_q8s_host(buf, 100, 1, buf) == bq.BQ_EINVAL
    assert L.bq_quantize_q8s_host(None, 256, 1, buf) == bq.BQ_EINVAL


def test_workspace_bytes():
    """bq_gemm_workspace_bytes (host arithmetic only): the K-split workspace
    of the prefill GEMMs, at most 32 MiB for any shape."""
    import bq
    L = bq.load()
    # one token tile of a 9216-row matrix: 72 tiles -> 7 slices for the 512
    # slots, evened to 6 over the raw tier's 24 stages (4 each); the 32-token
    # tile (144 tiles, 768 slots) takes 5: the larger is reserved
    assert L.bq_gemm_workspace_bytes(64, 3072, 9216) == 6 * 64 * 9216 * 4
    # 1152 tiles = 4 x 256 + 128 leftover tiles: the W144 tier cuts each
    # leftover tile into 2 K slices of 128 x 128 fp32 partial tiles
    assert L.bq_gemm_workspace_bytes(2048, 3072, 9216) == 128 * 2 * 128 * 128 * 4
    assert L.bq_gemm_workspace_bytes(4096, 3072, 9216) == 0      # 2304 tiles = 9 x 256: no leftover
    assert L.bq_gemm_workspace_bytes(0, 3072, 9216) == 0
    worst = max(L.bq_gemm_workspace_bytes(r, 3072, n) for r in list(range(1, 600, 7)) + list(range(600, 9000, 97))
                for n in (128, 1024, 9216, 36864))
    assert worst <= 32 << 20
