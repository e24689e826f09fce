"""GPU parity of the Q8_0 logits head: bq_quantize_q8s (k_bf16_to_q8,
bruce.cu:5159-5184) and bq_gemv_q8s (k_gemm_q8_logits, bruce.cu:4409-4449).

The conversion must match the oracle and the host twin bit for bit. GEMV
outputs must be within TOL, normwise per activation row, of the oracle
evaluated in double precision.
"""
import numpy as np
import pytest

from helpers import acts, dev, host

pytestmark = pytest.mark.gpu
TOL = 1e-4


def bf16_weights(oracle, seed, N, K, std=0.02):
    w = oracle.f32_to_bf16(oracle.gaussian(seed, N * K, 0.0, std).reshape(N, K))
    w[0, :32] = 0                                                             # all-zero group
    if K >= 128:
        w[0, 32:64] = oracle.f32_to_bf16(np.full(32, 1e-38, np.float32))     # denormal half scale
        w[0, [40, 47]] = 0                     # id = inf there: 0 * inf = NaN -> code 0 (cvt.rni)
        w[-1, 64:96] = oracle.f32_to_bf16(np.linspace(-3e4, 3e4, 32).astype(np.float32))
    return w


@pytest.mark.parametrize("N,K", [(3, 256), (1000, 2560), (64, 4096), (7, 8192)])
def test_quantize_q8s_bitexact(bq, oracle, N, K):
    import torch
    w = bf16_weights(oracle, 600 + N, N, K)
    got = bq.quantize_q8s(dev(w.view(np.int16)), K, N)
    torch.cuda.synchronize()
    ref = oracle.quantize_q8s(w)
    assert np.array_equal(host(got), ref)
    assert np.array_equal(bq.quantize_q8s_host(w, K, N), ref)


CASES = [(1, 1, 256), (1, 77, 2560), (1, 1000, 3072), (1, 130, 4096), (2, 50, 1024), (3, 333, 2560),
         (4, 64, 3072), (5, 200, 512), (7, 31, 768), (8, 129, 2560), (8, 96, 4096)]


@pytest.mark.parametrize("rows,N,K", CASES)
@pytest.mark.parametrize("with_rs", [True, False])
def test_gemv_q8s(bq, oracle, rows, N, K, with_rs):
    import torch
    print(f"gemv_q8s rows={rows} N={N} K={K} rs={with_rs}", flush=True)
    wq = oracle.quantize_q8s(bf16_weights(oracle, 700 + N, N, K))
    _, (xq, xd, _) = acts(800 + rows, rows, K)
    rs = oracle.gaussian(900 + N, N, 1.0, 0.2) if with_rs else None
    y = torch.full((rows, N), float("nan"), device="cuda")
    assert bq.gemv_q8s(y, dev(wq), dev(xq), dev(xd), K, N, rows, None if rs is None else dev(rs)) == bq.BQ_OK
    torch.cuda.synchronize()
    ref = oracle.gemv_q8s(wq, K, xq, xd, rs)
    assert oracle.normwise_err(host(y), ref) < TOL


def test_gemv_q8s_offset_rows(bq, oracle):
    """The reference's prefill call passes bm_xq + (rows-1)*K (bruce.cu:7833-7836):
    a row slice of a larger activation block, with xsum absent."""
    import torch
    N, K = 200, 2560
    wq = oracle.quantize_q8s(bf16_weights(oracle, 41, N, K))
    _, (xq, xd, _) = acts(42, 6, K)
    gq, gd = dev(xq), dev(xd)
    y = torch.empty((1, N), device="cuda")
    assert bq.gemv_q8s(y, dev(wq), gq[5:], gd[5:], K, N, 1) == bq.BQ_OK
    torch.cuda.synchronize()
    assert oracle.normwise_err(host(y), oracle.gemv_q8s(wq, K, xq[5:], xd[5:])) < TOL


def test_gemv_q8s_full_head(bq, oracle):
    """The full 131072 x 3072 head (427.8 MB of Q8S), batch 1: device-generated
    bf16 weights; 512 sampled rows of the conversion and the GEMV are checked
    against the oracle, and scaling rs by 2 must double every output exactly."""
    import torch
    N, K = 131072, 3072
    print("gemv_q8s full head 131072x3072", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1234)
    wb = (torch.randn((N, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
    wq = bq.quantize_q8s(wb, K, N)
    _, (xq, xd, _) = acts(43, 1, K)
    rs = torch.rand(N, generator=g, device="cuda") + 0.5
    y1 = torch.empty((1, N), device="cuda")
    y2 = torch.empty((1, N), device="cuda")
    gq, gd = dev(xq), dev(xd)
    assert bq.gemv_q8s(y1, wq, gq, gd, K, N, 1, rs) == bq.BQ_OK
    assert bq.gemv_q8s(y2, wq, gq, gd, K, N, 1, rs * 2) == bq.BQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y2, y1 * 2)
    rows = np.unique(np.concatenate([np.arange(8), np.arange(N - 8, N),
                                     np.random.default_rng(5).integers(0, N, 496)]))
    idx = torch.from_numpy(rows).cuda()
    w_s = host(wb[idx]).view(np.uint16)
    q_s = host(wq[idx])
    assert np.array_equal(q_s, oracle.quantize_q8s(w_s))
    ref = oracle.gemv_q8s(q_s, K, xq, xd, host(rs[idx]))
    assert oracle.normwise_err(host(y1[:, idx]), ref) < TOL
    del wb, wq


def test_gemv_q8s_rejects(bq, oracle):
    import torch
    K, N = 4352, 16
    w = torch.zeros((N, K // 256 * 272), dtype=torch.uint8, device="cuda")
    xq = torch.zeros((1, K), dtype=torch.int8, device="cuda")
    xd = torch.zeros((1, K // 32), device="cuda")
    y = torch.zeros((1, N), device="cuda")
    L = bq.load()
    assert bq.gemv_q8s(y, w, xq, xd, K, N, 1) == bq.BQ_UNSUPPORTED             # K > 4096
    assert bq.gemv_q8s(y, w, xq, xd, 4096, N, 0) == bq.BQ_UNSUPPORTED          # rows 0
    assert bq.gemv_q8s(y, w, xq, xd, 4096, N, 9) == bq.BQ_UNSUPPORTED          # rows 9
    with pytest.raises(bq.BqError):
        bq.gemv_q8s(y, w, xq, xd, 1000, N, 1)                                  # K % 256
    import ctypes
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.bq_gemv_q8s(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(w.data_ptr() + 8),
                         ctypes.c_void_p(xq.data_ptr()), ctypes.c_void_p(xd.data_ptr()), 256, N, 1,
                         None, st) == bq.BQ_EINVAL                             # misaligned weights
    assert L.bq_quantize_q8s(ctypes.c_void_p(w.data_ptr() + 2), 256, 1, ctypes.c_void_p(w.data_ptr()),
                             st) == bq.BQ_EINVAL
    torch.cuda.synchronize()
    assert torch.count_nonzero(y) == 0
