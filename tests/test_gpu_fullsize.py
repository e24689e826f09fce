"""Every output of the prefill GEMMs at BASELINE config 4's full size (M = 2048
and 8192), checked.

The oracle's scalar GEMM cannot finish M = 2048 x 9216 x 3072 in test time,
so the sampled oracle checks (test_gpu_pinned.py) are joined here by a
full-output cross-check against an independent kernel family: the multi-row
GEMV (bq_verify_fused / bq_q6_verify_fused, 8 activation rows per call),
which is itself pinned against the oracle at these shapes and every row
count.  The two share no code path (LDS-tiled int8 32x32x32 MFMA with K
split and per-group fp32 outer products vs. register-streamed dot4 / 4x4x4
MFMA lane tasks), so an indexing error in either shows up as a mismatch in
the outputs it touches.

The W144 tier computes the min term in fp16 (engine/src/bruce.cu:6604-6792:
sum_g f16(Dm) * f16(xdh)); the GEMV computes it exactly (-dmin*m * xd*xsum,
bruce.cu:384-440).  The difference is added to the GEMV's outputs exactly, in
float64, as a rank-K/32 product: Dm from the device repack (bit-exact with the
oracle, test_gpu_parity.py), xdh from the oracle, and dmin*m from a numpy
decode of the Q5_K header written from the block layout (d, dmin fp16;
scales[12]: m_j = scales[j+4] & 63 for j < 4, else
(scales[j+4] >> 4) | (scales[j] >> 6) << 4).

Tolerance: helpers.check, normwise 1e-4 per activation row and elementwise
1e-3 with a floor of 1e-2 x the row's largest output.
"""
import numpy as np
import pytest

from helpers import acts, check, dev, host, weights

pytestmark = pytest.mark.gpu

K, N = 3072, 9216   # BASELINE config 4 (M = 2048 and the bench's largest, 8192)
M = 2048


def _np_dmin_m(raw, K):
    """dmin * m_j per row and 32-value group, [N][K/32] float64."""
    n = raw.shape[0]
    b = raw.reshape(n, K // 256, 176)
    dmin = b[:, :, 2:4].copy().view(np.float16)[:, :, 0].astype(np.float64)
    s = b[:, :, 4:16].astype(np.int32)
    m = np.empty((n, K // 256, 8), np.int32)
    for j in range(8):
        if j < 4:
            m[:, :, j] = s[:, :, j + 4] & 63
        else:
            m[:, :, j] = (s[:, :, j + 4] >> 4) | ((s[:, :, j] >> 6) << 4)
    return (dmin[:, :, None] * m).reshape(n, K // 32)


def _gemv_chunks(fn, y, w, xq, xd, xs=None):
    """y[r0:r0+8] = GEMV of activation rows r0..r0+7, over all rows of y."""
    import torch
    for r0 in range(0, y.shape[0], 8):
        args = (xq[r0:r0 + 8], xd[r0:r0 + 8]) + ((xs[r0:r0 + 8],) if xs is not None else ())
        assert fn([y[r0:r0 + 8]], [w], 8, *args) == 0
    torch.cuda.synchronize()


def test_dmin_m_decoder_matches_oracle(oracle):
    """Pins the numpy min decoder above against the oracle's scale decode
    (which the GPU kernels are checked against) on every sub-block of a few
    blocks, including the split 6-bit fields of sub-blocks 4..7."""
    raw = weights(2400, 4, 512, "q5k")
    dm = _np_dmin_m(raw, 512)
    b = raw.reshape(4, 2, 176)
    for r in range(4):
        for sb in range(2):
            dmin = float(b[r, sb, 2:4].copy().view(np.float16)[0])
            for j in range(8):
                _, mj = oracle.q5k_scale(b[r, sb, 4:16], j)
                assert dm[r, 8 * sb + j] == dmin * mj


@pytest.mark.parametrize("M", [2048, 8192])
@pytest.mark.parametrize("prepacked", [False, True])
def test_config4_full_output_vs_gemv(bq, oracle, prepacked, M):
    import torch
    print(f"config4 full output M={M} prepacked={prepacked}", flush=True)
    raw = weights(2401, N, K, "q5k")
    x, (xq, xd, xs) = acts(2402 + M, M, K)
    gr = dev(raw)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    w_raw = bq.make_weight(gr, bq.TYPE_Q5_K, K, N)
    ref = torch.full((M, N), float("nan"), device="cuda")
    _gemv_chunks(bq.verify_fused, ref, w_raw, gq, gd, gs)
    ref = host(ref).astype(np.float64)
    assert np.isfinite(ref).all()

    if prepacked:
        w144, dmh = bq.repack_q5k(gr, K, N)
        w = bq.make_weight(gr, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dmh)
        xdh = oracle.fill_xdh(xd, xs)
        a16 = host(dmh).view(np.float16).reshape(N, K // 32).astype(np.float64)
        b16 = xdh.view(np.float16).astype(np.float64)
        xdxs = xd.astype(np.float64) * xs.astype(np.float64)
        # W144 min term minus the exact one, added to the GEMV's outputs
        ref += b16 @ a16.T + xdxs @ _np_dmin_m(raw, K).T
        gxdh = dev(xdh.view(np.int16))
    else:
        w = w_raw
        gxdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    y = torch.full((M, N), float("nan"), device="cuda")
    assert bq.try_mmq([y], [w], M, gq, gd, gs, gxdh) == bq.BQ_OK
    torch.cuda.synchronize()
    yh = host(y)
    assert np.isfinite(yh).all()
    check(oracle, yh, ref, what=f"MMQ vs GEMV, all {M}x{N} outputs")


def test_q6_gemm_full_output_vs_gemv(bq, oracle):
    """The Q6_K GEMM over W160 at the down projection's shape (3072 x 9216),
    M = 2048, every output against the W160 multi-row GEMV."""
    import torch
    Kq, Nq = 9216, 3072
    print(f"q6 gemm full output M={M}", flush=True)
    raw = weights(2403, Nq, Kq, "q6k")
    x, (xq, xd, _) = acts(2404, M, Kq)
    gr = dev(raw)
    gq, gd = dev(xq), dev(xd)
    w = bq.make_weight(gr, bq.TYPE_Q6_K, Kq, Nq, rep=bq.repack_q6k(gr, Kq, Nq))
    ref = torch.full((M, Nq), float("nan"), device="cuda")
    _gemv_chunks(bq.q6_verify_fused, ref, w, gq, gd)
    y = torch.full((M, Nq), float("nan"), device="cuda")
    bq.gemm_q6k_mma(y, w, M, gq, gd)
    torch.cuda.synchronize()
    yh, rh = host(y), host(ref)
    assert np.isfinite(yh).all() and np.isfinite(rh).all()
    check(oracle, yh, rh, what=f"Q6_K GEMM vs GEMV, all {M}x{Nq} outputs")
