"""GPU parity of bq_gate_up_silu: the gate and up GEMVs of one q8 row with the
elementwise silu*mul epilogue, h = silu(g*sg) * u * su, in one launch.

Reference: the two launches it replaces -- the two-part GEMV (bq_verify_fused
for Q5_K, bq_gemv per matrix for Q6_K: the same K split) followed by the
silu*mul producer.  g and u are the plain kernel's sums, so the producer's
norm of h (bq_norm_q8 "norm") must be bit-identical to the silu*mul producer
on g and u (bq_silu_mul_norm_q8), fp32 row and q8 row alike.  h itself is
checked against the oracle's GEMVs through the silu*mul formula (normwise
< 1e-4).
"""
import numpy as np
import pytest

from helpers import acts, dev, host, weights

pytestmark = pytest.mark.gpu

# (weight format, K, N): the decode gate+up (one wave per row, the shuffle
# epilogue), a K split over several waves (the LDS epilogue), Q6_K raw and W160
CASES = [
    ("q5k", 3072, 9216),
    ("q5k", 4096, 1024),
    ("q5k", 256, 32),
    ("q6k", 9216, 512),
    ("q6k_rep", 3072, 256),
]


def _weight(bq, fmt, raw, K, N):
    g = dev(raw)
    if fmt == "q5k":
        return g, bq.make_weight(g, bq.TYPE_Q5_K, K, N)
    if fmt == "q6k":
        return g, bq.make_weight(g, bq.TYPE_Q6_K, K, N)
    rep = bq.repack_q6k(g, K, N)
    return (g, rep), bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=rep)


@pytest.mark.parametrize("fmt,K,N", CASES)
def test_gate_up_silu_matches_two_launches(bq, oracle, fmt, K, N):
    import torch
    print(f"gate_up_silu {fmt} K={K} N={N}", flush=True)
    qt = "q5k" if fmt == "q5k" else "q6k"
    raw_g = weights(700 + K // 256, N, K, qt)
    raw_u = weights(701 + K // 256, N, K, qt)
    keep_g, wg = _weight(bq, fmt, raw_g, K, N)
    keep_u, wu = _weight(bq, fmt, raw_u, K, N)
    _, (xq, xd, xs) = acts(702, 1, K)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    sg = dev(oracle.gaussian(703, N, 1.0, 0.3).astype(np.float32))
    su = dev(oracle.gaussian(704, N, 1.0, 0.3).astype(np.float32))
    # two launches
    g = torch.empty(N, device="cuda")
    u = torch.empty(N, device="cuda")
    if fmt == "q5k":
        assert bq.verify_fused([g, u], [wg, wu], 1, gq, gd, gs) == bq.BQ_OK
    else:
        bq.gemv(g, wg, gq, gd, gs)
        bq.gemv(u, wu, gq, gd, gs)
    # one launch
    h = torch.full((N,), float("nan"), device="cuda")
    bq.gate_up_silu(h, wg, wu, sg, su, gq, gd, gs if fmt == "q5k" else None)
    # the silu*mul producer on (g, u) against the norm of h
    o1, o2 = torch.empty(N, device="cuda"), torch.empty(N, device="cuda")
    _, q1 = bq.norm_q8("silu", 1, N, out=o1.view(1, N), a=g.view(1, N), b=u.view(1, N), c=sg, d=su)
    _, q2 = bq.norm_q8("norm", 1, N, out=o2.view(1, N), a=h.view(1, N))
    torch.cuda.synchronize()
    assert np.array_equal(host(o1).view(np.uint32), host(o2).view(np.uint32))
    for a, b in zip(q1, q2):
        assert np.array_equal(host(a), host(b))
    # oracle: h from the oracle's GEMVs through the silu*mul formula
    if fmt == "q5k":
        rg, ru = oracle.gemm_q5k(raw_g, xq, xd, xs), oracle.gemm_q5k(raw_u, xq, xd, xs)
    else:
        rg, ru = oracle.gemm_q6k(raw_g, xq, xd), oracle.gemm_q6k(raw_u, xq, xd)
    gv = rg.astype(np.float64)[0] * host(sg).astype(np.float64)
    href = gv / (1.0 + np.exp(-gv)) * ru.astype(np.float64)[0] * host(su).astype(np.float64)
    assert oracle.normwise_err(host(h)[None], href[None]) < 1e-4
    del keep_g, keep_u


def test_gate_up_silu_rejects(bq):
    import torch
    K, N = 256, 32
    raw = dev(weights(710, N, K, "q5k"))
    w = bq.make_weight(raw, bq.TYPE_Q5_K, K, N)
    w16 = bq.make_weight(raw, bq.TYPE_Q5_K, K, 16)
    v = torch.zeros(N, device="cuda")
    xq = torch.zeros(K, dtype=torch.int8, device="cuda")
    xd = torch.zeros(K // 32, device="cuda")
    xs = torch.zeros(K // 32, dtype=torch.int32, device="cuda")
    with pytest.raises(bq.BqError) as e:
        bq.gate_up_silu(v, w, w16, v, v, xq, xd, xs)       # N differs
    assert e.value.code == bq.BQ_UNSUPPORTED
    with pytest.raises(bq.BqError):
        bq.gate_up_silu(v, w, w, v, v, xq, xd, None)      # Q5_K without xsum
