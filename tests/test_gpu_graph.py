"""Graph capture of a decode chain through the C ABI (the reference replays one
captured graph per token, bruce.cu:8046-8073, and per verify step, :7877-7900).

One FFN block of the decode step, with real data dependencies:
    resid -> q8 x; gate+up GEMV (q8 x); silu*mul norm -> q8 t; down GEMV (q8 t);
    resid -> q8 x.
It is captured once into a HIP graph. The graph is then replayed several times,
with eager work and synchronisations between replays, and every replay must be
bit-identical to the eager run of the same chain. The library's kernels
record no memset nodes, so each replay starts from the state the test sets up.
"""
import numpy as np
import pytest

from helpers import check, dev, host, weights

pytestmark = pytest.mark.gpu


def test_decode_chain_graph_replay(bq, oracle):
    import torch
    K, FF = 3072, 9216
    wg = dev(weights(21, FF, K, "q5k"))
    wu = dev(weights(22, FF, K, "q5k"))
    wd = dev(weights(23, K, FF, "q6k"))
    Wg = bq.make_weight(wg, bq.TYPE_Q5_K, K, FF)
    Wu = bq.make_weight(wu, bq.TYPE_Q5_K, K, FF)
    Wd = bq.make_weight(wd, bq.TYPE_Q6_K, FF, K)
    g = lambda s, n, m=0.0, sd=1.0: dev(oracle.gaussian(s, n, m, sd))
    x0, upd = g(1, K).view(1, K), g(2, K, 0.0, 3.0).view(1, K)
    alpha, alpha2 = g(3, K, 0.5, 0.2), g(4, K, 0.5, 0.2)
    sg, su = g(5, FF, 1.0, 0.3), g(6, FF, 1.0, 0.3)
    x = torch.empty_like(x0)
    xq = torch.empty((1, K), dtype=torch.int8, device="cuda")
    xd = torch.empty((1, K // 32), device="cuda")
    xs = torch.empty((1, K // 32), dtype=torch.int32, device="cuda")
    tq = torch.empty((1, FF), dtype=torch.int8, device="cuda")
    td = torch.empty((1, FF // 32), device="cuda")
    ts = torch.empty((1, FF // 32), dtype=torch.int32, device="cuda")
    yg, yu = torch.empty((1, FF), device="cuda"), torch.empty((1, FF), device="cuda")
    proj = torch.empty((1, K), device="cuda")

    xq_first = torch.empty_like(xq)
    xd_first = torch.empty_like(xd)
    xs_first = torch.empty_like(xs)

    def chain():
        assert bq.norm_q8("resid", 1, K, a=x, b=upd, c=alpha, q8=(xq, xd, xs))[0] == bq.BQ_OK
        xq_first.copy_(xq)
        xd_first.copy_(xd)
        xs_first.copy_(xs)
        assert bq.verify_fused([yg, yu], [Wg, Wu], 1, xq, xd, xs) == bq.BQ_OK
        assert bq.norm_q8("silu", 1, FF, out=None, a=yg, b=yu, c=sg, d=su, q8=(tq, td, ts))[0] == bq.BQ_OK
        bq.gemv(proj, Wd, tq, td, ts)
        assert bq.norm_q8("resid", 1, K, a=x, b=proj, c=alpha2, q8=(xq, xd, xs))[0] == bq.BQ_OK

    def snapshot():
        torch.cuda.synchronize()
        return [host(t).copy() for t in (x, xq, xd, xs, tq, td, ts, yg, yu, proj)]

    # eager reference
    x.copy_(x0)
    chain()
    ref = snapshot()
    # capture (a side stream, as torch.cuda.graph does) and replay
    graph = torch.cuda.CUDAGraph()
    x.copy_(x0)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        chain()
    for rep in range(4):
        x.copy_(x0)
        for t in (xq, tq, yg, yu, proj):
            t.zero_()
        # unrelated eager work between replays
        scratch = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        graph.replay()
        got = snapshot()
        for a, b in zip(got, ref):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"replay {rep}"
        del scratch
    # Each stage of the chain against the oracle, on the inputs the chain
    # produced: the GEMVs within 1e-4 (normwise and elementwise, helpers.check),
    # the resid producer's q8 row bit-exact with the oracle quantizer of its
    # fp32 row.
    x1 = oracle.norm_rows("resid", host(x0), host(upd), host(alpha)).astype(np.float32)
    q1 = oracle.q8_rows(x1)
    assert np.mean(q1[0] == host(xq_first)) > 0.999
    check(oracle, ref[7], oracle.gemm_q5k(host(wg), *[host(t) for t in (xq_first, xd_first, xs_first)]),
          what="gate")
    check(oracle, ref[8], oracle.gemm_q5k(host(wu), *[host(t) for t in (xq_first, xd_first, xs_first)]),
          what="up")
    check(oracle, ref[9], oracle.gemm_q6k(host(wd), ref[4], ref[5]), what="down")
    x2 = oracle.norm_rows("resid", x1, ref[9], host(alpha2))
    assert oracle.normwise_err(ref[0], x2) < 1e-5
    assert np.array_equal(oracle.q8_rows(ref[0])[0], ref[1])
    # the q8 row of t is the oracle's silu*mul norm of the GEMV outputs (fp32
    # rounding of the norm may move a code that sits on a rounding boundary)
    t_ref = oracle.norm_rows("silu", ref[7], ref[8], host(sg), host(su)).astype(np.float32)
    rq, _, _ = oracle.q8_rows(t_ref)
    assert np.mean(rq == ref[4]) > 0.999
