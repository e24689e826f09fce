"""bq_gemm_b_fused_noalloc: the allocation-free variant of bq_gemm_b_fused
(xdh and the K-split workspace in the library's static device scratch).

Called through the C ABI, its outputs must equal bq_gemm_b_fused's given its
own xdh and a workspace of the scratch's workspace size (12 MiB for a call
that takes the W144 tier, which also keeps xdh in the scratch; 16 MiB for any
other: the same split, so bit for bit), and the oracle's within 1e-4 -- on
two calls in a row, the second with a smaller input, for the W144 and raw
tiers (K split and not) and the 8-row GEMV path; device free memory does not
change across the calls; a W144 input beyond the xdh region is rejected with
BQ_ETOOBIG, while a Q6_K call of as many rows (no xdh) runs.
"""
import ctypes

import numpy as np
import pytest

from helpers import acts, check, dev, host, weights

pytestmark = pytest.mark.gpu

SCRATCH_WORK = 12 << 20   # the scratch's K-split workspace part beside the W144 tier's xdh
SCRATCH_ALL = 16 << 20    # the whole scratch: the workspace of every other call


def _arr(bq, ys, ws):
    return bq._arrays(ys, ws)


@pytest.mark.parametrize("prepacked", [True, False])
def test_noalloc_matches_gemm_b_fused(bq, oracle, prepacked):
    import torch
    K, Ns = 3072, [9216, 9216]
    L = bq.load()
    assert L.bq_noalloc_scratch_bytes() == 16 << 20
    ws, raws = [], []
    for i, n in enumerate(Ns):
        r = weights(2700 + i, n, K, "q5k")
        g = dev(r)
        raws.append(r)
        if prepacked:
            w144, dm = bq.repack_q5k(g, K, n)
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n, rep=w144, rep_min=dm))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
    work = torch.empty(SCRATCH_ALL // 4, device="cuda")
    for rows in (600, 128, 40, 5):        # each call after the first has a smaller input
        wbytes = SCRATCH_WORK if prepacked and rows > 8 else SCRATCH_ALL
        print(f"noalloc prepacked={prepacked} rows={rows}", flush=True)
        x, _ = acts(2710 + rows, rows, K)
        xq, xd, xs = oracle.q8_rows(x)
        gq, gd, gs = dev(xq), dev(xd), dev(xs)
        xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
        ya = [torch.full((rows, n), float("nan"), device="cuda") for n in Ns]
        yb = [torch.full((rows, n), float("nan"), device="cuda") for n in Ns]
        torch.cuda.synchronize()
        # the first launch of a kernel in a process loads its code object
        # (device memory the runtime takes once): load them before measuring
        yarr, warr = _arr(bq, ya, ws)
        assert L.bq_gemm_b_fused_noalloc(yarr, warr, 2, rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs),
                                         bq._stream()) == bq.BQ_OK
        for y in ya:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        yarr, warr = _arr(bq, ya, ws)
        assert L.bq_gemm_b_fused_noalloc(yarr, warr, 2, rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs),
                                         bq._stream()) == bq.BQ_OK
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0
        yarr2, warr2 = _arr(bq, yb, ws)
        assert L.bq_gemm_b_fused(yarr2, warr2, 2, rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs), bq._ptr(xdh),
                                 bq._ptr(work), wbytes, bq._stream()) == bq.BQ_OK
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(ya, yb)):
            a, b = host(a), host(b)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, i)
            if rows <= 128:   # oracle on the whole output; a 64-row sample at 600 rows
                sel = slice(None)
            else:
                sel = np.sort(np.random.default_rng(rows).choice(rows, 64, replace=False))
            r = raws[i]
            if prepacked and rows > 16:
                r144, rdm = oracle.repack_q5k_144(r, K)
                ref = oracle.gemm_q5k_144(r144, rdm, xq[sel], xd[sel], oracle.fill_xdh(xd[sel], xs[sel]), Ns[i])
            else:
                ref = oracle.gemm_q5k(r, xq[sel], xd[sel], xs[sel])
            check(oracle, a[sel], ref, what=f"rows {rows} part {i}")


def test_noalloc_rejects_too_big(bq):
    import torch
    K, N = 4096, 128
    rows = (4 << 20) // (K // 32 * 2) + 1          # xdh one row past its 4 MiB region
    raw = torch.zeros((N, K // 256 * 176), dtype=torch.uint8, device="cuda")
    # a prepacked weight: the W144 tier is the one that needs xdh (the check
    # comes before anything reads the weight)
    rep = torch.zeros(K // 128 * N * 144, dtype=torch.uint8, device="cuda")
    rep_min = torch.zeros(N * (K // 32), dtype=torch.int16, device="cuda")
    w = bq.make_weight(raw, bq.TYPE_Q5_K, K, N, rep=rep, rep_min=rep_min)
    y = torch.empty((1, N), device="cuda")
    yarr, warr = _arr(bq, [y], [w])
    L = bq.load()
    assert L.bq_gemm_b_fused_noalloc(yarr, warr, 1, rows, None, None, None, bq._stream()) == bq.BQ_ETOOBIG
    assert "static scratch" in bq.strerror(bq.BQ_ETOOBIG)


def test_noalloc_q6k_rows_past_xdh_region(bq, oracle):
    """Only the W144 tier reads xdh: a Q6_K down projection (K = 9216) of more
    rows than the xdh region could hold runs, with the whole scratch as its
    K-split workspace, and equals bq_gemm_b_fused given a 16 MiB workspace."""
    import torch
    K, N = 9216, 128
    rows = (4 << 20) // (K // 32 * 2) + 16         # 7298 rows: xdh would need 4.2 MB
    L = bq.load()
    raw = weights(2800, N, K, "q6k")
    g = dev(raw)
    w160 = bq.repack_q6k(g, K, N)
    w = bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=w160)
    x, _ = acts(2801, rows, K)
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    ya = torch.full((rows, N), float("nan"), device="cuda")
    yb = torch.full((rows, N), float("nan"), device="cuda")
    work = torch.empty(SCRATCH_ALL // 4, device="cuda")
    print(f"noalloc q6k rows={rows}", flush=True)
    yarr, warr = _arr(bq, [ya], [w])
    assert L.bq_gemm_b_fused_noalloc(yarr, warr, 1, rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs),
                                     bq._stream()) == bq.BQ_OK
    yarr2, warr2 = _arr(bq, [yb], [w])
    assert L.bq_gemm_b_fused(yarr2, warr2, 1, rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs), None,
                             bq._ptr(work), SCRATCH_ALL, bq._stream()) == bq.BQ_OK
    torch.cuda.synchronize()
    a, b = host(ya), host(yb)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    sel = np.sort(np.random.default_rng(2802).choice(rows, 48, replace=False))
    check(oracle, a[sel], oracle.gemm_q6k(raw, xq[sel], xd[sel]), what="q6k rows past the xdh region")
