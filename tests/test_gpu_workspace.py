"""The prefill GEMMs' K split with a caller-owned workspace.

A launch whose 128 x 128 tiles leave the GPU's workgroup slots unfilled is
split over K; the partial outputs go to the caller's workspace and a fixed-order
sum follows.  Checked here: multi-part launches (bq_gemm_b_fused, the
reference's launch_gemm_b_fused, bruce.cu:7421-7426) against the oracle at
every split class, bit-identical results for equal calls, and graph capture:
the same call captured in a HIP graph replays bit-identically to the eager
call (the reference captures these calls in its verify graphs,
bruce.cu:7877-7900), while device memory stays unchanged across calls (the
library allocates nothing).
"""
import ctypes

import numpy as np
import pytest

from helpers import acts, check, dev, host, weights

pytestmark = pytest.mark.gpu


def _parts(bq, seed, Ns, K, prepacked):
    raws = [weights(seed + i, n, K, "q5k") for i, n in enumerate(Ns)]
    ws = []
    for r, n in zip(raws, Ns):
        g = dev(r)
        if prepacked:
            w144, dm = bq.repack_q5k(g, K, n)
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n, rep=w144, rep_min=dm))
        else:
            ws.append(bq.make_weight(g, bq.TYPE_Q5_K, K, n))
    return raws, ws


def _ref(oracle, raw, K, n, xq, xd, xs, prepacked):
    if prepacked:
        w144, dm = oracle.repack_q5k_144(raw, K)
        return oracle.gemm_q5k_144(w144, dm, xq, xd, oracle.fill_xdh(xd, xs), n)
    return oracle.gemm_q5k(raw, xq, xd, xs)


@pytest.mark.parametrize("prepacked", [False, True])
@pytest.mark.parametrize("Ns", [[1024, 1024], [1024, 512, 256]])
@pytest.mark.parametrize("rows", [17, 28, 64, 128])
def test_gemm_b_fused_split(bq, oracle, prepacked, Ns, rows):
    import torch
    K = 3072
    print(f"gemm_b_fused Ns={Ns} rows={rows} prepacked={prepacked}", flush=True)
    raws, ws = _parts(bq, 2500 + rows, Ns, K, prepacked)
    x, _ = acts(2550 + rows, rows, K)
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    assert bq.workspace_bytes(rows, K, sum(Ns)) > 0   # these launches do split
    outs = []
    for work in ("auto", "auto", None):
        ys = [torch.full((rows, n), float("nan"), device="cuda") for n in Ns]
        bq.gemm_b_fused(ys, ws, rows, gq, gd, gs, xdh, work=work)
        torch.cuda.synchronize()
        outs.append([host(y) for y in ys])
    for a, b in zip(outs[0], outs[1]):                       # equal calls: equal bits
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for i, (r, n) in enumerate(zip(raws, Ns)):
        ref = _ref(oracle, r, K, n, xq, xd, xs, prepacked and rows >= 17)
        check(oracle, outs[0][i], ref, what=f"split part {i}")
        check(oracle, outs[2][i], ref, what=f"unsplit part {i}")


@pytest.mark.parametrize("rows", [17, 64, 128])
def test_gemm_b_graph_capture(bq, oracle, rows):
    """bq_gemm_b on the prompt-tail shape (W144 9216 x 3072, one token tile:
    split over K) captured in a HIP graph: every replay is bit-identical to
    the eager call with the same workspace, and device free memory does not
    change across eager calls, capture and replays."""
    import torch
    K, N = 3072, 9216
    print(f"gemm_b capture rows={rows}", flush=True)
    raw = weights(2600, N, K, "q5k")
    g = dev(raw)
    w144, dm = bq.repack_q5k(g, K, N)
    w = bq.make_weight(g, bq.TYPE_Q5_K, K, N, rep=w144, rep_min=dm)
    x, _ = acts(2601 + rows, rows, K)
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    xdh = torch.empty((rows, K // 32), dtype=torch.int16, device="cuda")
    work = bq.workspace(rows, K, N)
    assert work is not None
    y = torch.full((rows, N), float("nan"), device="cuda")
    L = bq.load()
    args = lambda: (bq._ptr(y), ctypes.byref(w), rows, bq._ptr(gq), bq._ptr(gd), bq._ptr(gs), bq._ptr(xdh),
                    bq._ptr(work), work.numel() * 4, bq._stream())
    assert L.bq_gemm_b(*args()) == bq.BQ_OK                     # first call: code objects load
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert L.bq_gemm_b(*args()) == bq.BQ_OK
    torch.cuda.synchronize()
    eager = host(y).copy()
    r144, rdm = oracle.repack_q5k_144(raw, K)
    check(oracle, eager, oracle.gemm_q5k_144(r144, rdm, xq, xd, oracle.fill_xdh(xd, xs), N), what="eager")
    assert torch.cuda.mem_get_info()[0] == free0
    graph = torch.cuda.CUDAGraph()
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        assert L.bq_gemm_b(*args()) == bq.BQ_OK
    for rep in range(3):
        y.fill_(float("nan"))
        work.fill_(float("nan"))
        torch.randn(1 << 20, device="cuda").sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(y).view(np.uint32), eager.view(np.uint32)), rep
    del graph


@pytest.mark.parametrize("prepacked", [True, False])
@pytest.mark.parametrize("M,Ns,K", [(1536, [9216], 3072), (2048, [9216], 3072), (2304, [9216], 3072),
                                    (2048, [9216, 2048], 3072), (2048, [7168], 2560)])
def test_q5k_leftover_tile_split(bq, oracle, M, Ns, K, prepacked):
    """Q5_K prefill GEMM (W144 and raw tiers) with more tiles than CUs and a
    remainder (M = 2048 on 9216 rows: 1152 tiles = 4 x 256 + 128; the reference
    model's 7168 x 2560 gate/up: 896 = 3 x 256 + 128): the leftover tiles run as K
    slices into the workspace and one more launch sums them.  Equal calls give
    equal bits; against the unsplit launch (no workspace) the outputs differ
    only by fp32 summation order; rows of the last token tile (whose tiles
    include leftover ones) are checked against the oracle."""
    import torch
    print(f"q5k leftover split M={M} Ns={Ns} K={K} prepacked={prepacked}", flush=True)
    assert bq.workspace_bytes(M, K, sum(Ns)) > 0
    raws, ws = _parts(bq, 2700 + M, Ns, K, prepacked)
    x, _ = acts(2750 + M, M, K)
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    outs = []
    for work in ("auto", "auto", None):
        ys = [torch.full((M, n), float("nan"), device="cuda") for n in Ns]
        assert bq.try_mmq(ys, ws, M, gq, gd, gs, xdh, work=work) == bq.BQ_OK
        torch.cuda.synchronize()
        outs.append([host(y) for y in ys])
    for i, n in enumerate(Ns):
        a, b, c = outs[0][i], outs[1][i], outs[2][i]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.isfinite(a).all()
        scale = np.abs(c).max(axis=1, keepdims=True)
        assert (np.abs(a - c) <= 1e-5 * scale).all(), f"part {i}: split vs unsplit"
        rows = np.arange(M - 12, M)                      # the last token tile's rows
        ref = _ref(oracle, raws[i], K, n, xq[rows], xd[rows], xs[rows], prepacked)
        check(oracle, a[rows], ref, what=f"part {i} last rows")


def test_w144_leftover_split_graph_capture(bq, oracle):
    """The leftover-tile split (two launches) captured in a HIP graph replays
    bit-identically to the eager call."""
    import torch
    K, N, M = 3072, 9216, 2048
    raws, ws = _parts(bq, 2800, [N], K, True)
    x, _ = acts(2801, M, K)
    xq, xd, xs = oracle.q8_rows(x)
    gq, gd, gs = dev(xq), dev(xd), dev(xs)
    xdh = torch.empty((M, K // 32), dtype=torch.int16, device="cuda")
    work = bq.workspace(M, K, N)
    y = torch.full((M, N), float("nan"), device="cuda")
    assert bq.try_mmq([y], ws, M, gq, gd, gs, xdh, work=work) == bq.BQ_OK
    torch.cuda.synchronize()
    eager = host(y).copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert bq.try_mmq([y], ws, M, gq, gd, gs, xdh, work=work) == bq.BQ_OK
    for rep in range(3):
        y.fill_(float("nan"))
        work.fill_(float("nan"))
        torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(y).view(np.uint32), eager.view(np.uint32)), rep
    del graph


def test_workspace_bytes_follow_the_device(bq):
    """bq_gemm_workspace_bytes sizes the split for the current device: it
    equals bq_gemm_workspace_bytes_cus at the device's CU count."""
    import torch
    L = bq.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for rows, n in ((64, 9216), (2048, 9216), (600, 18432), (16, 3072), (4096, 9216)):
        assert L.bq_gemm_workspace_bytes(rows, 3072, n) == L.bq_gemm_workspace_bytes_cus(rows, 3072, n, cus), \
            (rows, n, cus)
