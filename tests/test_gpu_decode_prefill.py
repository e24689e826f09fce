"""The step over a prompt chunk (rows > 8): the reference's forward_batch_impl
as bruce_prefill_chunk calls it (engine/src/bruce.cu:8274-8291, :7610-7843
with all_logits = false), the projections on the prefill GEMMs (the W144
tier with the step's xdh and K-split workspace for the Q5_K parts, the W160
GEMM for the Q6_K ones) and the last row's logits only (:7833-7836).

Two layers of BASELINE config 5's shapes and a Q8_0 logits head (as in
tests/test_gpu_decode.py), 40 and 136 token rows, each row its own residual
stream, input_h and attention output.  Every row is an independent instance
of the one-row recurrence, so the checks are that file's, on six rows spread
over the chunk (the oracle's scalar GEMVs take about 0.4 s per row and
block):
* every block of a checked row matches the oracle's block applied to the
  GPU's previous row within 2e-4 normwise, taking the candidate rounding of
  codes that lie on a rounding boundary; the oracle's Q5_K projections take
  the W144 tier's numerics (its fp16 min term, bruce.cu:6604-6792, through
  oracle.gemm_q5k_144), as the reference's prefill does;
* the last row's logits match the oracle's Q8_0 head on its final q8 row
  within 1e-4, and the logits buffer holds nothing else;
* each checked row's residual row after the whole chain from x0 stays
  within 2e-4 of the oracle's chain, the oracle taking the GPU's q8 code of
  a block's input where the two input rows straddle a rounding boundary (as
  in tests/test_gpu_decode.py) and the GPU's group scales xd (equal within
  2e-5: the fp16 min-term operand half(xd * xsum) turns a 1e-6 xd difference
  into a 2^-11 one where it crosses an fp16 rounding boundary); the logits
  are checked on the GPU's final q8 row above, not on the oracle chain's
  row, which requantizes to other codes at the boundaries;
* the captured graph replays bit-identically to the eager run, with
  unrelated eager work between replays;
* a 12-row chunk without xdh and workspace (the raw-Q5_K tier, whose exact
  min term is the plain oracle's) and with a Q6_K head passes the same checks.
"""
import ctypes

import numpy as np
import pytest

import test_gpu_decode as D
import test_gpu_decode_rows as DR
from helpers import dev, host

pytestmark = pytest.mark.gpu


class _W144Oracle:
    """The oracle with the W144 tier's numerics for Q5_K projections: the
    reference's prefill runs them on k_gemm_mmq_q5k_144 (bruce.cu:6604-6792),
    whose min term is the fp16 product of Dm and xdh = half(xd * xsum), not
    the exact one of the decode GEMV (oracle.gemm_q5k).  Across a requantized
    row that difference (up to ~1e-4 of an output) moves codes by far more
    than the boundary margin the candidate roundings cover, so each tier is
    checked against its own numerics.  Everything else is the oracle's."""

    def __init__(self, oracle):
        self._o, self._rep = oracle, {}

    def __getattr__(self, name):
        return getattr(self._o, name)

    def gemm_q5k(self, raw, xq, xd, xs):
        key = id(raw)
        if key not in self._rep:
            self._rep[key] = (raw, self._o.repack_q5k_144(raw, raw.shape[1] // 176 * 256))
        r144, rdm = self._rep[key][1]
        return self._o.gemm_q5k_144(r144, rdm, xq, xd, self._o.fill_xdh(xd, xs), raw.shape[0])


def _gpu_step_prefill(bq, m, R, scratch=True, head_q6=None):
    import torch
    E, A, FF, V = D.E, D.A, D.FF, D.V
    keep = []
    Dv = lambda a: keep.append(dev(np.ascontiguousarray(a))) or keep[-1]
    ptr = lambda t: t.data_ptr()

    def w5(raw, K, N):
        g = Dv(raw)
        rep, dm = bq.repack_q5k(g, K, N)
        keep.extend([rep, dm])
        return bq.make_weight(g, bq.TYPE_Q5_K, K, N, rep=rep, rep_min=dm)

    def w6(raw, K, N):
        g = Dv(raw)
        rep = bq.repack_q6k(g, K, N)
        keep.append(rep)
        return bq.make_weight(g, bq.TYPE_Q6_K, K, N, rep=rep)

    blocks = (bq.DecodeBlock * 4)()
    for l, L in enumerate(m["layers"]):
        qw = (bq.Weight * 4)()
        outs = []
        for i, (name, n, qt, raw) in enumerate(L["qkv"]):
            qw[i] = w5(raw, E, n) if qt == "q5k" else w6(raw, E, n)
            outs.append(torch.empty((R, n), device="cuda"))
        keep += [qw] + outs
        optr = (ctypes.c_void_p * 4)(*[o.data_ptr() for o in outs])
        keep.append(optr)
        wo, wg, wu, wd = w5(L["o"], A, E), w5(L["gate"], E, FF), w5(L["up"], E, FF), w6(L["down"], FF, E)
        keep += [wo, wg, wu, wd]
        a = blocks[2 * l]
        a.kind, a.norm_before, a.norm_after = bq.BLOCK_ATTN, int(l == 0), 0
        a.alpha = ptr(Dv(L["alpha_a"]))
        a.qkv, a.n_qkv, a.qkv_out = qw, 4, optr
        a.attn_out, a.attn_gate, a.sgate, a.n_attn = ptr(Dv(L["attn_out"])), outs[2].data_ptr(), ptr(Dv(L["sgate"])), A
        a.o = ctypes.pointer(wo)
        f = blocks[2 * l + 1]
        f.kind, f.norm_before, f.norm_after = bq.BLOCK_FFN, 0, int(l == len(m["layers"]) - 1)
        f.alpha = ptr(Dv(L["alpha_f"]))
        f.gate, f.up, f.down = ctypes.pointer(wg), ctypes.pointer(wu), ctypes.pointer(wd)
        f.s_gate, f.s_up, f.n_ff = ptr(Dv(L["sg"])), ptr(Dv(L["su"])), FF
    if head_q6 is None:
        head = bq.quantize_q8s(Dv(m["head"].view(np.int16)), E, V)
        keep.append(head)
    else:
        hw = bq.make_weight(Dv(head_q6), bq.TYPE_Q6_K, E, V)
        keep.append(hw)
    x = torch.empty((R, E), device="cuda")
    xq = torch.empty(R * FF, dtype=torch.int8, device="cuda")
    xd = torch.empty(R * FF // 32, device="cuda")
    xs = torch.empty(R * FF // 32, dtype=torch.int32, device="cuda")
    xdh = torch.empty(R * FF // 32, dtype=torch.int16, device="cuda")
    proj = torch.empty((R, E), device="cuda")
    fg, fu = torch.empty((R, FF), device="cuda"), torch.empty((R, FF), device="cuda")
    logits = torch.empty(2 * V, device="cuda")     # the second half must stay untouched
    # one workspace for every GEMM of the step: the largest any of them takes
    wb = max(bq.workspace_bytes(R, K, n) for K, n in ((E, 2 * A + 512), (E, 512), (A, E), (E, 2 * FF), (FF, E)))
    work = torch.empty(max(wb, 16) // 4, device="cuda")
    keep += [x, xq, xd, xs, xdh, proj, fg, fu, logits, blocks, work]
    st = bq.DecodeStep()
    st.n_blocks, st.blocks, st.n_embd, st.fold, st.rows = 4, blocks, E, 0, R
    st.x, st.input_h = x.data_ptr(), ptr(Dv(m["input_h"]))
    st.xq, st.xd, st.xsum = xq.data_ptr(), xd.data_ptr(), xs.data_ptr()
    st.proj, st.ffn_g, st.ffn_u = proj.data_ptr(), fg.data_ptr(), fu.data_ptr()
    if head_q6 is None:
        st.head_q8s, st.head_rs = head.data_ptr(), ptr(Dv(m["rs"]))
    else:
        st.head = ctypes.pointer(hw)
    st.vocab, st.logits = V, logits.data_ptr()
    if scratch:
        st.xdh, st.work, st.work_bytes = xdh.data_ptr(), work.data_ptr(), work.numel() * 4
    x0 = Dv(m["x0"])

    def reset():
        x.copy_(x0)
        q = bq.quantize_q8(x)
        xq[:R * E].copy_(q[0].view(-1))
        xd[:R * E // 32].copy_(q[1].view(-1))
        xs[:R * E // 32].copy_(q[2].view(-1))
        logits.fill_(float("nan"))
    return st, keep, reset, x, logits


@pytest.mark.parametrize("rows", [40, 136])
def test_decode_prefill_graph_vs_oracle(bq, oracle, rows):
    print(f"prompt chunk rows={rows}", flush=True)
    saved, D.MAX_AMBIG = D.MAX_AMBIG, 14
    try:
        _run(bq, oracle, rows)
    finally:
        D.MAX_AMBIG = saved


def test_decode_prefill_raw_tier_kquant_head(bq, oracle):
    """A 12-row chunk with no xdh and no workspace: the Q5_K projections take
    the raw-Q5_K GEMM (exact fp32 min term, so the plain oracle's numerics)
    unsplit, and a Q6_K head gives the last row's logits through the one-row
    GEMV on that row's q8 codes."""
    print("prompt chunk rows=12, raw tier, Q6_K head", flush=True)
    from helpers import weights
    saved, D.MAX_AMBIG = D.MAX_AMBIG, 14
    try:
        _run(bq, oracle, 12, scratch=False, head_q6=weights(3990, D.V, D.E, "q6k"))
    finally:
        D.MAX_AMBIG = saved


def _run(bq, oracle, rows, scratch=True, head_q6=None):
    import torch
    if scratch:
        oracle = _W144Oracle(oracle)
    m = DR._model_rows(bq, oracle, rows)
    st, keep, reset, x, logits = _gpu_step_prefill(bq, m, rows, scratch, head_q6)
    check = sorted({0, 1, rows // 3, rows // 2 + 1, rows - 2, rows - 1})
    rms = {r: DR._row_model(m, r) for r in check}
    prev = m["x0"].copy()
    gpu_x = []
    for nb in range(1, 5):
        st.n_blocks = nb
        reset()
        bq.decode_enqueue(st)
        torch.cuda.synchronize()
        got = host(x).copy()
        assert np.isfinite(got).all(), nb
        worst = 0.0
        for r in check:
            cands, namb = D._oracle_block(oracle, rms[r], nb - 1, prev[r])
            err, _ = D._closest(oracle, got[r], cands)
            worst = max(worst, err)
            assert err < 2e-4, (nb, r, err, namb)
        print(f"  block {nb - 1}: worst checked row vs oracle {worst:.2e}", flush=True)
        gpu_x.append(got)
        prev = got
    el = host(logits).copy()
    V = D.V
    assert np.isnan(el[V:]).all(), "logits past the last row's were written"
    last = rows - 1
    if head_q6 is None:
        lref = D._oracle_logits(oracle, rms[last], prev[last])
    else:
        q = oracle.q8_rows(prev[last][None])
        lref = oracle.gemm_q6k(head_q6, q[0], q[1])[0]
    lerr = oracle.normwise_err(el[:V], lref)
    print(f"  last row's logits vs oracle head: {lerr:.2e}", flush=True)
    assert lerr < 1e-4
    for r in check:
        rx = m["x0"][r].copy()
        for bi in range(4):
            like = gpu_x[bi - 1][r] if bi else None
            _, rx = D._closest(oracle, gpu_x[bi][r], D._oracle_block(oracle, rms[r], bi, rx, like, like_xd=scratch)[0])
        cx = oracle.normwise_err(prev[r], rx)
        assert cx < 2e-4, (r, cx)
    print(f"  whole chains of the checked rows within bounds", flush=True)
    g = bq.DecodeGraph(st)
    for rep in range(3):
        reset()
        torch.randn(1 << 20, device="cuda").sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        g.launch()
        torch.cuda.synchronize()
        assert np.array_equal(host(x).view(np.uint32), prev.view(np.uint32)), rep
        assert np.array_equal(host(logits)[:V].view(np.uint32), el[:V].view(np.uint32)), rep
    g.close()
