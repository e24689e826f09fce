"""The decode step over rows 2..8 (the speculative-verify step): the
reference's forward_batch_impl with all logits (engine/src/bruce.cu:7610-7843),
captured once per row count as capture_verify_graphs does (:7877-7900) and
replayed as verify_launch does (:7862-7875).

Two layers of BASELINE config 5's shapes and a Q8_0 logits head (as in
tests/test_gpu_decode.py) over rows = 2, 4 and 8 token rows, each row its own
residual stream, input_h and attention output.  Every row is an independent
instance of the one-row recurrence, so the checks are that file's, per row:
* every block of every row matches the oracle's block applied to the GPU's
  previous row, within 2e-4 normwise, taking the candidate rounding of codes
  that lie on a rounding boundary (see tests/test_gpu_decode.py);
* every row's logits match the oracle's Q8_0 head on its final q8 row within 1e-4;
* every row's whole chain from x0 stays within 2e-4 of the oracle's chain;
* the graph of each row count replays bit-identically to its eager run, with
  unrelated eager work between replays;
* fold = 1 with more than one row is refused (BQ_UNSUPPORTED), and more
  than BQ_MAX_STEP_ROWS rows are invalid.
"""
import ctypes

import numpy as np
import pytest

import test_gpu_decode as D
from helpers import dev, host, weights

pytestmark = pytest.mark.gpu


def _model_rows(bq, oracle, R):
    m = D._model(bq, oracle)
    g = lambda s, n, mean=0.0, sd=1.0: oracle.gaussian(s, n, mean, sd).astype(np.float32)
    m["x0"] = np.stack([m["x0"]] + [g(3950 + r, D.E) for r in range(1, R)])
    m["input_h"] = np.stack([m["input_h"]] + [g(3970 + r, D.E) for r in range(1, R)])
    for l, L in enumerate(m["layers"]):
        L["attn_out"] = np.stack([L["attn_out"]] + [g(3990 + 10 * l + r, D.A) for r in range(1, R)])
    return m


def _row_model(m, r):
    """The one-row model of row r (the shape tests/test_gpu_decode.py's oracle takes)."""
    mr = dict(m)
    mr["x0"], mr["input_h"] = m["x0"][r], m["input_h"][r]
    mr["layers"] = [dict(L, attn_out=L["attn_out"][r]) for L in m["layers"]]
    return mr


def _gpu_step_rows(bq, m, R):
    import torch
    E, A, FF, V = D.E, D.A, D.FF, D.V
    keep = []
    Dv = lambda a: keep.append(dev(np.ascontiguousarray(a))) or keep[-1]
    ptr = lambda t: t.data_ptr()
    blocks = (bq.DecodeBlock * 4)()
    for l, L in enumerate(m["layers"]):
        qw = (bq.Weight * 4)()
        outs = []
        for i, (name, n, qt, raw) in enumerate(L["qkv"]):
            qw[i] = bq.make_weight(Dv(raw), bq.TYPE_Q5_K if qt == "q5k" else bq.TYPE_Q6_K, E, n)
            outs.append(torch.empty((R, n), device="cuda"))
        keep += [qw] + outs
        optr = (ctypes.c_void_p * 4)(*[o.data_ptr() for o in outs])
        keep.append(optr)
        wo = bq.make_weight(Dv(L["o"]), bq.TYPE_Q5_K, A, E)
        wg, wu = bq.make_weight(Dv(L["gate"]), bq.TYPE_Q5_K, E, FF), bq.make_weight(Dv(L["up"]), bq.TYPE_Q5_K, E, FF)
        wd = bq.make_weight(Dv(L["down"]), bq.TYPE_Q6_K, FF, E)
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
    head = bq.quantize_q8s(Dv(m["head"].view(np.int16)), E, V)
    keep.append(head)
    x = torch.empty((R, E), device="cuda")
    xq = torch.empty(R * FF, dtype=torch.int8, device="cuda")
    xd = torch.empty(R * FF // 32, device="cuda")
    xs = torch.empty(R * FF // 32, dtype=torch.int32, device="cuda")
    proj = torch.empty((R, E), device="cuda")
    fg, fu = torch.empty((R, FF), device="cuda"), torch.empty((R, FF), device="cuda")
    logits = torch.empty((R, V), device="cuda")
    keep += [x, xq, xd, xs, proj, fg, fu, logits, blocks]
    st = bq.DecodeStep()
    st.n_blocks, st.blocks, st.n_embd, st.fold, st.rows = 4, blocks, E, 0, R
    st.x, st.input_h = x.data_ptr(), ptr(Dv(m["input_h"]))
    st.xq, st.xd, st.xsum = xq.data_ptr(), xd.data_ptr(), xs.data_ptr()
    st.proj, st.ffn_g, st.ffn_u = proj.data_ptr(), fg.data_ptr(), fu.data_ptr()
    st.head_q8s, st.head_rs, st.vocab, st.logits = head.data_ptr(), ptr(Dv(m["rs"])), V, logits.data_ptr()
    x0 = Dv(m["x0"])

    def reset():
        x.copy_(x0)
        q = bq.quantize_q8(x)
        xq[:R * E].copy_(q[0].view(-1))
        xd[:R * E // 32].copy_(q[1].view(-1))
        xs[:R * E // 32].copy_(q[2].view(-1))
        logits.fill_(float("nan"))
    return st, keep, reset, x, logits


@pytest.mark.parametrize("rows", [2, 4, 8])
def test_decode_rows_graph_vs_oracle(bq, oracle, rows):
    import torch
    print(f"decode step rows={rows}", flush=True)
    # more rows, more requantized rows: allow up to 14 boundary codes per row
    # (about 3.7 expected in a 9216-value row)
    saved, D.MAX_AMBIG = D.MAX_AMBIG, 14
    try:
        _run_rows(bq, oracle, rows)
    finally:
        D.MAX_AMBIG = saved


def _run_rows(bq, oracle, rows):
    import torch
    m = _model_rows(bq, oracle, rows)
    st, keep, reset, x, logits = _gpu_step_rows(bq, m, rows)
    rms = [_row_model(m, r) for r in range(rows)]
    prev = m["x0"].copy()
    gpu_x = []
    for nb in range(1, 5):
        st.n_blocks = nb
        reset()
        bq.decode_enqueue(st)
        torch.cuda.synchronize()
        got = host(x).copy()
        worst = 0.0
        for r in range(rows):
            cands, namb = D._oracle_block(oracle, rms[r], nb - 1, prev[r])
            err, _ = D._closest(oracle, got[r], cands)
            worst = max(worst, err)
            assert err < 2e-4, (nb, r, err, namb)
        print(f"  block {nb - 1}: worst row vs oracle {worst:.2e}", flush=True)
        gpu_x.append(got)
        prev = got
    el = host(logits).copy()
    for r in range(rows):
        lerr = oracle.normwise_err(el[r], D._oracle_logits(oracle, rms[r], prev[r]))
        assert lerr < 1e-4, (r, lerr)
        rx = m["x0"][r].copy()
        for bi in range(4):
            like = gpu_x[bi - 1][r] if bi else None
            _, rx = D._closest(oracle, gpu_x[bi][r], D._oracle_block(oracle, rms[r], bi, rx, like)[0])
        cx = oracle.normwise_err(prev[r], rx)
        cl = oracle.normwise_err(el[r], D._oracle_logits(oracle, rms[r], rx, prev[r]))
        assert cx < 2e-4 and cl < 2e-4, (r, cx, cl)
    print(f"  logits and whole chains of {rows} rows within bounds", flush=True)
    g = bq.DecodeGraph(st)
    for rep in range(3):
        reset()
        torch.randn(1 << 20, device="cuda").sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        g.launch()
        torch.cuda.synchronize()
        assert np.array_equal(host(x).view(np.uint32), prev.view(np.uint32)), rep
        assert np.array_equal(host(logits).view(np.uint32), el.view(np.uint32)), rep
    g.close()


def test_decode_rows_rejects_fold(bq):
    st = bq.DecodeStep()
    blocks = (bq.DecodeBlock * 1)()
    st.n_blocks, st.blocks, st.n_embd, st.fold, st.rows = 0, blocks, 3072, 1, 2
    import torch
    bufs = [torch.empty(8 * 3072, device="cuda") for _ in range(5)]
    st.x, st.xq, st.xd, st.xsum, st.proj = [b.data_ptr() for b in bufs]
    L = bq.load()
    assert L.bq_decode_enqueue(ctypes.byref(st), bq._stream()) == bq.BQ_UNSUPPORTED
    st.rows = 9                                     # a prompt chunk: fold = 1 is one-row only
    assert L.bq_decode_enqueue(ctypes.byref(st), bq._stream()) == bq.BQ_UNSUPPORTED
    st.rows = 8193                                  # above BQ_MAX_STEP_ROWS
    assert L.bq_decode_enqueue(ctypes.byref(st), bq._stream()) == bq.BQ_EINVAL
