"""The decode step (bq_decode_enqueue / bq_decode_graph_*): the reference's
per-token launch sequence (forward_launch, engine/src/bruce.cu:7902-8037)
over a block list, replayed from one captured HIP graph (capture_graph
:8046-8055).

Two layers of BASELINE config 5's shapes (hidden 3072, attention width 4096,
FF 9216; QKV as Q5_K q / k / gate parts plus a Q6_K v, O Q5_K, gate/up Q5_K,
down Q6_K) and a Q8_0 logits head are run eagerly and from the graph:
* every block matches the oracle's block -- the same sequence evaluated with
  the oracle's GEMVs (double precision over the q8 codes), norms
  (orc_norm_rows) and quantizer -- applied to the same input row, within 2e-4
  normwise.  Inside a block one fp32 row is requantized (the gate norm of
  attention, the silu*mul norm of the FFN).  The GPU computes its norm in
  fp32 (a tree-ordered sum of squares), the oracle in double, so a value
  whose exact code-space value t/d lies within AMBIG of a rounding boundary
  may round either way; one such code moving by one shifts the block output
  by about 2e-4.  The oracle therefore also evaluates the block with those
  codes rounded the other way (every combination of up to MAX_AMBIG codes;
  the GEMV after the requantization is linear in the codes, so each flip is
  one extra oracle GEMV of a one-hot row), and the block must match one of
  these candidates;
* the logits match the oracle's Q8_0 head on the final q8 row within 1e-4;
* the whole chain from x0 stays within 2e-4 of the oracle's whole chain, the
  oracle taking at each block the candidate rounding that the GPU's block
  output matches, and the GPU's q8 code of the block's input (and of the
  final row the logits are taken from) where the two rows (equal to ~2e-7)
  straddle a rounding boundary;
* every graph replay is bit-identical to the eager run.
The folded forms (fold = 1: gate norm inside the O GEMV, silu*mul inside the
gate+up epilogue, its norm inside the down GEMV; fold = 2: also the resid ->
q8 of each FFN block inside the next attention block's QKV GEMV, the
residual row alternating between x and x_alt, the other updates as their own
launches) are checked the same way, and with fold = 2 the row the QKV GEMV
wrote must equal, bit for bit, the standalone producer's row that ended the
shorter step.
"""
import ctypes

import numpy as np
import pytest

from helpers import dev, host, weights

pytestmark = pytest.mark.gpu

E, A, FF, V = 3072, 4096, 9216, 8192
PARTS = [("q", A, "q5k"), ("k", 512, "q5k"), ("gate", A, "q5k"), ("v", 512, "q6k")]


def _model(bq, oracle):
    import torch
    g = lambda s, n, m=0.0, sd=1.0: oracle.gaussian(s, n, m, sd).astype(np.float32)
    layers = []
    for l in range(2):
        s0 = 3000 + 100 * l
        qkv = [(name, n, qt, weights(s0 + i, n, E, qt)) for i, (name, n, qt) in enumerate(PARTS)]
        layers.append({
            "qkv": qkv,
            "o": weights(s0 + 10, E, A, "q5k"),
            "gate": weights(s0 + 11, FF, E, "q5k"), "up": weights(s0 + 12, FF, E, "q5k"),
            "down": weights(s0 + 13, E, FF, "q6k"),
            "attn_out": g(s0 + 20, A), "sgate": g(s0 + 21, A, 1.0, 0.3),
            "sg": g(s0 + 22, FF, 1.0, 0.3), "su": g(s0 + 23, FF, 1.0, 0.3),
            "alpha_a": g(s0 + 24, E, 0.5, 0.2), "alpha_f": g(s0 + 25, E, 0.5, 0.2),
        })
    head_bf16 = oracle.f32_to_bf16(g(3900, V * E, 0.0, 0.02).reshape(V, E))
    return {"layers": layers, "x0": g(3901, E), "input_h": g(3902, E), "head": head_bf16,
            "rs": g(3903, V, 1.0, 0.1)}


AMBIG = 2e-4    # code units: |t/d - (k + 1/2)| below this can round either way
MAX_AMBIG = 10  # such codes per requantized row the check enumerates (2^10 roundings)


def _q8_flips(oracle, t):
    """The oracle's q8 row of the fp32 row t (1 x n), and the codes whose
    exact value t/d lies within AMBIG of a rounding boundary, each as (index,
    change to the code that rounds the other way)."""
    xq, xd, xs = oracle.q8_rows(t)
    d = np.repeat(xd[0].astype(np.float64), 32)
    v = np.divide(t[0].astype(np.float64), d, out=np.zeros_like(d), where=d > 0)
    amb = np.nonzero((np.abs(v - np.floor(v) - 0.5) < AMBIG) & (np.abs(v) < 127))[0]
    assert len(amb) <= MAX_AMBIG, f"{len(amb)} codes on a rounding boundary"
    flips = []
    for i in amb:
        lo = int(np.floor(v[i]))
        alt = lo if int(xq[0, i]) == lo + 1 else lo + 1
        flips.append((int(i), alt - int(xq[0, i])))
    return (xq, xd, xs), flips


def _gemv_candidates(gemv, q, flips):
    """The GEMV (double) of the q8 row q and of every rounding of its
    ambiguous codes.  The GEMV is linear in the codes and xsum, so a flipped
    code adds the GEMV of a one-hot code row (xsum changed alike)."""
    xq, xd, xs = q
    base = np.asarray(gemv(xq, xd, xs), np.float64)
    deltas = []
    for i, dv in flips:
        dq, ds = np.zeros_like(xq), np.zeros_like(xs)
        dq[0, i], ds[0, i // 32] = dv, dv
        deltas.append(np.asarray(gemv(dq, xd, ds), np.float64))
    for mask in range(1 << len(flips)):
        yield base + sum((deltas[j] for j in range(len(flips)) if mask >> j & 1), np.zeros_like(base))


def _oracle_block(oracle, m, bi, x, like=None, like_xd=False):
    """Block bi (even: attention of layer bi // 2, odd: its FFN) of the
    reference's sequence applied to the fp32 row x, with the oracle's GEMVs
    (double precision over the q8 codes), norms and quantizer.  Returns the
    candidate new x rows (fp32), one per rounding of the block's requantized
    row's ambiguous codes (_q8_flips), and the number of those codes.
    like (optional): the GPU's row that x stands for; where the q8 codes of
    the two differ, each such code of x lies on a rounding boundary (checked)
    and the block takes the GPU's code, as it takes the GPU's rounding of the
    requantized row.  like_xd: also take the GPU row's group scales xd
    (checked equal within 2e-5 relative: the two rows agree to ~1e-6), for
    a tier whose fp16 min-term operand half(xd * xsum) turns a 1e-6 xd
    difference into a 2^-11 one where it crosses an fp16 rounding boundary."""
    f32 = lambda a: np.asarray(a, np.float32)
    L = m["layers"][bi // 2]
    x = x[None]
    if bi == 0:
        x = f32(oracle.norm_rows("add", x, m["input_h"][None]))
    q = oracle.q8_rows(x)
    if like is not None:
        ql = oracle.q8_rows(like[None])
        diff = np.nonzero(q[0][0] != ql[0][0])[0]
        if len(diff):
            amb = {i for i, _ in _q8_flips(oracle, x)[1]}
            assert all(int(i) in amb for i in diff), ("input codes differ off a rounding boundary", diff)
            xq = ql[0].copy()
            xs = xq.reshape(1, -1, 32).astype(np.int32).sum(axis=2).astype(q[2].dtype)
            q = (xq, q[1], xs)
        if like_xd:
            assert np.allclose(ql[1], q[1], rtol=2e-5, atol=0), "group scales differ by more than the rows do"
            q = (q[0], ql[1].copy(), q[2])
    outs = []
    if bi % 2 == 0:
        ys = {}
        for name, n, qt, raw in L["qkv"]:
            ys[name] = f32(oracle.gemm_q5k(raw, *q) if qt == "q5k" else oracle.gemm_q6k(raw, q[0], q[1]))
        t = f32(oracle.norm_rows("gate", L["attn_out"][None], ys["gate"], L["sgate"][None]))
        qa, flips = _q8_flips(oracle, t)
        for proj in _gemv_candidates(lambda a, b, c: oracle.gemm_q5k(L["o"], a, b, c), qa, flips):
            outs.append(f32(oracle.norm_rows("resid", x, f32(proj), L["alpha_a"][None]))[0])
    else:
        yg, yu = f32(oracle.gemm_q5k(L["gate"], *q)), f32(oracle.gemm_q5k(L["up"], *q))
        t = f32(oracle.norm_rows("silu", yg, yu, L["sg"][None], L["su"][None]))
        qt, flips = _q8_flips(oracle, t)
        for proj in _gemv_candidates(lambda a, b, c: oracle.gemm_q6k(L["down"], a, b), qt, flips):
            xo = f32(oracle.norm_rows("resid", x, f32(proj), L["alpha_f"][None]))
            if bi == 2 * len(m["layers"]) - 1:
                xo = f32(oracle.norm_rows("norm", xo))
            outs.append(xo[0])
    return outs, len(flips)


def _closest(oracle, got, cands):
    errs = [oracle.normwise_err(got, c.astype(np.float64)) for c in cands]
    k = int(np.argmin(errs))
    return errs[k], cands[k]


def _oracle_logits(oracle, m, x, like=None):
    """The oracle's Q8_0 head on the q8 row of x.  like (optional): the GPU's
    final row that x stands for; where the two rows' q8 codes differ, each
    such code of x lies on a rounding boundary (checked) and the GPU's code is
    taken, as _oracle_block takes a block input's codes."""
    q = oracle.q8_rows(x[None])
    if like is not None:
        ql = oracle.q8_rows(like[None])
        diff = np.nonzero(q[0][0] != ql[0][0])[0]
        if len(diff):
            amb = {i for i, _ in _q8_flips(oracle, x[None])[1]}
            assert all(int(i) in amb for i in diff), ("final codes differ off a rounding boundary", diff)
            q = (ql[0], q[1], q[2])
    return oracle.gemv_q8s(oracle.quantize_q8s(m["head"]), E, q[0], q[1], m["rs"])[0]


def _gpu_step(bq, m, fold):
    """Device buffers and the bq_decode_step for the model (kept alive in `keep`)."""
    import torch
    keep = []
    D = lambda a: keep.append(dev(np.ascontiguousarray(a))) or keep[-1]
    ptr = lambda t: t.data_ptr()
    blocks = (bq.DecodeBlock * 4)()
    for l, L in enumerate(m["layers"]):
        qw = (bq.Weight * 4)()
        outs = []
        for i, (name, n, qt, raw) in enumerate(L["qkv"]):
            qw[i] = bq.make_weight(D(raw), bq.TYPE_Q5_K if qt == "q5k" else bq.TYPE_Q6_K, E, n)
            outs.append(torch.empty(n, device="cuda"))
        keep += [qw] + outs
        optr = (ctypes.c_void_p * 4)(*[o.data_ptr() for o in outs])
        keep.append(optr)
        wo = bq.make_weight(D(L["o"]), bq.TYPE_Q5_K, A, E)
        wg, wu = bq.make_weight(D(L["gate"]), bq.TYPE_Q5_K, E, FF), bq.make_weight(D(L["up"]), bq.TYPE_Q5_K, E, FF)
        wd = bq.make_weight(D(L["down"]), bq.TYPE_Q6_K, FF, E)
        keep += [wo, wg, wu, wd]
        a = blocks[2 * l]
        a.kind, a.norm_before, a.norm_after = bq.BLOCK_ATTN, int(l == 0), 0
        a.alpha = ptr(D(L["alpha_a"]))
        a.qkv, a.n_qkv, a.qkv_out = qw, 4, optr
        a.attn_out, a.attn_gate, a.sgate, a.n_attn = ptr(D(L["attn_out"])), outs[2].data_ptr(), ptr(D(L["sgate"])), A
        a.o = ctypes.pointer(wo)
        f = blocks[2 * l + 1]
        f.kind, f.norm_before, f.norm_after = bq.BLOCK_FFN, 0, int(l == len(m["layers"]) - 1)
        f.alpha = ptr(D(L["alpha_f"]))
        f.gate, f.up, f.down = ctypes.pointer(wg), ctypes.pointer(wu), ctypes.pointer(wd)
        f.s_gate, f.s_up, f.n_ff = ptr(D(L["sg"])), ptr(D(L["su"])), FF
        keep.append(outs)
    head = bq.quantize_q8s(D(m["head"].view(np.int16)), E, V)
    keep.append(head)
    x = torch.empty(E, device="cuda")
    xq = torch.empty(FF, dtype=torch.int8, device="cuda")
    xd = torch.empty(FF // 32, device="cuda")
    xs = torch.empty(FF // 32, dtype=torch.int32, device="cuda")
    proj, fg, fu = torch.empty(E, device="cuda"), torch.empty(FF, device="cuda"), torch.empty(FF, device="cuda")
    logits = torch.empty(V, device="cuda")
    xalt = torch.full((E,), float("nan"), device="cuda")
    keep += [x, xalt, xq, xd, xs, proj, fg, fu, logits, blocks]
    st = bq.DecodeStep()
    st.n_blocks, st.blocks, st.n_embd, st.fold = 4, blocks, E, fold
    st.x, st.input_h = x.data_ptr(), ptr(D(m["input_h"]))
    st.xq, st.xd, st.xsum = xq.data_ptr(), xd.data_ptr(), xs.data_ptr()
    st.proj, st.ffn_g, st.ffn_u = proj.data_ptr(), fg.data_ptr(), fu.data_ptr()
    st.head_q8s, st.head_rs, st.vocab, st.logits = head.data_ptr(), ptr(D(m["rs"])), V, logits.data_ptr()
    if fold == 2:
        st.x_alt = xalt.data_ptr()
    x0 = D(m["x0"])

    def reset():
        x.copy_(x0)
        q = bq.quantize_q8(x.view(1, E))
        xq[:E].copy_(q[0][0])
        xd[:E // 32].copy_(q[1][0])
        xs[:E // 32].copy_(q[2][0])
        logits.fill_(float("nan"))
    return st, keep, reset, x, logits, xalt


@pytest.mark.parametrize("fold", [0, 1, 2])
def test_decode_graph_vs_oracle(bq, oracle, fold):
    import torch
    print(f"decode step fold={fold}", flush=True)
    m = _model(bq, oracle)
    st, keep, reset, x, logits, xalt = _gpu_step(bq, m, fold)
    # block by block: the first nb - 1 blocks on the GPU, then block nb on the
    # GPU and in the oracle from the same fp32 row
    prev = m["x0"].copy()
    gpu_x = []
    for nb in range(1, 5):
        st.n_blocks = nb
        reset()
        bq.decode_enqueue(st)
        torch.cuda.synchronize()
        got = host(x).copy()
        cands, namb = _oracle_block(oracle, m, nb - 1, prev)
        err, _ = _closest(oracle, got, cands)
        print(f"  block {nb - 1}: x vs oracle {err:.2e} ({namb} codes within {AMBIG:g} of a rounding boundary, "
              f"unrounded-as-GPU error {oracle.normwise_err(got, cands[0].astype(np.float64)):.2e})", flush=True)
        assert err < 2e-4, (nb, err)
        if fold == 2 and nb >= 3:
            # x_alt holds block 1's residual row as block 2's QKV GEMV wrote it
            # (the folded producer): bit-identical to the standalone
            # producer's row that ended the 2-block step
            assert np.array_equal(host(xalt).view(np.uint32), gpu_x[1].view(np.uint32)), nb
        gpu_x.append(got)
        prev = got
    el = host(logits).copy()
    lerr = oracle.normwise_err(el, _oracle_logits(oracle, m, prev))
    print(f"  logits vs oracle head on the final q8 row: {lerr:.2e}", flush=True)
    assert lerr < 1e-4
    # the whole chain in the oracle from x0, each block's ambiguous roundings
    # (of its requantized row, and of its input row's q8 codes) taken as the
    # GPU's block output shows them (without that choice a code that rounds
    # the other way compounds over the blocks)
    rx = m["x0"].copy()
    for bi in range(4):
        e, rx = _closest(oracle, gpu_x[bi], _oracle_block(oracle, m, bi, rx, gpu_x[bi - 1] if bi else None)[0])
        print(f"  chain block {bi}: closest candidate {e:.2e}", flush=True)
    cx, cl = oracle.normwise_err(prev, rx), oracle.normwise_err(el, _oracle_logits(oracle, m, rx, prev))
    print(f"  whole chain vs oracle chain: x {cx:.2e}, logits {cl:.2e}", flush=True)
    assert cx < 2e-4 and cl < 2e-4
    # graph replays: bit-identical to the eager run
    ex = prev
    g = bq.DecodeGraph(st)
    for rep in range(3):
        reset()
        torch.randn(1 << 20, device="cuda").sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        g.launch()
        torch.cuda.synchronize()
        assert np.array_equal(host(x).view(np.uint32), ex.view(np.uint32)), rep
        assert np.array_equal(host(logits).view(np.uint32), el.view(np.uint32)), rep
    g.close()


def test_decode_rejects(bq):
    st = bq.DecodeStep()
    assert bq.load().bq_decode_enqueue(ctypes.byref(st), bq._stream()) == bq.BQ_EINVAL


def test_decode_fold2_rejects(bq):
    """fold = 2 needs x_alt (16-byte aligned, not x) and one row."""
    import torch
    st = bq.DecodeStep()
    blocks = (bq.DecodeBlock * 1)()
    st.n_blocks, st.blocks, st.n_embd, st.fold = 0, blocks, 3072, 2
    bufs = [torch.empty(8 * 3072, device="cuda") for _ in range(8)]
    st.x, st.xq, st.xd, st.xsum, st.proj, st.ffn_g, st.ffn_u = [b.data_ptr() for b in bufs[:7]]
    L = bq.load()
    run = lambda: L.bq_decode_enqueue(ctypes.byref(st), bq._stream())
    assert run() == bq.BQ_EINVAL                     # no x_alt
    st.x_alt = st.x
    assert run() == bq.BQ_EINVAL                     # x_alt is x
    st.x_alt = bufs[7].data_ptr() + 4
    assert run() == bq.BQ_EINVAL                     # misaligned
    st.x_alt = bufs[7].data_ptr()
    st.ffn_u = None
    assert run() == bq.BQ_OK                         # an empty block list
    st.rows = 2
    assert run() == bq.BQ_UNSUPPORTED
    st.rows, st.fold = 1, 3
    assert run() == bq.BQ_EINVAL
