#!/usr/bin/env python3
"""Benchmark of the MI355X k-quant matmul path (libbq) on one GPU.

Headline (BASELINE metric "GEMV GB/s (% HBM peak) at batch 1"): the decode FFN
GEMV set of BASELINE config 2 -- per step, quantize the block input (q8) and
run the fused gate+up Q5_K GEMV 2 x (9216 x 3072), then quantize the
down-projection input and run the down Q6_K GEMV 3072 x 9216 -- batch 1,
synthetic Gaussian data, weight sets rotated so the working set exceeds the
256 MB last-level cache.  Each quantize+GEMV pair is one bq_gemv_q8_fused
launch; the reference's four-launch form (bq_quantize_q8 + GEMV, twice) is
reported beside it.  Steps are replayed from a HIP graph holding one step per
weight set.  `value` is algorithmic bytes (GGUF weight bytes + q8 activations
+ fp32 outputs) per step x steps / timed region.

Also reported: the prefill GEMM of config 4 (M = 2048, int8 MFMA, TOPS and
fraction of the dense int8 peak), the multi-row GEMV of config 3, config 1,
and the reference's scalar host loop timed on this machine's CPU.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--decode-only]
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bruce-engine_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
METRIC = "GEMV GB/s (% HBM peak) at batch 1; prefill GEMM int8 TOPS (% MFMA peak)"
SEED = 0xB5CE
K, FF = 3072, 9216
LLC_BYTES = 256e6


def q8_bytes(rows, k):
    return rows * (k + (k // 32) * 8)


def gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9


def traffic_for(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    calibrated on a copy kernel), committed in profiles/traffic.json; None if absent."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def cpu_baseline(gate, up, down, x, t, threads, budget_s=12.0):
    """The reference's scalar host loop (restated in oracle/bq_oracle.c) on full
    decode FFN steps of the same inputs, with `threads` host threads splitting
    the output rows (the C calls release the GIL).  Returns (steps, seconds)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from concurrent.futures import ThreadPoolExecutor
    xq, xd, xs = O.q8_rows(x)
    tq, td, ts = O.q8_rows(t)
    jobs = []
    for w, fn, args in ((gate, O.gemm_q5k_f32, (xq, xd, xs)), (up, O.gemm_q5k_f32, (xq, xd, xs)),
                        (down, O.gemm_q6k_f32, (tq, td))):
        n = w.shape[0]
        for i in range(threads):
            lo, hi = n * i // threads, n * (i + 1) // threads
            jobs.append((fn, np.ascontiguousarray(w[lo:hi]), args))
    steps, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while True:
            list(ex.map(lambda j: j[0](j[1], *j[2]), jobs))
            steps += 1
            el = time.perf_counter() - t0
            if el > budget_s or steps >= 5000:
                break
    return steps, el


def cpu_rate(parts, threads, budget_s):
    """Time full passes of `parts` [(fn, w, args)] -- the oracle's scalar fp32
    restatement of the reference's host loop -- with each weight matrix's rows
    split over `threads` host threads (the C calls release the GIL).  Returns
    passes per second."""
    from concurrent.futures import ThreadPoolExecutor
    jobs = []
    for fn, w, args in parts:
        n = w.shape[0]
        for i in range(threads):
            lo, hi = n * i // threads, n * (i + 1) // threads
            if hi > lo:
                jobs.append((fn, np.ascontiguousarray(w[lo:hi]), args))
    calls, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while True:
            list(ex.map(lambda j: j[0](j[1], *j[2]), jobs))
            calls += 1
            el = time.perf_counter() - t0
            if el > budget_s or calls >= 5000:
                break
    return calls / el


def cpu_configs(synth, w_gate, w_down, threads, budget_s=1.2):
    """The CPU baseline (oracle/bq_oracle.c: the reference's scalar host loop,
    tools/mmq_test.cu:269-294, and the Q6_K formula of bruce.cu:4330-4345) on
    BASELINE configs 1, 3, 4 and 5, on `threads` host threads.  Config 4 times
    a slice of token rows and scales linearly to M (the loop is row-major in
    M); config 5 times one layer's four matrices and an 8192-row block of the
    131072-row lm_head and scales to 32 layers + the whole head."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    res = {}
    x8 = synth.gaussian(SEED + 20, (8, FF))
    q = {k: O.q8_rows(np.ascontiguousarray(x8[:, :k])) for k in (K, KO, FF)}
    g5, g6 = O.gemm_q5k_f32, O.gemm_q6k_f32
    a5 = lambda k, r=1: tuple(np.ascontiguousarray(t[:r]) for t in q[k])
    a6 = lambda k, r=1: tuple(np.ascontiguousarray(t[:r]) for t in q[k][:2])
    c1 = synth.quantize_q5k(synth.gaussian(SEED + 8, (K, K), 0.02))
    r = cpu_rate([(g5, c1, a5(K))], threads, budget_s)
    res["config1_3072x3072"] = {"GBps": round((c1.nbytes + q8_bytes(1, K) + 4 * K) * r / 1e9, 3)}
    for rows in (1, 8):
        r = cpu_rate([(g5, w_gate, a5(K, rows))], threads, budget_s)
        res[f"config3_rows{rows}"] = {"GBps": round((w_gate.nbytes + q8_bytes(rows, K) + 4 * rows * FF) * r / 1e9, 3),
                                      "ms_per_call": round(1e3 / r, 2)}
    S = 16 * threads                                   # token-row slice of the config 4 GEMM
    xs_ = synth.gaussian(SEED + 21, (S, K))
    r = cpu_rate([(g5, w_gate, O.q8_rows(xs_))], threads, budget_s)
    tops = 2.0 * S * FF * K * r / 1e12
    res["config4_gemm"] = {"tops": round(tops, 5), "slice_rows": S,
                           "ms_M2048": round(2.0 * 2048 * FF * K / (tops * 1e12) * 1e3, 1),
                           "ms_M8192": round(2.0 * 8192 * FF * K / (tops * 1e12) * 1e3, 1)}
    qkv = synth.quantize_q5k(synth.gaussian(SEED + 30, (NQKV, K), 0.02))
    wo = synth.quantize_q5k(synth.gaussian(SEED + 31, (K, KO), 0.02))
    head = synth.quantize_q6k(synth.gaussian(SEED + 32, (8192, K), 0.02))
    r_layer = cpu_rate([(g5, qkv, a5(K)), (g5, wo, a5(KO)), (g5, w_gate, a5(K)), (g5, w_gate, a5(K)),
                        (g6, w_down, a6(FF))], threads, budget_s)
    r_head = cpu_rate([(g6, head, a6(K))], threads, budget_s)
    tok_s = LAYERS / r_layer + (VOCAB // 8192) / r_head
    res["config5_whole_stack"] = {"ms_per_token": round(tok_s * 1e3, 1),
                                  "GBps": round(2942042112 / tok_s / 1e9, 3)}
    return res


LAYERS, KO, NQKV, VOCAB = 32, 4096, 5120, 131072


def whole_stack(B, bq, synth, torch, w_gate, w_up, w_down, sp, ptr, steps=20, warmup=3):
    """32 x [QKV Q5_K 5120x3072, O Q5_K 3072x4096, gate/up Q5_K
    2x(9216x3072), down Q6_K 3072x9216] + lm_head Q6_K 131072x3072 per token, every
    layer's weights in their own device memory (2.94 GB/token, > 10x the MALL).
    Synthetic weights: one seeded encoding per matrix shape, copied per layer; the
    lm_head is 16 copies of a seeded 8192-row Q6_K block.  Every GEMV is one
    bq_gemv_q8_fused launch (q8 quantization of the fp32 input inside)."""
    w_qkv = synth.quantize_q5k(synth.gaussian(SEED + 9, (NQKV, K), 0.02))
    w_o = synth.quantize_q5k(synth.gaussian(SEED + 10, (K, KO), 0.02))
    w_lm = synth.quantize_q6k(synth.gaussian(SEED + 11, (VOCAB // 16, K), 0.02))
    src = [torch.from_numpy(a).cuda() for a in (w_qkv, w_o, w_gate, w_up, w_down)]
    shapes = [(bq.TYPE_Q5_K, K, NQKV), (bq.TYPE_Q5_K, KO, K), (bq.TYPE_Q5_K, K, FF), (bq.TYPE_Q5_K, K, FF),
              (bq.TYPE_Q6_K, FF, K)]
    keep, ws = [], (bq.Weight * (5 * LAYERS))()
    for l in range(LAYERS):
        for j, (t, k, n) in enumerate(shapes):
            c = src[j].clone()
            keep.append(c)
            ws[5 * l + j] = bq.make_weight(c, t, k, n)
    lm = torch.from_numpy(w_lm).cuda().repeat(16, 1).contiguous()
    lmw = bq.make_weight(lm, bq.TYPE_Q6_K, K, VOCAB)
    x = torch.from_numpy(synth.gaussian(SEED + 12, (K,))).cuda()
    a = torch.from_numpy(synth.gaussian(SEED + 13, (KO,))).cuda()
    t = torch.from_numpy(synth.gaussian(SEED + 14, (FF,))).cuda()
    y0, y1 = torch.empty(VOCAB, device="cuda"), torch.empty(FF, device="cuda")
    xq = torch.empty(FF, dtype=torch.int8, device="cuda")
    xd = torch.empty(FF // 32, device="cuda")
    xs = torch.empty(FF // 32, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    out = (ctypes.c_double * 4)()
    r = B.bqb_stack(steps, warmup, LAYERS, ws, ctypes.byref(lmw), ptr(x), ptr(a), ptr(t), ptr(y0), ptr(y1),
                    ptr(xq), ptr(xd), ptr(xs), sp, out)
    if r != 0:
        raise RuntimeError(f"bqb_stack failed: {r}")
    ms = out[0] / steps
    # the same weights in the reference's dependent decode sequence, with the
    # q8 producers (gate norm, resid, silu*mul norm) between GEMVs, as the
    # library's captured decode step (bq_decode_graph_*, one graph per token)
    g = torch.Generator(device="cuda").manual_seed(SEED + 15)
    vec = lambda n: torch.rand(n, generator=g, device="cuda") * 0.5 + 0.25
    R = 8   # buffers for up to 8 token rows (the verify steps)
    fb = {"x": torch.randn((R, K), generator=g, device="cuda"), "aout": torch.randn((R, KO), generator=g, device="cuda"),
          "qkv": torch.empty((R, NQKV), device="cuda"), "proj": torch.empty((R, K), device="cuda"),
          "xalt": torch.empty(K, device="cuda"),
          "fg": torch.empty((R, FF), device="cuda"), "fu": torch.empty((R, FF), device="cuda"),
          "logits": torch.empty((R, VOCAB), device="cuda"), "alpha": vec(K), "alpha2": vec(K), "sgate": vec(KO),
          "sg": vec(FF), "su": vec(FF)}
    qb = [torch.empty(R * FF, dtype=torch.int8, device="cuda"), torch.empty(R * FF // 32, device="cuda"),
          torch.empty(R * FF // 32, dtype=torch.int32, device="cuda")]
    xq0, xd0, xs0 = bq.quantize_q8(fb["x"])
    qb[0][:R * K].copy_(xq0.view(-1)); qb[1][:R * K // 32].copy_(xd0.view(-1)); qb[2][:R * K // 32].copy_(xs0.view(-1))
    qout = (ctypes.c_void_p * 1)(fb["qkv"].data_ptr())
    blocks = (bq.DecodeBlock * (2 * LAYERS))()
    for l in range(LAYERS):
        a, f = blocks[2 * l], blocks[2 * l + 1]
        a.kind, a.alpha = bq.BLOCK_ATTN, fb["alpha"].data_ptr()
        a.qkv, a.n_qkv, a.qkv_out = ctypes.pointer(ws[5 * l]), 1, qout
        a.attn_out, a.attn_gate, a.sgate, a.n_attn = fb["aout"].data_ptr(), fb["qkv"].data_ptr(), fb["sgate"].data_ptr(), KO
        a.o = ctypes.pointer(ws[5 * l + 1])
        f.kind, f.alpha = bq.BLOCK_FFN, fb["alpha2"].data_ptr()
        f.gate, f.up, f.down = ctypes.pointer(ws[5 * l + 2]), ctypes.pointer(ws[5 * l + 3]), ctypes.pointer(ws[5 * l + 4])
        f.s_gate, f.s_up, f.n_ff = fb["sg"].data_ptr(), fb["su"].data_ptr(), FF
    blocks[2 * LAYERS - 1].norm_after = 1
    chain = {}
    # (rows, fold): the one-token step unfolded and folded, and the verify
    # steps over 2 / 4 / 8 token rows (one graph per row count)
    for rows, fold in ((1, 0), (1, 1), (1, 2), (2, 0), (4, 0), (8, 0)):
        stp = bq.DecodeStep()
        stp.n_blocks, stp.blocks, stp.n_embd, stp.fold, stp.rows = 2 * LAYERS, blocks, K, fold, rows
        stp.x, stp.xq, stp.xd, stp.xsum = fb["x"].data_ptr(), qb[0].data_ptr(), qb[1].data_ptr(), qb[2].data_ptr()
        stp.proj, stp.ffn_g, stp.ffn_u = fb["proj"].data_ptr(), fb["fg"].data_ptr(), fb["fu"].data_ptr()
        stp.head, stp.logits = ctypes.pointer(lmw), fb["logits"].data_ptr()
        stp.x_alt = fb["xalt"].data_ptr()
        dg = bq.DecodeGraph(stp)
        for _ in range(warmup):
            dg.launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            dg.launch()
        e1.record()
        torch.cuda.synchronize()
        chain[(rows, fold)] = e0.elapsed_time(e1) / steps
        dg.close()
    chain_ms, folded_ms, folded2_ms = chain[(1, 0)], chain[(1, 1)], chain[(1, 2)]
    verify = {f"rows{r}": {"ms_per_step": round(chain[(r, 0)], 4), "ms_per_token": round(chain[(r, 0)] / r, 4),
                           "step_vs_one_row": round(chain[(r, 0)] / chain_ms, 3)} for r in (2, 4, 8)}
    del fb, qb
    wbytes = LAYERS * sum(a.nbytes for a in (w_qkv, w_o, w_gate, w_up, w_down)) + lm.numel()
    act = LAYERS * (2 * (4 * K + q8_bytes(1, K)) + (4 * KO + q8_bytes(1, KO)) + (4 * FF + q8_bytes(1, FF))) \
        + 4 * K + q8_bytes(1, K)
    outb = 4 * (LAYERS * (NQKV + K + 2 * FF + K) + VOCAB)
    tot = wbytes + act + outb
    del keep, lm
    return {"config": "32 layers x (QKV 5120x3072, O 3072x4096, gate/up 2x9216x3072 Q5_K; down 3072x9216 "
                      "Q6_K) + lm_head Q6_K 131072x3072, batch 1, one HIP graph per token",
            "weight_bytes_per_token": wbytes, "bytes_per_token": tot, "ms_per_token": round(ms, 4),
            "GBps": round(gbs(tot, ms), 1), "hbm_frac": round(gbs(tot, ms) / HBM_PEAK_GBS, 4),
            "launches_per_token": 4 * LAYERS + 1,
            "decode_chain": {"what": "the reference's dependent decode sequence per layer through the library's "
                                     "captured decode step (bq_decode_graph, fold = 0): QKV GEMV, gate norm -> q8, "
                                     "O GEMV, resid -> q8, gate+up GEMV, silu*mul norm -> q8, down GEMV, resid -> q8; "
                                     "final norm -> q8, lm_head (attention excluded; aout a fixed input)",
                             "ms_per_token": round(chain_ms, 4), "GBps": round(gbs(tot, chain_ms), 1),
                             "launches_per_token": 8 * LAYERS + 1},
            "decode_chain_folded": {"what": "the same step with fold = 1: the gate norm inside the O GEMV, the "
                                            "silu*mul in the gate+up epilogue (bq_gate_up_silu) and its norm -> q8 "
                                            "inside the down GEMV (bq_gemv_norm_fused)",
                                    "ms_per_token": round(folded_ms, 4), "GBps": round(gbs(tot, folded_ms), 1),
                                    "launches_per_token": 6 * LAYERS + 1},
            "decode_chain_folded2": {"what": "fold = 2: as fold = 1, and each FFN block's resid -> q8 inside the "
                                             "next layer's QKV GEMV (bq_gemv_norm_fused with BQ_OP_RESID), the first "
                                             "layer's loop-start norm inside its QKV GEMV (BQ_OP_ADD)",
                                     "ms_per_token": round(folded2_ms, 4), "GBps": round(gbs(tot, folded2_ms), 1),
                                     "launches_per_token": 5 * LAYERS + 1},
            "decode_chain_verify": {"what": "the same step (fold = 0) over 2 / 4 / 8 token rows, the speculative-"
                                            "verify step with every row's logits (forward_batch_impl with "
                                            "all_logits, bruce.cu:7610-7843; one captured graph per row count as "
                                            "capture_verify_graphs, :7877-7900); ms_per_token = step / rows",
                                    **verify}}


def prompt_chunk(bq, synth, torch, w_gate, w_up, w_down, steps=10, warmup=2):
    """A prompt chunk through the library's step (bq_decode_graph with rows = M
    > 8): the reference's forward_batch_impl as bruce_prefill_chunk calls it
    (bruce.cu:8274-8291, :7610-7843), here 4 layers of config 5's shapes (QKV
    one Q5_K 5120x3072, O Q5_K 3072x4096, gate/up Q5_K 9216x3072 with their
    W144 repacks; down Q6_K 3072x9216 with its W160 repack), each layer its
    own weight copy, no logits (a chunk that is not the prompt's last), at M =
    512 (the reference's largest chunk, MBUF) and 2048 (config 4's M).  Per
    layer: the whole step (row producers, xdh fills, the prefill GEMMs and
    their K-split sums; attention excluded, aout a fixed input) against the
    same GEMM calls alone (bq_gemm_b / bq_gemm_b_fused, eager, events)."""
    NL = 4
    w_qkv = synth.quantize_q5k(synth.gaussian(SEED + 9, (NQKV, K), 0.02))
    w_o = synth.quantize_q5k(synth.gaussian(SEED + 10, (K, KO), 0.02))
    keep, ws = [], []
    for l in range(NL):
        lw = []
        for a, kk, n in ((w_qkv, K, NQKV), (w_o, KO, K), (w_gate, K, FF), (w_up, K, FF)):
            g = torch.from_numpy(a).cuda()
            rep, dm = bq.repack_q5k(g, kk, n)
            keep += [g, rep, dm]
            lw.append(bq.make_weight(g, bq.TYPE_Q5_K, kk, n, rep=rep, rep_min=dm))
        g = torch.from_numpy(w_down).cuda()
        rep = bq.repack_q6k(g, FF, K)
        keep += [g, rep]
        lw.append(bq.make_weight(g, bq.TYPE_Q6_K, FF, K, rep=rep))
        ws.append(lw)
    gen = torch.Generator(device="cuda").manual_seed(SEED + 16)
    vec = lambda n: torch.rand(n, generator=gen, device="cuda") * 0.5 + 0.25
    alpha, alpha2, sgate, sg, su = vec(K), vec(K), vec(KO), vec(FF), vec(FF)
    res = {}
    for M in (512, 2048):
        x = torch.randn((M, K), generator=gen, device="cuda")
        aout = torch.randn((M, KO), generator=gen, device="cuda")
        qkv, proj = torch.empty((M, NQKV), device="cuda"), torch.empty((M, K), device="cuda")
        fg, fu = torch.empty((M, FF), device="cuda"), torch.empty((M, FF), device="cuda")
        xq = torch.empty(M * FF, dtype=torch.int8, device="cuda")
        xd = torch.empty(M * FF // 32, device="cuda")
        xs = torch.empty(M * FF // 32, dtype=torch.int32, device="cuda")
        xdh = torch.empty(M * FF // 32, dtype=torch.int16, device="cuda")
        q = bq.quantize_q8(x)
        xq[:M * K].copy_(q[0].view(-1)); xd[:M * K // 32].copy_(q[1].view(-1)); xs[:M * K // 32].copy_(q[2].view(-1))
        wb = max(bq.workspace_bytes(M, kk, n) for kk, n in ((K, NQKV), (KO, K), (K, 2 * FF), (FF, K)))
        work = torch.empty(max(wb, 16) // 4, device="cuda")
        qout = (ctypes.c_void_p * 1)(qkv.data_ptr())
        blocks = (bq.DecodeBlock * (2 * NL))()
        for l in range(NL):
            a, f = blocks[2 * l], blocks[2 * l + 1]
            a.kind, a.alpha = bq.BLOCK_ATTN, alpha.data_ptr()
            a.qkv, a.n_qkv, a.qkv_out = ctypes.pointer(ws[l][0]), 1, qout
            a.attn_out, a.attn_gate, a.sgate, a.n_attn = aout.data_ptr(), qkv.data_ptr(), sgate.data_ptr(), KO
            a.o = ctypes.pointer(ws[l][1])
            f.kind, f.alpha = bq.BLOCK_FFN, alpha2.data_ptr()
            f.gate, f.up, f.down = ctypes.pointer(ws[l][2]), ctypes.pointer(ws[l][3]), ctypes.pointer(ws[l][4])
            f.s_gate, f.s_up, f.n_ff = sg.data_ptr(), su.data_ptr(), FF
        blocks[2 * NL - 1].norm_after = 1
        stp = bq.DecodeStep()
        stp.n_blocks, stp.blocks, stp.n_embd, stp.fold, stp.rows = 2 * NL, blocks, K, 0, M
        stp.x, stp.xq, stp.xd, stp.xsum = x.data_ptr(), xq.data_ptr(), xd.data_ptr(), xs.data_ptr()
        stp.proj, stp.ffn_g, stp.ffn_u = proj.data_ptr(), fg.data_ptr(), fu.data_ptr()
        stp.xdh, stp.work, stp.work_bytes = xdh.data_ptr(), work.data_ptr(), work.numel() * 4
        dg = bq.DecodeGraph(stp)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(warmup):
            dg.launch()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            dg.launch()
        e1.record()
        torch.cuda.synchronize()
        step_ms = e0.elapsed_time(e1) / steps / NL
        dg.close()

        def gemms():
            for l in range(NL):
                bq.gemm_b(qkv, ws[l][0], M, xq, xd, xs, xdh, work)
                bq.gemm_b(proj, ws[l][1], M, xq, xd, xs, xdh, work)
                bq.gemm_b_fused([fg, fu], [ws[l][2], ws[l][3]], M, xq, xd, xs, xdh, work)
                bq.gemm_b(proj, ws[l][4], M, xq, xd, xs, xdh, work)
        for _ in range(warmup):
            gemms()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            gemms()
        e1.record()
        torch.cuda.synchronize()
        gemm_ms = e0.elapsed_time(e1) / steps / NL
        ops = 2 * M * (K * (NQKV + 2 * FF) + KO * K + FF * K)
        res[f"M{M}"] = {"ms_per_layer": round(step_ms, 4), "gemms_ms_per_layer": round(gemm_ms, 4),
                        "rest_ms_per_layer": round(step_ms - gemm_ms, 4),
                        "tops": round(ops / step_ms / 1e9, 1), "gemm_tops": round(ops / gemm_ms / 1e9, 1),
                        "tokens_per_s_32_layers": round(M / (32 * step_ms / 1e3), 1)}
        del x, aout, qkv, proj, fg, fu, xq, xd, xs, xdh, work, dg
    del keep
    return {"what": " ".join(prompt_chunk.__doc__.split()), **res}


def q8s_head(B, bq, torch, sp, ptr, steps=50):
    """Q8_0 logits head (bruce.cu:4400-4449): Q8S 131072 x K GEMV, rows 1 and 8,
    at the BASELINE hidden size (K = 3072) and the reference model's (K = 2560).
    Weights: device-generated N(0, 0.02) bf16, converted by bq_quantize_q8s;
    two copies rotate so the 256 MB last-level cache cannot serve them."""
    N = 131072
    out = (ctypes.c_double * 4)()
    res = {}
    g = torch.Generator(device="cuda").manual_seed(SEED + 9)
    for K in (3072, 2560):
        copies = []
        for _ in range(2):
            wb = (torch.randn((N, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
            copies.append(bq.quantize_q8s(wb, K, N))
            del wb
        wsa = (ctypes.c_void_p * 2)(*[c.data_ptr() for c in copies])
        x = torch.randn((8, K), generator=g, device="cuda")
        xq, xd, _ = bq.quantize_q8(x)
        rs = torch.rand(N, generator=g, device="cuda") + 0.5
        y = torch.empty((8, N), device="cuda")
        res_k = {}
        for rows in (1, 8):
            r = B.bqb_q8s(steps, 5, 2, wsa, K, N, rows, ptr(xq), ptr(xd), ptr(rs), ptr(y), sp, out)
            if r != 0:
                raise RuntimeError(f"bqb_q8s failed: {r}")
            kms = out[1] / steps
            nbytes = copies[0].numel() + rows * (K + K // 32 * 4) + 4 * N + 4 * rows * N
            res_k[f"rows{rows}"] = {"us": round(kms * 1e3, 2), "GBps": round(gbs(nbytes, kms), 1),
                                    "hbm_frac": round(gbs(nbytes, kms) / HBM_PEAK_GBS, 4)}
        res[f"K{K}"] = dict(res_k, weight_bytes=copies[0].numel())
        del copies, x, xq, xd, rs, y
        torch.cuda.empty_cache()
    return {"config": "Q8_0 logits head 131072 x K (Q8S, 272 B / 256 values) x q8 rows, fp32 out * rs",
            "kernel": "k_gemv_q8s", **res}


def q8_producers(B, torch, sp, ptr, steps=100):
    """The norm kernels that emit q8 activations (bruce.cu:541-641): each op at
    its decode shape (1 row: launch/latency-bound) and as a 2048-row prompt
    batch (HBM-bound: bytes = inputs + fp32 out + q8 out)."""
    out_t = (ctypes.c_double * 4)()
    # op id, name, n, fp32 row arrays read, per-column vectors read, fp32 out written
    ops = [(0, "norm", 3072, 1, 0, 1), (1, "add_norm", 3072, 2, 0, 1), (2, "resid", 3072, 2, 1, 1),
           (3, "gate_norm", 4096, 2, 1, 1), (4, "silu_mul_norm", 9216, 2, 2, 0)]
    g = torch.Generator(device="cuda").manual_seed(SEED + 10)
    res = {}
    for op, name, n, nin, nvec, nout in ops:
        r_ = {}
        for rows in (1, 2048):
            bufs = [torch.randn((rows, n), generator=g, device="cuda") for _ in range(nin)]
            vecs = [torch.rand(n, generator=g, device="cuda") + 0.5 for _ in range(nvec)]
            outb = torch.empty((rows, n), device="cuda") if op in (0, 3) else None
            xq = torch.empty((rows, n), dtype=torch.int8, device="cuda")
            xd = torch.empty((rows, n // 32), device="cuda")
            xs = torch.empty((rows, n // 32), dtype=torch.int32, device="cuda")
            ab = bufs + vecs
            a = ab[0]
            b = ab[1] if len(ab) > 1 else None
            c = ab[2] if len(ab) > 2 else None
            d = ab[3] if len(ab) > 3 else None
            rc = B.bqb_norm(op, steps, 10, None if outb is None else ptr(outb), ptr(a),
                            None if b is None else ptr(b), None if c is None else ptr(c),
                            None if d is None else ptr(d), rows, n, ptr(xq), ptr(xd), ptr(xs), sp, out_t)
            if rc != 0:
                raise RuntimeError(f"bqb_norm({name}) failed: {rc}")
            kms = out_t[1] / steps
            nbytes = rows * n * 4 * (nin + nout) + nvec * n * 4 + rows * (n + n // 32 * 8)
            r_[f"rows{rows}"] = {"us": round(kms * 1e3, 2), "GBps": round(gbs(nbytes, kms), 1)}
            del bufs, vecs, outb, xq, xd, xs
        res[f"{name}_n{n}"] = r_
    return {"kernel": "k_norm_q8<op>", **res}


def gguf_load(bq, torch):
    """GGUF streaming loader (bq_gguf_load): the 131072 x 3072 Q6_K lm_head
    (330 MB) from a page-cached file through the pinned slots to HBM, plus its
    W160 repack.  Random blocks with finite scales; the file lives in /tmp only
    for this measurement."""
    import tempfile
    import time
    N, K = 131072, 3072
    rng = np.random.default_rng(SEED + 11)
    blocks = rng.integers(0, 256, size=(N, K // 256, 210), dtype=np.uint8)
    blocks[..., 208:210] = np.full((N, K // 256), 0.01, np.float16).view(np.uint8).reshape(N, K // 256, 2)
    payload = blocks.reshape(-1)
    del blocks
    import struct
    name = b"output.weight"
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", len(name)) + name
    head += struct.pack("<I", 2) + struct.pack("<QQ", K, N) + struct.pack("<IQ", 14, 0)
    head += b"\0" * ((-len(head)) % 32)
    fd, path = tempfile.mkstemp(suffix=".gguf", dir="/tmp")
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(head)
            payload.tofile(f)
        raw = torch.empty(payload.size, dtype=torch.uint8, device="cuda")
        w160 = torch.empty(bq.load().bq_repack_q6k_bytes(K, N), dtype=torch.uint8, device="cuda")
        res = {}
        with bq.Gguf(path) as g:
            g.load(0, raw, w160)        # allocates the staging slots; warms the page cache
            torch.cuda.synchronize()
            times = []
            for _ in range(3):
                t0 = time.perf_counter()
                g.load(0, raw, w160)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
        sec = min(times)
        res = {"tensor": "Q6_K 131072x3072 lm_head + W160 repack", "bytes": int(payload.size),
               "ms": round(sec * 1e3, 2), "GBps": round(payload.size / sec / 1e9, 2),
               "source": "page-cached file, pread into 2 x 64 MiB pinned slots, hipMemcpyAsync"}
        del raw, w160
        return res
    finally:
        os.unlink(path)


def mfma_ceiling(B, torch, sp):
    """Dense int8 MFMA throughput measured on the box (k_mfma_peak in
    bq_bench.hip: 8 waves per CU, four independent v_mfma_i32_32x32x32_i8
    chains per wave, no memory traffic), beside the published 5.0 POPS."""
    out = (ctypes.c_double * 4)()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    props = torch.cuda.get_device_properties(0)
    blocks = 2 * props.multi_processor_count
    r = B.bqb_mfma_peak(blocks, 20000, ctypes.c_void_p(sink.data_ptr()), sp, out)
    if r != 0:
        raise RuntimeError("bqb_mfma_peak failed")
    tops = out[1] / (out[0] * 1e-3) / 1e12
    return {"kernel": "k_mfma_peak", "tops": round(tops, 1), "frac_of_published": round(tops / INT8_PEAK_TOPS, 4),
            "cus": props.multi_processor_count}


def stream_ceiling(B, torch, sp, sizes=(6504192, 19464192, 23224320, 39018240, 330301440)):
    """HBM streaming-read ceiling per launch size, the bound a GEMV of that
    many bytes can reach in one launch: the faster of two read-only kernels in
    bq_bench.hip (k_stream: one 16 KB chunk per workgroup; k_stream_gs: a
    grid of 4 workgroups per CU looping over 16 KB chunks), 16-byte loads of
    every byte once, buffers rotated past the last-level cache.  Sizes:
    config 1, config 3, the down projection, the fused gate+up and the
    lm_head launches."""
    res = {}
    out = (ctypes.c_double * 4)()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for nbytes in sizes:
        nb = max(2, math.ceil(3 * LLC_BYTES / nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nb)]
        arr = (ctypes.c_void_p * nb)(*[b.data_ptr() for b in bufs])
        steps = 200 if nbytes < 100e6 else 40
        per = {}
        for pattern, name in ((0, "k_stream"), (1, "k_stream_gs")):
            # warm-up: one pass over every buffer (a fresh buffer's first touch is slower)
            r = B.bqb_stream(pattern, steps, nb + 10, nb, arr, nbytes, ctypes.c_void_p(sink.data_ptr()), sp, out)
            if r != 0:
                raise RuntimeError("bqb_stream failed")
            per[name] = out[0] / steps * 1e3
        best = min(per, key=per.get)
        us = per[best]
        res[f"{nbytes / 1e6:.1f}MB"] = {"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
                                        "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "kernel": best,
                                        "us_per_kernel": {k: round(v, 3) for k, v in per.items()}}
        del bufs
    return res


def issue_probes(B, torch, sp):
    """Issue rates of the instructions the GEMV / GEMM kernels are built from
    (k_inst_rate in bq_bench.hip: 8 waves per CU, 4 independent chains per
    wave, no memory traffic), as wave instructions per second per SIMD and
    relative to v_mfma_i32_32x32x32_i8, and the dispatch-event duration of an
    empty kernel (k_empty, 1024 x 256 threads), the fixed cost of a launch."""
    out = (ctypes.c_double * 4)()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    blocks = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    names = ["v_mfma_i32_32x32x32_i8", "v_mfma_i32_32x32x16_i8", "v_mfma_f32_32x32x16_f16",
             "v_mfma_f32_32x32x1_2b_f32", "v_mfma_i32_4x4x4_16b_i8", "v_fma_f32", "v_cvt_f32_i32 + v_add_f32"]
    rates = {}
    for w, name in enumerate(names):
        if B.bqb_inst_rate(w, blocks, 20000, ctypes.c_void_p(sink.data_ptr()), sp, out) != 0:
            raise RuntimeError("bqb_inst_rate failed")
        rates[name] = out[1] / (out[0] * 1e-3)
    base = rates[names[0]]
    res = {"instructions_per_us_per_simd": {k: round(v / 1e6, 2) for k, v in rates.items()},
           "time_relative_to_i8_32x32x32": {k: round(base / v, 3) for k, v in rates.items()}}
    if B.bqb_empty(200, 1024, ctypes.c_void_p(sink.data_ptr()), sp, out) != 0:
        raise RuntimeError("bqb_empty failed")
    res["empty_kernel_us"] = {"back_to_back": round(out[0] / 200 * 1e3, 3),
                              "after_sync": round(out[1] / 200 * 1e3, 3)}
    return res


def gemm_section(B, bq, synth, torch, g_gate, g_down, sp, ptr, out):
    """Config 4 (Q5_K 9216 x 3072 GEMM at M = 2048 / 512 / 8192, both tiers),
    the prompt-batch tail through bq_gemm_b and the Q6_K GEMM (down projection
    over W160, M = 2048)."""
    gemm = {}
    gw144, gdm = bq.repack_q5k(g_gate, K, FF)
    for M in (2048, 512, 8192):
        xm = torch.from_numpy(synth.gaussian(SEED + 6, (M, K))).cuda()
        mq, md, ms_, mh = bq.quantize_q8(xm, with_xdh=True)
        ym = torch.empty((M, FF), device="cuda")
        res = {}
        # the caller's K-split workspace, sized by bq_gemm_workspace_bytes as
        # an engine caller allocates it; the call time runs from the GEMM kernel's
        # start to the end of the call, so a leftover-tile sum is included
        work = bq.workspace(M, K, FF)
        wptr, wbytes = (ptr(work), work.numel() * 4) if work is not None else (None, 0)
        for name, w in (("w144", bq.make_weight(g_gate, bq.TYPE_Q5_K, K, FF, rep=gw144, rep_min=gdm)),
                        ("raw", bq.make_weight(g_gate, bq.TYPE_Q5_K, K, FF))):
            gsteps = 20 if M == 8192 else 50
            r = B.bqb_gemm(gsteps, 5, ctypes.byref(w), M, ptr(mq), ptr(md), ptr(ms_), ptr(mh), ptr(ym), wptr,
                           wbytes, sp, out)
            if r != 0:
                raise RuntimeError(f"bqb_gemm failed: {r}")
            cms, kms = out[2] / gsteps, out[1] / gsteps
            tops = 2.0 * M * FF * K / (cms * 1e-3) / 1e12
            res[name] = {"ms": round(cms, 4), "kernel_ms": round(kms, 4), "tops": round(tops, 1),
                         "frac": round(tops / INT8_PEAK_TOPS, 4)}
        del work
        # bytes of one launch (weights as streamed: W144 + Dm or GGUF; q8 X
        # with xd, xsum, xdh; fp32 Y) over the time, against 8 TB/s: the GEMM
        # is near the int8 ridge at M = 512
        xbytes = M * K + M * (K // 32) * 10
        for name, wb in (("w144", gw144.nbytes + gdm.nbytes), ("raw", g_gate.nbytes)):
            res[name]["hbm_frac"] = round((wb + xbytes + 4 * M * FF) / (res[name]["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        gemm[f"M{M}"] = res
        del xm, mq, md, ms_, mh, ym
    # prompt-batch tail (rows 9..95, bq_gemm_b: 8-row GEMV chunks or the
    # MMQ tile) and the Q6_K GEMM (down projection over W160, M = 2048)
    def ev_time(fn, n=20):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n
    wp = bq.make_weight(g_gate, bq.TYPE_Q5_K, K, FF, rep=gw144, rep_min=gdm)
    xt = torch.from_numpy(synth.gaussian(SEED + 9, (96, K))).cuda()
    tq, td_, ts_, th = bq.quantize_q8(xt, with_xdh=True)
    yt = torch.empty((96, FF), device="cuda")
    tail = {}
    tw = torch.empty(8 << 20, device="cuda")      # K-split workspace: 32 MiB covers any split
    for rows in (16, 32, 48, 64, 95):
        tms = ev_time(lambda: bq.gemm_b(yt, wp, rows, tq, td_, ts_, th, work=tw))
        tail[f"rows{rows}"] = {"us": round(tms * 1e3, 1),
                               "tops": round(2.0 * rows * FF * K / (tms * 1e-3) / 1e12, 1)}
    del xt, tq, td_, ts_, th, yt
    w160 = bq.repack_q6k(g_down, FF, K)
    wd6 = bq.make_weight(g_down, bq.TYPE_Q6_K, FF, K, rep=w160)
    x6 = torch.from_numpy(synth.gaussian(SEED + 10, (2048, FF))).cuda()
    q6q, q6d, _ = bq.quantize_q8(x6)
    y6 = torch.empty((2048, K), device="cuda")
    q6ms = ev_time(lambda: bq.gemm_q6k_mma(y6, wd6, 2048, q6q, q6d, work=None), n=10)
    q6tops = 2.0 * 2048 * K * FF / (q6ms * 1e-3) / 1e12
    del w160, x6, q6q, q6d, y6
    g = gemm["M2048"]["w144"]
    gemm_obj = {
        "mfma_int8_ceiling": mfma_ceiling(B, torch, sp),
        "config": "prefill GEMM Q5_K 9216x3072 (W144 repack, fp16 min term), M=2048 q8 tokens, fp32 out",
        "value": g["tops"], "unit": "TOPS", "ms": g["ms"],
        "roofline": {"bound": "mfma", "achieved": g["tops"], "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": g["frac"], "traffic": traffic_for("mmq_w144_M2048"),
                     "kernel": "k_mmq_w144", "ops_per_launch": 2 * 2048 * FF * K},
        "shapes": gemm,
        "tail_rows_bq_gemm_b": {"what": "Q5_K 9216x3072 W144, bq_gemm_b: the MMQ tile (32-token at these rows, K-split) "
                                        "above 8 rows", **tail},
        "q6k_down_M2048": {"what": "Q6_K 3072x9216 over W160 (k_mmq_q6k_dma), M=2048", "ms": round(q6ms, 4),
                           "tops": round(q6tops, 1), "frac": round(q6tops / INT8_PEAK_TOPS, 4)},
    }
    return gemm_obj


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode FFN step (for kernel traces); implies --no-cpu")
    ap.add_argument("--mfma-only", action="store_true",
                    help="only the dense int8 MFMA throughput probe; prints its JSON object")
    ap.add_argument("--stream-only", action="store_true",
                    help="only the HBM streaming-read ceilings per launch size; prints their JSON object")
    ap.add_argument("--probe-only", action="store_true",
                    help="only the instruction issue-rate probes and the empty-kernel launch cost; "
                         "prints their JSON object")
    ap.add_argument("--stack-only", action="store_true",
                    help="only config 5 (the whole-stack decode and the decode-step chains); prints its JSON object")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip config 5 (the whole-stack decode and the decode-step graphs), e.g. for counter runs")
    ap.add_argument("--chunk-only", action="store_true",
                    help="only the prompt-chunk step (bq_decode_graph over 512 / 2048 rows); prints its JSON object")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the prefill GEMMs of config 4 and the Q6_K GEMM (for counter profiles); "
                         "prints their JSON object")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the k-quant matmul path has no multi-GPU mode in this "
              "build (it would shard weight rows N across GPUs); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import bq
    import synth

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    bq.load()
    B = ctypes.CDLL(os.path.join(ROOT, "bruce-engine_amd", "libbq_bench.so"))
    P, I = ctypes.c_void_p, ctypes.c_int
    WP = ctypes.POINTER(bq.Weight)
    D4 = ctypes.c_double * 4
    B.bqb_decode_ffn.argtypes = [I, I, I, I, WP, WP, WP, P, P, P, P, P, P, P, P, P, P, P, P, P]
    B.bqb_gemm.argtypes = [I, I, WP, I, P, P, P, P, P, P, ctypes.c_size_t, P, P]
    B.bqb_gemv_rows.argtypes = [I, I, I, WP, I, P, P, P, P, P, P]
    B.bqb_stream.argtypes = [I, I, I, I, P, ctypes.c_size_t, P, P, P]
    B.bqb_inst_rate.argtypes = [I, I, I, P, P, P]
    B.bqb_empty.argtypes = [I, I, P, P, P]
    B.bqb_mfma_peak.argtypes = [I, I, P, P, P]
    B.bqb_stack.argtypes = [I, I, I, WP, WP, P, P, P, P, P, P, P, P, P, P]
    B.bqb_q8s.argtypes = [I, I, I, P, I, I, I, P, P, P, P, P, P]
    B.bqb_norm.argtypes = [I, I, I, P, P, P, P, P, I, I, P, P, P, P, P]
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())

    # ---------------------------------------------------------------- data
    w_gate = synth.quantize_q5k(synth.gaussian(SEED + 1, (FF, K), 0.02))
    w_up = synth.quantize_q5k(synth.gaussian(SEED + 2, (FF, K), 0.02))
    w_down = synth.quantize_q6k(synth.gaussian(SEED + 3, (K, FF), 0.02))
    x = synth.gaussian(SEED + 4, (1, K))
    t = synth.gaussian(SEED + 5, (1, FF))
    wbytes = w_gate.nbytes + w_up.nbytes + w_down.nbytes
    nsets = max(2, math.ceil(3 * LLC_BYTES / wbytes))
    g_gate = torch.from_numpy(w_gate).cuda()
    g_up = torch.from_numpy(w_up).cuda()
    g_down = torch.from_numpy(w_down).cuda()
    keep = []
    gates, ups, downs = (bq.Weight * nsets)(), (bq.Weight * nsets)(), (bq.Weight * nsets)()
    for s in range(nsets):
        a, b, c = g_gate.clone(), g_up.clone(), g_down.clone()
        keep += [a, b, c]
        gates[s] = bq.make_weight(a, bq.TYPE_Q5_K, K, FF)
        ups[s] = bq.make_weight(b, bq.TYPE_Q5_K, K, FF)
        downs[s] = bq.make_weight(c, bq.TYPE_Q6_K, FF, K)
    dx, dt = torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda()
    xq = torch.empty((1, K), dtype=torch.int8, device="cuda")
    xd = torch.empty((1, K // 32), device="cuda")
    xs = torch.empty((1, K // 32), dtype=torch.int32, device="cuda")
    tq = torch.empty((1, FF), dtype=torch.int8, device="cuda")
    td = torch.empty((1, FF // 32), device="cuda")
    ts = torch.empty((1, FF // 32), dtype=torch.int32, device="cuda")
    yg, yu, yd = (torch.empty(FF, device="cuda"), torch.empty(FF, device="cuda"),
                  torch.empty(K, device="cuda"))
    # a plain 64 MiB device copy: the reference point that scales rocprofv3's
    # FETCH_SIZE / WRITE_SIZE counters to bytes (profiles/traffic.json)
    calib_src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    calib_dst = torch.empty_like(calib_src)
    calib_dst.copy_(calib_src)
    del calib_src, calib_dst
    torch.cuda.synchronize()

    out = D4()
    if args.mfma_only:
        print(json.dumps({"mfma_int8_ceiling": mfma_ceiling(B, torch, sp)}), flush=True)
        return
    if args.stream_only:
        print(json.dumps({"hbm_read_ceiling": stream_ceiling(B, torch, sp)}), flush=True)
        return
    if args.probe_only:
        print(json.dumps({"issue_probes": issue_probes(B, torch, sp)}), flush=True)
        return
    if args.gemm_only:
        print(json.dumps({"gemm": gemm_section(B, bq, synth, torch, g_gate, g_down, sp, ptr, out)}), flush=True)
        return
    if args.chunk_only:
        print(json.dumps({"prompt_chunk": prompt_chunk(bq, synth, torch, w_gate, w_up, w_down)}), flush=True)
        return
    if args.stack_only:
        print(json.dumps({"config5_whole_stack": whole_stack(B, bq, synth, torch, w_gate, w_up, w_down, sp, ptr)}),
              flush=True)
        return

    # ---------------------------------------------------------------- decode FFN step
    step_bytes = wbytes + q8_bytes(1, K) + q8_bytes(1, FF) + 4 * (2 * FF + K)

    def decode(mode, warmup):
        r = B.bqb_decode_ffn(mode, args.steps, warmup, nsets, gates, ups, downs, ptr(dx), ptr(dt), ptr(xq),
                             ptr(xd), ptr(xs), ptr(tq), ptr(td), ptr(ts), ptr(yg), ptr(yu), ptr(yd), sp, out)
        if r != 0:
            raise RuntimeError(f"bqb_decode_ffn(mode {mode}) failed: {r} {bq.strerror(r)}")
        return out[0], out[1] / args.steps, out[2] / args.steps

    # headline: K steps of the fused form (bq_gemv_q8_fused: each GEMV quantizes
    # its fp32 input), replayed from HIP graphs -- the timed region
    total_ms, _, _ = decode(2, args.warmup)
    # second timed region, same K steps launched directly: the GEMV kernels'
    # own durations from dispatch start/end events
    _, gu_ms, dn_ms = decode(3, 0)
    value = gbs(step_bytes * args.steps, total_ms)
    # the same step as the reference issues it: quantize, GEMV, quantize, GEMV
    un_ms, un_gu, un_dn = decode(0, args.warmup)
    _, un_gu, un_dn = decode(1, 0)
    unfused = {"ms_per_step": round(un_ms / args.steps, 5), "GBps": round(gbs(step_bytes * args.steps, un_ms), 1),
               "gateup_us": round(un_gu * 1e3, 3), "down_us": round(un_dn * 1e3, 3)}
    # fused gate+up launch: fp32 x in, q8 x out, both weight matrices, two fp32 outputs
    gu_bytes = w_gate.nbytes + w_up.nbytes + 4 * K + q8_bytes(1, K) + 4 * 2 * FF
    dn_bytes = w_down.nbytes + 4 * FF + q8_bytes(1, FF) + 4 * K
    achieved = gbs(gu_bytes, gu_ms)

    gemm_obj, rows_res, c1_obj, stack_obj, q8s_obj, norm_obj, load_obj = None, None, None, None, None, None, None
    ceil_obj, probe_obj, chunk_obj = None, None, None
    if not args.decode_only:
        gemm_obj = gemm_section(B, bq, synth, torch, g_gate, g_down, sp, ptr, out)
        ceil_obj = stream_ceiling(B, torch, sp)
        probe_obj = issue_probes(B, torch, sp)

        # ---------------------------------------------------------------- config 3 / config 1 GEMV
        rows_res = {}
        xr = torch.from_numpy(synth.gaussian(SEED + 7, (8, K))).cuda()
        rq, rd, rs = bq.quantize_q8(xr)
        yr = torch.empty((8, FF), device="cuda")
        # config 3 streams one 19.5 MB matrix: rotate >= 3 x the last-level
        # cache of copies (the gate sets plus extra device copies)
        n3 = max(nsets, math.ceil(3 * LLC_BYTES / w_gate.nbytes))
        c3g = [g_gate.clone() for _ in range(n3 - nsets)]
        gsets = (bq.Weight * n3)(*([gates[s] for s in range(nsets)] +
                                   [bq.make_weight(a, bq.TYPE_Q5_K, K, FF) for a in c3g]))
        for rows in (1, 2, 4, 8):
            # warm-up: one pass over every copy (the first touch of a fresh
            # copy is slower), then the timed launches
            r = B.bqb_gemv_rows(100, n3 + 10, n3, gsets, rows, ptr(rq), ptr(rd), ptr(rs), ptr(yr), sp, out)
            kms = out[1] / 100
            rows_res[f"rows{rows}"] = {"us": round(kms * 1e3, 2),
                                       "GBps": round(gbs(w_gate.nbytes + q8_bytes(rows, K) + 4 * rows * FF, kms), 1)}
        del c3g
        c1 = synth.quantize_q5k(synth.gaussian(SEED + 8, (K, K), 0.02))
        n1 = max(2, math.ceil(3 * LLC_BYTES / c1.nbytes))
        c1g = [torch.from_numpy(c1).cuda() for _ in range(n1)]
        c1w = (bq.Weight * n1)(*[bq.make_weight(a, bq.TYPE_Q5_K, K, K) for a in c1g])
        r = B.bqb_gemv_rows(200, n1 + 10, n1, c1w, 1, ptr(rq), ptr(rd), ptr(rs), ptr(yr), sp, out)
        c1ms = out[1] / 200
        del c1g
        c1_obj = {"us": round(c1ms * 1e3, 2), "GBps": round(gbs(c1.nbytes + q8_bytes(1, K) + 4 * K, c1ms), 1)}

        # ------------------------------------------------------------ config 5: whole-stack token
        if not args.no_stack:
            stack_obj = whole_stack(B, bq, synth, torch, w_gate, w_up, w_down, sp, ptr)

        # ------------------------------------------------------------ prompt chunk (prefill step)
        chunk_obj = prompt_chunk(bq, synth, torch, w_gate, w_up, w_down)

        # ------------------------------------------------------------ Q8_0 logits head
        q8s_obj = q8s_head(B, bq, torch, sp, ptr)

        # ------------------------------------------------------------ q8 producers (norm + quantize)
        norm_obj = q8_producers(B, torch, sp, ptr)

        # ------------------------------------------------------------ GGUF streaming load + repack
        load_obj = gguf_load(bq, torch)

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not (args.no_cpu or args.decode_only):
        ncpu = min(16, os.cpu_count() or 1)  # the GPU box's CPU share is 16 cores
        steps1, el1 = cpu_baseline(w_gate, w_up, w_down, x, t, 1, budget_s=8.0)
        stepsn, eln = cpu_baseline(w_gate, w_up, w_down, x, t, ncpu, budget_s=8.0)
        cpu = {"value": round(gbs(step_bytes * stepsn, eln * 1e3), 3), "unit": "GB/s", "cores": ncpu,
               "kind": "port",
               "sample": f"{stepsn} full decode FFN steps (gate+up Q5_K + down Q6_K, batch 1, same inputs) "
                         f"through the scalar fp32 restatement of the reference host loop "
                         f"(tools/mmq_test.cu:269-294), output rows split over {ncpu} threads",
               "seconds": round(eln, 2), "host_threads_available": os.cpu_count(),
               "single_thread": {"value": round(gbs(step_bytes * steps1, el1 * 1e3), 3), "unit": "GB/s",
                                 "steps": steps1, "seconds": round(el1, 2)},
               "other_configs": {"what": "the same loop on configs 1, 3, 4 (a token-row slice scaled to M) and "
                                         "5 (one layer + an 8192-row lm_head block, scaled to 32 layers + "
                                         "131072 rows); each timed ~1.2 s",
                                 f"threads_{ncpu}": cpu_configs(synth, w_gate, w_down, ncpu),
                                 "threads_1": cpu_configs(synth, w_gate, w_down, 1)}}

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "BASELINE config 2: decode FFN GEMV set, batch 1 -- q8-quantize x + fused "
                               "gate+up Q5_K 2x(9216x3072) in one launch, q8-quantize t + down Q6_K "
                               "3072x9216 (raw GGUF) in one launch (bq_gemv_q8_fused)",
                   "K": K, "FF": FF, "weight_sets_rotated": nsets, "bytes_per_step": step_bytes,
                   "hbm_frac_of_step": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for("gemv_q5k_gateup_fused"),
                     "kernel": "k_gemv<FmtQ5K, 1, 3, 1, 256, 3072> (quantize x + gate+up)", "bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(gu_ms * 1e3, 3)},
        "down_gemv": {"kernel": "k_gemv<FmtQ6KRaw, 1, 2, 1, 1024, 9216> (quantize t + down)", "avg_launch_us": round(dn_ms * 1e3, 3),
                      "GBps": round(gbs(dn_bytes, dn_ms), 1)},
        "decode_ffn_unfused": unfused,
        "hbm_read_ceiling": ceil_obj,
        "issue_probes": probe_obj,
        "gemv_config1_3072x3072": c1_obj,
        "gemv_config3_9216x3072": rows_res,
        "config5_whole_stack": stack_obj,
        "prompt_chunk": chunk_obj,
        "q8s_logits_head": q8s_obj,
        "q8_producers": norm_obj,
        "gguf_load": load_obj,
        "gemm": gemm_obj,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
