// bq_decode.hip -- the per-token decode step as one launch sequence and as a
// captured HIP graph (host C++ over the C ABI).
//
// Mirrors the reference's forward_launch (engine/src/bruce.cu:7902-8037), the
// per-block launch sequence of one decoded token, and capture_graph
// (:8046-8055) / the graph replay of bruce_decode_step (:8246-8252); with
// rows 2..8 its speculative-verify form, forward_batch_impl over `rows` tokens
// with all logits (:7610-7843), captured once per row count as
// capture_verify_graphs does (:7877-7900) and replayed by verify_launch
// (:7862-7875); with more rows a prompt chunk, forward_batch_impl as
// bruce_prefill_chunk calls it (:8274-8291: the MMQ GEMMs, the last row's
// logits only).  The reference's attention kernels (:7940-7970, :7716-7737)
// are outside this library: a caller hook enqueues them between the QKV
// projection and the gate norm, so they land in the same graph.
#include <string.h>

#include "../../include/bq.h"
#include "bq_internal.hpp"

namespace {

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// fold = 2 launches the resid producer directly (flush below): its buffers
// are checked here as the public producer entry points check theirs
bool fold2_ok(const bq_decode_step* s) {
    return s->x_alt && s->x_alt != s->x && al16(s->x) && al16(s->x_alt) && al16(s->proj) &&
           al16(s->xq) && al16(s->xd) && al16(s->xsum) && s->n_embd <= bq::kNormMaxN;
}

bool dims_ok(const bq_decode_step* s) {
    return s && s->n_blocks >= 0 && (s->n_blocks == 0 || s->blocks) && s->x && s->xq && s->xd && s->xsum &&
           s->proj && s->n_embd > 0 && (s->n_embd % 32) == 0 && s->rows >= 0 && s->rows <= BQ_MAX_STEP_ROWS &&
           s->fold >= 0 && s->fold <= 2 && (s->fold < 2 || fold2_ok(s)) && (s->work || !s->work_bytes);
}

// fold = 2: the resid -> q8 (k_resid :8017) of a block followed by an
// attention block runs inside that block's QKV GEMV (bq_gemv_norm_fused with
// BQ_OP_RESID), which writes the new residual row to the other of x / x_alt:
// every workgroup of that GEMV reads the old row, so it cannot be updated in
// place.  An attention block's loop-start norm (norm_before: k_add_norm
// :7914) runs inside its QKV GEMV the same way (BQ_OP_ADD).  `cur` is the
// buffer holding the residual row; a pending update is
// materialised (flush) by the standalone producer into x wherever the QKV
// GEMV cannot take it: before norm_before / norm_after, when the QKV has no
// Q5_K part or the fused form refuses it, and at the end of the step, so that
// x holds the step's result as in the other modes.  Before an FFN block the
// update stays a launch of its own: inside the gate+up GEMV every one of its
// ~1150 workgroups recomputes it from 36 KB of rows (about the matrix's own
// byte count again through L2), which measured slower than the launch.
struct Resid {
    float* cur = nullptr;
    const float* alpha = nullptr;  // non-null: an update of cur by proj is pending
    const float* add = nullptr;    // non-null: the loop-start norm of cur + add is pending
};

float* other_of(const bq_decode_step* s, const float* cur) { return cur == s->x ? s->x_alt : s->x; }

int flush(const bq_decode_step* s, Resid& rs, bq_stream_t st) {
    if (rs.add) {
        const hipError_t e = bq::launch_norm_q8(bq::kOpAdd, s->x, rs.cur, rs.add, nullptr, nullptr, 1, s->n_embd,
                                                s->xq, s->xd, s->xsum, (hipStream_t)st);
        rs.cur = s->x;
        rs.add = nullptr;
        if (e != hipSuccess) return -(int)e;
    }
    if (!rs.alpha) return BQ_OK;
    const hipError_t e = bq::launch_norm_q8(bq::kOpResid, s->x, rs.cur, s->proj, rs.alpha, nullptr, 1, s->n_embd,
                                            s->xq, s->xd, s->xsum, (hipStream_t)st);
    rs.cur = s->x;
    rs.alpha = nullptr;
    return e == hipSuccess ? BQ_OK : -(int)e;
}

// tokens per step: 0 means 1
int rows_of(const bq_decode_step* s) { return s->rows > 0 ? s->rows : 1; }

// values ffn_u holds per row: the largest n_ff of the step's FFN blocks
int max_ffn(const bq_decode_step* s) {
    int m = 0;
    for (int i = 0; i < s->n_blocks; ++i)
        if (s->blocks[i].kind == BQ_BLOCK_FFN && s->blocks[i].n_ff > m) m = s->blocks[i].n_ff;
    return m;
}

// y [rows][N] of a k-quant weight over the q8 rows: the single-row GEMV at one
// row (launch_gemv, :7982 / :8008), the prompt-batch dispatcher above
// (launch_gemm_b, :7750 / :7800: the multi-row kernels at 2..8 rows, the MMQ
// GEMMs with the step's xdh and workspace above)
int gemv_rows_of(float* y, const bq_weight* w, int rows, const bq_decode_step* s, bq_stream_t st) {
    if (rows == 1) return bq_gemv(y, w, s->xq, s->xd, s->xsum, st);
    return bq_gemm_b(y, w, rows, s->xq, s->xd, s->xsum, s->xdh, s->work, s->work_bytes, st);
}

// The Q5_K parts sharing the q8 rows in one launch where the kernels allow it:
// the fused GEMV / verify kernel up to 8 rows (launch_verify_fused), one MMQ
// launch over the parts above (launch_gemm_b_fused, :7421-7426); otherwise
// one launch per part
int parts_rows_of(float* const* ys, const bq_weight* const* ws, int n, int rows, const bq_decode_step* s,
                  bq_stream_t st) {
    if (rows > BQ_MAX_ROWS)
        return bq_gemm_b_fused(ys, ws, n, rows, s->xq, s->xd, s->xsum, s->xdh, s->work, s->work_bytes, st);
    const int r = bq_verify_fused(ys, ws, n, rows, s->xq, s->xd, s->xsum, 0, st);
    if (r != BQ_UNSUPPORTED) return r;
    for (int p = 0; p < n; ++p)
        if (int e = gemv_rows_of(ys[p], ws[p], rows, s, st)) return e;
    return BQ_OK;
}

// one attention block: bruce.cu:7915-7993 (QKV, attention, gate norm, O);
// rows 2..8: :7636-7757
int attn_block(const bq_decode_step* s, const bq_decode_block& b, int bi, int rows, Resid& rs, bq_stream_t st) {
    if (b.n_qkv < 1 || b.n_qkv > BQ_MAX_PARTS || !b.qkv || !b.qkv_out || !b.o || !b.attn_out || !b.attn_gate ||
        !b.sgate || b.n_attn <= 0 || (b.n_attn % 32) != 0)
        return BQ_EINVAL;
    // QKV: one fused launch over the parts (launch_verify_fused rows = 1,
    // :7921-7924); parts the fused kernel does not take (a Q6_K V, :7925-7926)
    // run as their own GEMVs
    const bq_weight* wp[BQ_MAX_PARTS];
    float* yp[BQ_MAX_PARTS];
    int nf = 0;
    for (int p = 0; p < b.n_qkv; ++p)
        if (b.qkv[p].ggml_type == BQ_TYPE_Q5_K) {
            wp[nf] = &b.qkv[p];
            yp[nf++] = b.qkv_out[p];
        }
    // fold >= 1: the QKV launch also writes its gate part times sg (the part
    // attn_gate starts, at most n_ff rows) into the scratch row ffn_u (unused
    // by the folded FFN block), so that the O GEMV's workgroups read two rows
    // instead of three; the same fp32 product the gate norm forms itself, so
    // the results are unchanged.  For a Q5_K O it writes the product's
    // sigmoid denominator 1 + exp(-gate * sg) instead, and the O GEMV's
    // producer only divides (kOpGateDen), with the same results.
    float* gate_s = nullptr;
    if (s->fold && s->ffn_u && al16(s->ffn_u) && rows == 1)
        for (int p = 0; p < nf; ++p)
            if (yp[p] == b.attn_gate && wp[p]->N >= b.n_attn && wp[p]->N <= max_ffn(s)) gate_s = s->ffn_u;
    // a Q5_K O projection takes the gate as its sigmoid denominators
    const bool den_o = b.o->ggml_type == BQ_TYPE_Q5_K && b.o->raw;
    auto arm = [&] {
        if (gate_s) {
            bq::ScaledCopy& sc = bq::next_scaled_copy();
            for (int p = 0; p < nf; ++p)
                if (yp[p] == b.attn_gate) sc.w = wp[p]->raw;
            sc.y = gate_s;
            sc.s = b.sgate;
            sc.den = den_o;
        }
    };
    auto disarm = [&] { bq::next_scaled_copy() = bq::ScaledCopy(); };
    bool qkv_done = false;
    if (nf > 0 && rs.alpha) {
        // the pending resid -> q8 inside the QKV GEMV; its q8 row is written
        // out only for the parts that run as their own GEMVs
        float* nx = other_of(s, rs.cur);
        const bool q8out = nf < b.n_qkv;
        arm();
        const int r = bq_gemv_norm_fused(yp, wp, nf, BQ_OP_RESID, nx, rs.cur, s->proj, rs.alpha, nullptr,
                                         q8out ? s->xq : nullptr, q8out ? s->xd : nullptr,
                                         q8out ? s->xsum : nullptr, st);
        disarm();
        if (r != BQ_OK && r != BQ_UNSUPPORTED) return r;
        if (r == BQ_OK) {
            rs.cur = nx;
            rs.alpha = nullptr;
            qkv_done = true;
        }
    } else if (nf > 0 && rs.add) {
        // the pending loop-start norm (k_add_norm, :7914) inside the QKV GEMV,
        // the same way
        float* nx = other_of(s, rs.cur);
        const bool q8out = nf < b.n_qkv;
        arm();
        const int r = bq_gemv_norm_fused(yp, wp, nf, BQ_OP_ADD, nx, rs.cur, rs.add, nullptr, nullptr,
                                         q8out ? s->xq : nullptr, q8out ? s->xd : nullptr,
                                         q8out ? s->xsum : nullptr, st);
        disarm();
        if (r != BQ_OK && r != BQ_UNSUPPORTED) return r;
        if (r == BQ_OK) {
            rs.cur = nx;
            rs.add = nullptr;
            qkv_done = true;
        }
    }
    if (int e = flush(s, rs, st)) return e;
    if (nf > 0 && !qkv_done) {
        arm();
        const int e = parts_rows_of(yp, wp, nf, rows, s, st);
        disarm();
        if (e) return e;
    }
    for (int p = 0; p < b.n_qkv; ++p)
        if (b.qkv[p].ggml_type != BQ_TYPE_Q5_K)
            if (int e = gemv_rows_of(b.qkv_out[p], &b.qkv[p], rows, s, st)) return e;
    if (s->attention) s->attention(s->user, bi, st);
    // gate norm -> q8, then O (k_gate_norm :7975-7978, launch_gemv :7982;
    // rows: k_gate_norm_vec4 :7740, launch_gemm_b :7757); folded: the gate
    // norm runs inside the O GEMV (bq_gemv_norm_fused, one row)
    if (s->fold) {
        float* yo[1] = {s->proj};
        const bq_weight* po[1] = {b.o};
        if (gate_s && den_o)
            // the QKV launch wrote the sigmoid denominators 1 + exp(-gate * sg)
            // (the exponential once per value instead of in every O workgroup:
            // folded chain fold 1 / 2 1.234 / 1.168 -> 1.230 / 1.164 ms/token)
            return bq::gemv_gate_den_fused(s->proj, b.o->raw, b.o->K, b.o->N, b.attn_out, gate_s, st);
        if (gate_s)  // the scaled gate row: gate * sg, sg already applied
            return bq_gemv_norm_fused(yo, po, 1, BQ_OP_GATE, nullptr, b.attn_out, gate_s, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, st);
        return bq_gemv_norm_fused(yo, po, 1, BQ_OP_GATE, nullptr, b.attn_out, b.attn_gate, b.sgate, nullptr,
                                  nullptr, nullptr, nullptr, st);
    }
    if (int e = bq_gate_norm_q8(nullptr, b.attn_out, b.attn_gate, b.sgate, rows, b.n_attn, s->xq, s->xd, s->xsum,
                                st))
        return e;
    return gemv_rows_of(s->proj, b.o, rows, s, st);
}

// one FFN block: bruce.cu:7994-8012 (gate+up, silu*mul norm, down); rows
// 2..8: :7759-7800
int ffn_block(const bq_decode_step* s, const bq_decode_block& b, int rows, Resid& rs, bq_stream_t st) {
    if (!b.gate || !b.up || !b.down || !b.s_gate || !b.s_up || !s->ffn_g || b.n_ff <= 0 || (b.n_ff % 32) != 0)
        return BQ_EINVAL;
    if (int e = flush(s, rs, st)) return e;
    if (s->fold) {
        // silu*mul in the gate+up epilogue (h -> ffn_g), its norm + q8 inside the down GEMV
        if (int e = bq_gate_up_silu(s->ffn_g, b.gate, b.up, b.s_gate, b.s_up, s->xq, s->xd, s->xsum, st)) return e;
        float* yd[1] = {s->proj};
        const bq_weight* pd[1] = {b.down};
        return bq_gemv_norm_fused(yd, pd, 1, BQ_OP_NORM, nullptr, s->ffn_g, nullptr, nullptr, nullptr, nullptr,
                                  nullptr, nullptr, st);
    }
    if (!s->ffn_u) return BQ_EINVAL;
    float* y2[2] = {s->ffn_g, s->ffn_u};
    const bq_weight* p2[2] = {b.gate, b.up};
    if (int r = parts_rows_of(y2, p2, 2, rows, s, st)) return r;
    if (int e = bq_silu_mul_norm_q8(nullptr, s->ffn_g, s->ffn_u, b.s_gate, b.s_up, rows, b.n_ff, s->xq, s->xd,
                                    s->xsum, st))
        return e;
    return gemv_rows_of(s->proj, b.down, rows, s, st);
}

}  // namespace

struct bq_decode_graph {
    hipGraphExec_t exec;
};

extern "C" {

int bq_decode_enqueue(const bq_decode_step* s, bq_stream_t st) {
    if (int r = bq_init()) return r;
    if (!dims_ok(s)) return BQ_EINVAL;
    const int n = s->n_embd, rows = rows_of(s);
    // the folded producers are one-row GEMV epilogues / prologues
    if (s->fold && rows > 1) return BQ_UNSUPPORTED;
    Resid rs;
    rs.cur = s->x;
    for (int i = 0; i < s->n_blocks; ++i) {
        const bq_decode_block& b = s->blocks[i];
        // loop start: x = norm(x + input_h) (k_add_norm, :7914; rows: k_add_norm_rows :7633)
        if (b.norm_before) {
            if (int e = flush(s, rs, st)) return e;
            if (!s->input_h) return BQ_EINVAL;
            if (s->fold == 2 && b.kind == BQ_BLOCK_ATTN) {
                rs.add = s->input_h;  // fold = 2: inside the block's QKV GEMV (attn_block)
            } else if (int e = bq_add_norm_q8(s->x, s->input_h, rows, n, s->xq, s->xd, s->xsum, st)) {
                return e;
            }
        }
        const int r = b.kind == BQ_BLOCK_FFN ? ffn_block(s, b, rows, rs, st) : b.kind == BQ_BLOCK_ATTN
                                                                                 ? attn_block(s, b, i, rows, rs, st)
                                                                                 : BQ_EINVAL;
        if (r) return r;
        if (!b.alpha) return BQ_EINVAL;
        if (b.norm_after) {
            // the block's resid -> q8 and the loop-end norm (k_resid :8017,
            // k_norm :8022; rows: :7803-7818) in one launch, bit-identical to
            // the two; it also takes up a pending update (fold = 2)
            if (int e = flush(s, rs, st)) return e;
            const hipError_t he = bq::launch_norm_q8(bq::kOpResidNorm, s->x, rs.cur, s->proj, b.alpha, nullptr, rows,
                                                     n, s->xq, s->xd, s->xsum, (hipStream_t)st);
            if (he != hipSuccess) return -(int)he;
            rs.cur = s->x;
            continue;
        }
        // x = resid(x, proj, alpha) -> q8 x (k_resid_vec4, :8017; rows: :7803-7815);
        // fold = 2: left pending for the next block's QKV GEMV
        if (s->fold == 2) {
            rs.alpha = b.alpha;
            const bool to_qkv = i + 1 < s->n_blocks && s->blocks[i + 1].kind == BQ_BLOCK_ATTN;
            if (!to_qkv)
                if (int e = flush(s, rs, st)) return e;
        } else if (int e = bq_resid_q8(s->x, s->proj, b.alpha, rows, n, s->xq, s->xd, s->xsum, st)) {
            return e;
        }
    }
    if (int e = flush(s, rs, st)) return e;
    // logits from the q8 rows of x: every row up to 8 rows (:8026-8032; rows:
    // launch_logits_b :7832), the last row of a prompt chunk (:7833-7836)
    if ((s->head_q8s || s->head) && !s->logits) return BQ_EINVAL;
    const int lr = rows > BQ_MAX_ROWS ? 1 : rows;
    const size_t off = (size_t)(rows - lr) * n;
    if (s->head_q8s)
        return bq_gemv_q8s(s->logits, s->head_q8s, s->xq + off, s->xd + off / 32, n, s->vocab, lr, s->head_rs, st);
    if (s->head) {
        if (lr == 1) return bq_gemv(s->logits, s->head, s->xq + off, s->xd + off / 32, s->xsum + off / 32, st);
        return gemv_rows_of(s->logits, s->head, rows, s, st);
    }
    return BQ_OK;
}

int bq_decode_graph_create(const bq_decode_step* s, bq_stream_t st, bq_decode_graph** out) {
    if (!out) return BQ_EINVAL;
    *out = nullptr;
    if (int r = bq_init()) return r;
    if (!dims_ok(s)) return BQ_EINVAL;
    // capture on a private stream that follows the caller's, as capture_graph
    // does on S (:8046-8055), in thread-local mode so other threads' work is
    // not captured
    hipStream_t cs;
    hipError_t e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
    if (e != hipSuccess) return -(int)e;
    int r = BQ_OK;
    hipGraph_t g = nullptr;
    hipGraphExec_t ex = nullptr;
    if ((e = hipStreamSynchronize((hipStream_t)st)) != hipSuccess ||
        (e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal)) != hipSuccess) {
        r = -(int)e;
    } else {
        r = bq_decode_enqueue(s, (bq_stream_t)cs);
        e = hipStreamEndCapture(cs, &g);
        if (!r && e != hipSuccess) r = -(int)e;
        if (!r && (e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0)) != hipSuccess) r = -(int)e;
        if (g) (void)hipGraphDestroy(g);
    }
    (void)hipStreamDestroy(cs);
    if (r) {
        if (ex) (void)hipGraphExecDestroy(ex);
        return r;
    }
    bq_decode_graph* dg = new bq_decode_graph;
    dg->exec = ex;
    *out = dg;
    return BQ_OK;
}

int bq_decode_graph_launch(const bq_decode_graph* g, bq_stream_t st) {
    if (!g) return BQ_EINVAL;
    const hipError_t e = hipGraphLaunch(g->exec, (hipStream_t)st);
    return e == hipSuccess ? BQ_OK : -(int)e;
}

void bq_decode_graph_destroy(bq_decode_graph* g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    delete g;
}

}  // extern "C"
