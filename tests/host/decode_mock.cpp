// Host-only check of bq_decode_enqueue's call sequence (bq_decode.hip built
// for the host alone): every entry point it calls is replaced by a recorder
// that checks each pointer argument lies inside a registered buffer with room
// for the elements the call touches, and counts the calls.  Run by
// tests/test_decode_host.py; prints one line per (fold, blocks) step and the
// number of bad arguments.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>
#include <hip/hip_runtime.h>
#include "bq.h"
#include "bq_internal.hpp"

namespace bq {
ScaledCopy& next_scaled_copy() {
    static ScaledCopy c;
    return c;
}
}

struct Buf { const char* name; size_t bytes; };
static std::map<uintptr_t, Buf> g_bufs;
static int g_bad = 0;
static int g_calls = 0;
static bool g_verbose = false;
static void* reg(const char* name, size_t bytes) {
    void* p = aligned_alloc(256, (bytes + 255) / 256 * 256);
    g_bufs[(uintptr_t)p] = {name, bytes};
    return p;
}
static void chk(const char* call, const char* arg, const void* p, size_t bytes) {
    if (!p) { printf("  %s: %s NULL (needs %zu B)\n", call, arg, bytes); g_bad++; return; }
    auto it = g_bufs.upper_bound((uintptr_t)p);
    if (it == g_bufs.begin()) { printf("  %s: %s=%p not a buffer\n", call, arg, p); g_bad++; return; }
    --it;
    const size_t off = (uintptr_t)p - it->first;
    if (off + bytes > it->second.bytes) {
        printf("  %s: %s in %s off %zu + %zu > %zu\n", call, arg, it->second.name, off, bytes, it->second.bytes);
        g_bad++;
    }
}
static const char* nm(const void* p) {
    if (!p) return "null";
    auto it = g_bufs.upper_bound((uintptr_t)p); --it; return it->second.name;
}
static size_t wbytes(const bq_weight* w) { return (size_t)w->N * (w->K / 256) * (w->ggml_type == BQ_TYPE_Q5_K ? 176 : 210); }

// a launch over these parts consumes an armed scaled copy of the part it names
static int g_scaled = 0;
static void consume_scaled(const char* call, const bq_weight* const* ws, int n) {
    bq::ScaledCopy& sc = bq::next_scaled_copy();
    for (int p = 0; sc.y && p < n; ++p)
        if (ws[p]->raw == sc.w) {
            chk(call, "scaled y", sc.y, 4 * (size_t)ws[p]->N);
            chk(call, "scaled s", sc.s, 4 * (size_t)ws[p]->N);
            sc = bq::ScaledCopy();
            ++g_scaled;
        }
}

extern "C" {
int bq_init(void) { return 0; }
int bq_verify_fused(float* const* ys, const bq_weight* const* ws, int n, int rows, const int8_t* xq, const float* xd,
                    const int32_t* xs, int, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("verify_fused n=%d rows=%d\n", n, rows);
    consume_scaled("verify", ws, n);
    for (int p = 0; p < n; ++p) { chk("verify", "y", ys[p], 4 * ws[p]->N * rows); chk("verify", "w", ws[p]->raw, wbytes(ws[p])); }
    chk("verify", "xq", xq, ws[0]->K * rows); chk("verify", "xd", xd, ws[0]->K / 8 * rows); chk("verify", "xs", xs, ws[0]->K / 8 * rows);
    return 0;
}
int bq_gemv(float* y, const bq_weight* w, const int8_t* xq, const float* xd, const int32_t* xs, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("gemv N=%d K=%d y=%s\n", w->N, w->K, nm(y));
    chk("gemv", "y", y, 4 * w->N); chk("gemv", "w", w->raw, wbytes(w)); chk("gemv", "xq", xq, w->K);
    chk("gemv", "xd", xd, w->K / 8); if (w->ggml_type == BQ_TYPE_Q5_K) chk("gemv", "xs", xs, w->K / 8);
    return 0;
}
static void gemm_args(const char* call, int rows, int K, const int8_t* xq, const float* xd, const int32_t* xs,
                      const uint16_t* xdh, const void* work, size_t work_bytes) {
    chk(call, "xq", xq, (size_t)K * rows); chk(call, "xd", xd, (size_t)K / 8 * rows); chk(call, "xs", xs, (size_t)K / 8 * rows);
    if (rows > BQ_MAX_ROWS && xdh) chk(call, "xdh", xdh, (size_t)K / 16 * rows);
    if (work) chk(call, "work", work, work_bytes);
}
int bq_gemm_b(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd, const int32_t* xs, uint16_t* xdh,
              void* work, size_t work_bytes, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("gemm_b rows=%d N=%d y=%s\n", rows, w->N, nm(y));
    chk("gemm_b", "y", y, 4 * (size_t)w->N * rows); chk("gemm_b", "w", w->raw, wbytes(w));
    gemm_args("gemm_b", rows, w->K, xq, xd, xs, xdh, work, work_bytes);
    return 0;
}
int bq_gemm_b_fused(float* const* ys, const bq_weight* const* ws, int n, int rows, const int8_t* xq, const float* xd,
                    const int32_t* xs, uint16_t* xdh, void* work, size_t work_bytes, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("gemm_b_fused n=%d rows=%d\n", n, rows);
    if (rows <= BQ_MAX_ROWS) { printf("  gemm_b_fused at %d rows\n", rows); g_bad++; }
    for (int p = 0; p < n; ++p) { chk("gbf", "y", ys[p], 4 * (size_t)ws[p]->N * rows); chk("gbf", "w", ws[p]->raw, wbytes(ws[p])); }
    gemm_args("gemm_b_fused", rows, ws[0]->K, xq, xd, xs, xdh, work, work_bytes);
    return 0;
}
int bq_gemv_norm_fused(float* const* ys, const bq_weight* const* ws, int nparts, int op, float* out, const float* a,
                       const float* b, const float* c, const float* d, int8_t* xq, float* xd, int32_t* xsum, bq_stream_t) {
    const int K = ws[0]->K;
    ++g_calls; if (g_verbose) printf("norm_fused op=%d parts=%d K=%d out=%s a=%s b=%s c=%s d=%s xq=%s\n", op, nparts, K, nm(out), nm(a), nm(b), nm(c), nm(d), nm(xq));
    consume_scaled("nf", ws, nparts);
    for (int p = 0; p < nparts; ++p) { chk("nf", "y", ys[p], 4 * ws[p]->N); chk("nf", "w", ws[p]->raw, wbytes(ws[p])); }
    chk("nf", "a", a, 4 * K);
    if (op != BQ_OP_NORM) chk("nf", "b", b, 4 * K);
    if (op >= BQ_OP_RESID && (op != BQ_OP_GATE || c)) chk("nf", "c", c, 4 * K);  // gate: c NULL = b scaled
    if (op == BQ_OP_SILU) chk("nf", "d", d, 4 * K);
    if (out) chk("nf", "out", out, 4 * K);
    if (xq) { chk("nf", "xq", xq, K); chk("nf", "xd", xd, K / 8); chk("nf", "xs", xsum, K / 8); }
    if (out && (out == a || out == b)) { printf("  out aliases input\n"); g_bad++; }
    return 0;
}
int bq_gate_up_silu(float* h, const bq_weight* wg, const bq_weight* wu, const float* sg, const float* su, const int8_t* xq, const float* xd, const int32_t* xs, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("gate_up_silu\n"); chk("gus", "h", h, 4 * wg->N); return 0;
}
static void nq(const char* op, float* out, const float* a, const float* b, const float* c, const float* d, int rows, int n, int8_t* xq, float* xd, int32_t* xs) {
    ++g_calls; if (g_verbose) printf("%s n=%d out=%s a=%s b=%s c=%s\n", op, n, nm(out), nm(a), nm(b), nm(c));
    if (out) chk(op, "out", out, 4 * n * rows); chk(op, "a", a, 4 * n * rows);
    if (b) chk(op, "b", b, 4 * n * rows); if (c) chk(op, "c", c, 4 * n); if (d) chk(op, "d", d, 4 * n);
    chk(op, "xq", xq, n * rows); chk(op, "xd", xd, n / 8 * rows); chk(op, "xs", xs, n / 8 * rows);
}
int bq_add_norm_q8(float* x, const float* h, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t) { nq("add_norm", x, x, h, 0, 0, rows, n, xq, xd, xs); return 0; }
int bq_resid_q8(float* x, const float* u, const float* al, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t) { nq("resid", x, x, u, al, 0, rows, n, xq, xd, xs); return 0; }
int bq_norm_q8(float* dst, const float* src, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t) { nq("norm", dst, src, 0, 0, 0, rows, n, xq, xd, xs); return 0; }
int bq_gate_norm_q8(float* dst, const float* a, const float* g, const float* sg, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t) { nq("gate_norm", dst, a, g, sg, 0, rows, n, xq, xd, xs); return 0; }
int bq_silu_mul_norm_q8(float* dst, const float* g, const float* u, const float* sg, const float* su, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t) { nq("silu_norm", dst, g, u, sg, su, rows, n, xq, xd, xs); return 0; }
int bq_gemv_q8s(float* y, const void* w, const int8_t* xq, const float* xd, int K, int N, int rows, const float* rs, bq_stream_t) {
    ++g_calls; if (g_verbose) printf("gemv_q8s K=%d N=%d rows=%d\n", K, N, rows); chk("q8s", "y", y, 4 * N * rows); chk("q8s", "xq", xq, K * rows); chk("q8s", "xd", xd, K / 8 * rows); return 0;
}
}
namespace bq {
int gemv_gate_den_fused(float* y, const void* w_raw, int K, int N, const float* a, const float* den, void*) {
    ++g_calls; if (g_verbose) printf("gate_den_fused K=%d N=%d\n", K, N);
    chk("gden", "y", y, 4 * (size_t)N); chk("gden", "w", w_raw, (size_t)N * (K / 256) * 176);
    chk("gden", "a", a, 4 * (size_t)K); chk("gden", "den", den, 4 * (size_t)K);
    return 0;
}
hipError_t launch_norm_q8(int op, float* out, const float* a, const float* b, const float* c, const float* d, int rows, int n, int8_t* xq, float* xd, int32_t* xs, hipStream_t) {
    nq(op == 2 ? "launch_norm_q8(resid)" : "launch_norm_q8", out, a, b, c, d, rows, n, xq, xd, xs); return hipSuccess;
}
}

int main(int argc, char** argv) {
    g_verbose = argc > 1;
    const int E = 3072, A = 4096, FF = 9216, V = 8192, R = 40;
    const int PN[4] = {A, 512, A, 512};
    bq_decode_block blocks[4];
    memset(blocks, 0, sizeof(blocks));
    std::vector<bq_weight*> keep;
    for (int l = 0; l < 2; ++l) {
        bq_weight* qw = new bq_weight[4]();
        float** outs = new float*[4];
        for (int i = 0; i < 4; ++i) {
            qw[i].K = E; qw[i].N = PN[i]; qw[i].ggml_type = i == 3 ? BQ_TYPE_Q6_K : BQ_TYPE_Q5_K;
            qw[i].raw = reg("qkvw", (size_t)PN[i] * (E / 256) * (i == 3 ? 210 : 176));
            outs[i] = (float*)reg("qkv_out", 4 * (size_t)PN[i] * R);
        }
        bq_weight* wo = new bq_weight(); wo->K = A; wo->N = E; wo->ggml_type = BQ_TYPE_Q5_K; wo->raw = reg("wo", (size_t)E * (A / 256) * 176);
        bq_weight* wg = new bq_weight(); wg->K = E; wg->N = FF; wg->ggml_type = BQ_TYPE_Q5_K; wg->raw = reg("wg", (size_t)FF * (E / 256) * 176);
        bq_weight* wu = new bq_weight(); *wu = *wg; wu->raw = reg("wu", (size_t)FF * (E / 256) * 176);
        bq_weight* wd = new bq_weight(); wd->K = FF; wd->N = E; wd->ggml_type = BQ_TYPE_Q6_K; wd->raw = reg("wd", (size_t)E * (FF / 256) * 210);
        bq_decode_block& a = blocks[2 * l];
        a.kind = BQ_BLOCK_ATTN; a.norm_before = l == 0; a.norm_after = 0;
        a.alpha = (float*)reg("alpha_a", 4 * E);
        a.qkv = qw; a.n_qkv = 4; a.qkv_out = outs;
        a.attn_out = (float*)reg("attn_out", 4 * (size_t)A * R); a.attn_gate = outs[2]; a.sgate = (float*)reg("sgate", 4 * A); a.n_attn = A;
        a.o = wo;
        bq_decode_block& f = blocks[2 * l + 1];
        f.kind = BQ_BLOCK_FFN; f.norm_before = 0; f.norm_after = l == 1;
        f.alpha = (float*)reg("alpha_f", 4 * E);
        f.gate = wg; f.up = wu; f.down = wd;
        f.s_gate = (float*)reg("sg", 4 * FF); f.s_up = (float*)reg("su", 4 * FF); f.n_ff = FF;
    }
    bq_decode_step st;
    memset(&st, 0, sizeof(st));
    st.blocks = blocks; st.n_embd = E;
    st.x = (float*)reg("x", 4 * E * R); st.input_h = (float*)reg("input_h", 4 * E * R);
    st.xq = (int8_t*)reg("xq", FF * R); st.xd = (float*)reg("xd", FF / 8 * R); st.xsum = (int32_t*)reg("xsum", FF / 8 * R);
    st.proj = (float*)reg("proj", 4 * E * R); st.ffn_g = (float*)reg("fg", 4 * FF * R); st.ffn_u = (float*)reg("fu", 4 * FF * R);
    st.head_q8s = reg("head", (size_t)V * E / 256 * 272); st.head_rs = (float*)reg("rs", 4 * V); st.vocab = V;
    st.logits = (float*)reg("logits", 4 * V * 8);  // every row's logits up to 8 rows, the last row's above
    float* xalt = (float*)reg("x_alt", 4 * E);
    for (int fold = 0; fold <= 2; ++fold)
        for (int nb = 1; nb <= 4; ++nb) {
            st.fold = fold; st.n_blocks = nb; st.x_alt = fold == 2 ? xalt : nullptr;
            g_calls = 0;
            const int bad0 = g_bad;
            const int r = bq_decode_enqueue(&st, nullptr);
            if (r) { printf("  returned %d\n", r); g_bad++; }
            if (bq::next_scaled_copy().y) { printf("  scaled copy left armed\n"); g_bad++; }
            printf("fold %d blocks %d calls %d bad %d scaled %d\n", fold, nb, g_calls, g_bad - bad0, g_scaled);
            g_scaled = 0;
        }
    // the verify step (8 rows) and a prompt chunk (R rows: the prefill GEMMs,
    // with and without xdh / workspace)
    uint16_t* xdh = (uint16_t*)reg("xdh", (size_t)FF / 16 * R);
    void* work = reg("work", 1 << 20);
    for (int c = 0; c < 3; ++c) {
        st.fold = 0; st.n_blocks = 4; st.x_alt = nullptr;
        st.rows = c == 0 ? 8 : R;
        st.xdh = c == 2 ? xdh : nullptr; st.work = c == 2 ? work : nullptr; st.work_bytes = c == 2 ? 1 << 20 : 0;
        g_calls = 0;
        const int bad0 = g_bad;
        const int r = bq_decode_enqueue(&st, nullptr);
        if (r) { printf("  returned %d\n", r); g_bad++; }
        printf("rows %d scratch %d calls %d bad %d\n", st.rows, c == 2, g_calls, g_bad - bad0);
    }
    st.rows = R; st.work = nullptr; st.work_bytes = 16;
    if (bq_decode_enqueue(&st, nullptr) != BQ_EINVAL) { printf("  work_bytes without work accepted\n"); g_bad++; }
    st.work_bytes = 0; st.rows = BQ_MAX_STEP_ROWS + 1;
    if (bq_decode_enqueue(&st, nullptr) != BQ_EINVAL) { printf("  rows above the limit accepted\n"); g_bad++; }
    printf("bad = %d\n", g_bad);
    return g_bad != 0;
}
