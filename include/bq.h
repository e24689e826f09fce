/*
 * bq.h -- C ABI of the MI355X k-quant matmul path (libbq.so).
 *
 * Drop-in replacement for the quantized-matmul launchers of the reference
 * engine (engine/src/bruce.cu).  Every compute entry point is stream-ordered,
 * allocates nothing, never synchronises and never exits; all buffers are
 * caller-owned device memory (weights, q8 activations, outputs, repack
 * targets, and the prefill GEMMs' scratch: xdh and the K-split workspace), as
 * the reference preallocates its scratch once (alloc_buffers, bruce.cu:5525-5547).
 * The GGUF loader (host file I/O) is the one exception, see below.
 *
 * Return codes: BQ_OK (0); BQ_UNSUPPORTED (1) = shape/type not handled, nothing
 * was enqueued and the caller should fall back (the reference's `return false`,
 * bruce.cu:7147-7161, :7366-7390); BQ_EINVAL (2) = bad argument (null pointer,
 * K not a multiple of 256, a weight / activation / fp32 row buffer that does
 * not start 16-byte aligned, ...); BQ_ETOOBIG (3) = larger than the static
 * scratch of the allocation-free entry point; a negative value = -(hipError_t) of a failed
 * launch.  bq_strerror() names each code.
 *
 * Layouts (GGUF blocks are read unchanged):
 *   Q5_K  176 B / 256 values: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
 *   Q6_K  210 B / 256 values: ql[128] | qh[64] | sc i8[16] | d f16
 *   q8 activations (structure of arrays, bruce.cu:123-127):
 *         xq int8 [rows][K], xd fp32 [rows][K/32], xsum int32 [rows][K/32]
 *   W144  Q5_K repack, stage-major [K/128][N][144]: 128 u8 codes + 4 fp32 d*sc,
 *         plus Dm fp16 [N][K/32] = half(-dmin*m)          (bruce.cu:5747-5789)
 *   W160  Q6_K repack, row-major [N][K/128][160]: 128 int8 (code-32) + 8 fp32 d*sc
 *                                                          (bruce.cu:4783-4811)
 *   outputs fp32 y[row][N], fully overwritten.
 */
#ifndef BQ_H
#define BQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* bq_stream_t; /* == hipStream_t; NULL = default stream */

enum { BQ_OK = 0, BQ_UNSUPPORTED = 1, BQ_EINVAL = 2, BQ_ETOOBIG = 3 };
enum { BQ_TYPE_Q5_K = 13, BQ_TYPE_Q6_K = 14 }; /* GGML type ids (gguf.h:29-30) */
enum { BQ_MAX_PARTS = 4, BQ_MAX_ROWS = 8, BQ_MAX_STEP_ROWS = 8192 };

/* Weight descriptor.  Mirrors `struct TensorW { d, dp, dm, type, K, N }`
 * (bruce.cu:78): raw = GGUF blocks, rep = W144 (Q5_K) or W160 (Q6_K) repack or
 * NULL, rep_min = Dm fp16 for Q5_K W144 or NULL. */
typedef struct bq_weight {
    const void* raw;
    const void* rep;
    const void* rep_min;
    uint32_t ggml_type;
    int32_t K, N;
} bq_weight;

/* Library set-up: reads the current device's limits.  Optional (every entry
 * point calls it on first use); call it outside graph capture. */
int bq_init(void);
const char* bq_strerror(int code);
const char* bq_version(void);

/* ---- activation quantizer ------------------------------------------------
 * Replaces k_q8_quant (bruce.cu:518-539, launched :7907) and k_q8_rows
 * (bruce.cu:1081-1108, launched :7621); with xdh != NULL it also writes
 * xdh = half(xd*xsum), replacing k_fill_xdh (bruce.cu:6598-6602, :7402).
 * Per 32 values: d = amax*(1/127), id = d>0 ? 1/d : 0, q = clamp(rint(v*id),
 * -127, 127), xsum = sum q.  Bit-exact with the reference.  K % 32 == 0. */
int bq_quantize_q8(const float* x, int rows, int K, int8_t* xq, float* xd, int32_t* xsum,
                   uint16_t* xdh, bq_stream_t st);
/* xdh = half(xd*xsum) on its own (k_fill_xdh, bruce.cu:6598-6602). */
int bq_fill_xdh(const float* xd, const int32_t* xsum, int n, uint16_t* xdh, bq_stream_t st);

/* ---- q8 producers: elementwise op -> row L2 norm -> q8 ---------------------
 * The kernels that feed the GEMVs on the reference's decode / batch paths emit
 * the q8 activations themselves.  Per row of n values (rows >= 0, one
 * workgroup each): t = op(inputs), v = t * l2_scale(sum t^2, n) with
 * l2_scale(ss, n) = (1/sqrt(ss/n + 1e-6/n)) * (1/sqrt(n)) (bruce.cu:305-307),
 * then the q8 row of v exactly as bq_quantize_q8 would produce it from v
 * (q8_emit, bruce.cu:338-366).  The fp32 output is written unless it is NULL
 * (it is x itself for add / resid).  alpha, sg, su are per-column vectors [n].
 * n % 32 == 0 and n <= 32768 (else BQ_UNSUPPORTED); every pointer 16-byte
 * aligned except xd / xsum.  exp is the accurate expf (the reference uses the
 * fast __expf), so fp32 outputs agree to rounding, not bit for bit. */
/* dst = norm(src); k_norm (bruce.cu:541-554), k_norm_rows (:1110-1126). */
int bq_norm_q8(float* dst, const float* src, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
               bq_stream_t st);
/* x = norm(x + h); k_add_norm (:556-569), k_add_norm_rows (:1128-1145). */
int bq_add_norm_q8(float* x, const float* h, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
                   bq_stream_t st);
/* x = norm(a + (b - a)*alpha), a = norm(x), b = norm(upd); k_resid (:571-600),
 * k_resid_rows (:1146-1179), k_resid_vec4 (:1475-1527). */
int bq_resid_q8(float* x, const float* upd, const float* alpha, int rows, int n, int8_t* xq, float* xd,
                int32_t* xsum, bq_stream_t st);
/* dst = norm(aout / (1 + exp(-gate*sg))); k_gate_norm (:602-620),
 * k_gate_norm_rows (:1181-1203), k_gate_norm_vec4 (:1529-1572). */
int bq_gate_norm_q8(float* dst, const float* aout, const float* gate, const float* sg, int rows, int n,
                    int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st);
/* dst = norm(silu(g*sg) * u * su); k_silu_mul_norm (:622-641),
 * k_silu_mul_norm_rows (:1205-1228), k_silu_mul_norm_vec4 (:1427-1473). */
int bq_silu_mul_norm_q8(float* dst, const float* g, const float* u, const float* sg, const float* su, int rows,
                        int n, int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st);

/* ---- decode GEMV ----------------------------------------------------------
 * The GEMV / multi-row entry points take K <= 49152 (BQ_UNSUPPORTED above). 
 * y[N] = W x for one activation row.  Replaces launch_gemv(y, w, x, st)
 * (bruce.cu:5624-5640): Q5_K raw -> k_gemv_q5k (:384-440); Q6_K with a W160
 * repack -> k_gemv_q6k_dp (:4452-4513), else raw Q6_K -> k_gemm_q6k (:4282). */
int bq_gemv(float* y, const bq_weight* w, const int8_t* xq, const float* xd,
            const int32_t* xsum, bq_stream_t st);

/* Fused multi-matrix GEMV / verify GEMM: nparts (1..4) Q5_K matrices sharing
 * K and the activation rows, rows 1..8, row r reads activation row xoff+r.
 * Replaces launch_verify_fused (bruce.cu:7141-7229): rows==1 -> the fused GEMV
 * k_gemv_q5k_fused (:5815-5887), rows 2..8 -> k_gemm_tc_verify_q5k (:5889-6076).
 * Returns BQ_UNSUPPORTED (nothing enqueued) on non-Q5_K parts, mismatched K,
 * K % 256 != 0, N % 16 != 0 or rows outside 1..8. */
int bq_verify_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                    const int8_t* xq, const float* xd, const int32_t* xsum, int xoff,
                    bq_stream_t st);

/* Q6_K multi-row (2..8) over the W160 repack, 1..4 parts.  Replaces
 * launch_q6_verify_fused (bruce.cu:7231-7283; kernel k_gemm_tc_verify_q6k :6078). */
int bq_q6_verify_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                       const int8_t* xq, const float* xd, int xoff, bq_stream_t st);

/* Q6_K GEMV over the W160 repack, rows 1..8.  Replaces launch_gemm_q6k_dp
 * (bruce.cu:7285-7364; kernel k_gemv_q6k_dp :4452-4513). */
int bq_gemm_q6k_dp(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                   int xoff, bq_stream_t st);

/* Q6_K multi-row over the raw 210 B blocks, rows 1..8.  Replaces the Q6_K arm of
 * launch_gemm_b_impl (bruce.cu:7108-7124; kernel k_gemm_q6k :4282-4362). */
int bq_gemm_q6k_raw(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                    int xoff, bq_stream_t st);

/* Fused quantize + GEMV of one fp32 activation row x[K] against nparts (1..4)
 * matrices of one type sharing K (all Q5_K raw, or all Q6_K: W160 repacks if
 * part 0 has one, else raw blocks).  Replaces the decode pair "quantize, then
 * GEMV" -- k_q8_quant (bruce.cu:518-539) followed by launch_verify_fused rows==1
 * (:7141-7229) or launch_gemv (:5624-5640) -- with one launch: every workgroup
 * quantizes x itself, bit-exactly as bq_quantize_q8.  xq/xd/xsum (all three or
 * none) receive the q8 row for later consumers.  K % 256 == 0 and
 * K <= 49152 (the GEMV kernels' limit), else BQ_UNSUPPORTED.
 * An extension of this library: the reference has no single-launch form. */
int bq_gemv_q8_fused(float* const* ys, const bq_weight* const* ws, int nparts, const float* x,
                     int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st);

/* q8 producer + GEMV of the produced row in one launch: one of the q8
 * producers above (op: BQ_OP_NORM, BQ_OP_ADD, BQ_OP_RESID, BQ_OP_GATE,
 * BQ_OP_SILU with the inputs a, b, c, d in the order of bq_norm_q8 ..
 * bq_silu_mul_norm_q8: norm a; add a, h=b; resid x=a, upd=b, alpha=c; gate
 * aout=a, gate=b, sg=c, where c NULL means b already holds gate*sg; silu
 * g=a, u=b, sg=c, su=d) computed by every
 * workgroup for the one activation row, quantized and consumed by the GEMV
 * over nparts (1..4) matrices sharing K (types as bq_gemv_q8_fused).
 * Replaces the decode pair "q8 producer, then GEMV" of the reference --
 * e.g. k_silu_mul_norm (bruce.cu:622) + launch_gemv (:5624) for the down
 * projection, k_resid (:571) + launch_verify_fused (:7141) for gate+up, k_gate_norm
 * (:602) + launch_gemv for the O projection -- with one launch.
 * out (optional) receives the producer's fp32 row (the new x for add /
 * resid: the reference updates x in place, here out must not be a or b,
 * which every workgroup reads; BQ_EINVAL otherwise); xq/xd/xsum (all or
 * none) its q8 row.  out and the q8 row are bit-identical to the standalone
 * producer's; ys equal bq_gemv_q8_fused on that fp32 row up to fp32
 * summation order (the K split may differ: this path keeps the fewest
 * workgroups, since each one recomputes the producer).
 * K % 256 == 0 and K <= 16384, else BQ_UNSUPPORTED.  An extension of this
 * library: the reference has no fused form. */
/* Gate and up projections of one q8 activation row with the elementwise
 * silu*mul epilogue: h[n] = silu(g[n] * sg[n]) * u[n] * su[n] with g = Wg x,
 * u = Wu x (silu(v) = v / (1 + exp(-v))), in one launch that reads both
 * matrices once and writes only h.  Replaces the gate+up GEMV
 * (launch_verify_fused, bruce.cu:7141) and the elementwise half of
 * k_silu_mul_norm (:622); the norm + q8 half then runs inside the down
 * projection's GEMV (bq_gemv_norm_fused with BQ_OP_NORM on h).  g and u are
 * bit-identical to bq_verify_fused / bq_gemv on the same inputs, and h to
 * silu_mul of them.  wg, wu: same type (Q5_K raw, or Q6_K raw / W160), K and
 * N; K % 256 == 0, N % 16 == 0, else BQ_UNSUPPORTED; xsum required for Q5_K.
 * An extension of this library: the reference has no fused form. */
int bq_gate_up_silu(float* h, const bq_weight* wg, const bq_weight* wu, const float* sg, const float* su,
                    const int8_t* xq, const float* xd, const int32_t* xsum, bq_stream_t st);

#define BQ_OP_NORM 0
#define BQ_OP_ADD 1
#define BQ_OP_RESID 2
#define BQ_OP_GATE 3
#define BQ_OP_SILU 4
int bq_gemv_norm_fused(float* const* ys, const bq_weight* const* ws, int nparts, int op, float* out,
                       const float* a, const float* b, const float* c, const float* d, int8_t* xq,
                       float* xd, int32_t* xsum, bq_stream_t st);

/* ---- prefill GEMM ----------------------------------------------------------
 * K-split workspace.  A GEMM whose 128x128 tiles leave the GPU's workgroup
 * slots unfilled (e.g. one 128-token tile of a 9216-row matrix) is split over
 * K; the slices' partial outputs go to a caller-owned workspace and one more
 * launch sums them in a fixed order.  The split is chosen from the shape and
 * work_bytes alone, so equal calls (eager or captured in a graph) take equal
 * paths and give equal bits.  work = NULL (or too small) means a smaller or no
 * split.  bq_gemm_workspace_bytes gives the size that allows the full split of
 * a launch of `rows` activation rows over matrices of n_total = sum N_p rows
 * (0: that launch never splits); on 256 CUs it is at most 32 MiB for any
 * shape (in general at most the larger of 32 MiB and CUs x 128 KiB).  The
 * size is the largest any tier (W144, raw Q5_K, Q6_K) takes for the shape, so
 * one workspace serves every call of that shape.  The split counts the
 * workgroup slots of the device, so the size is for the current device (0
 * when there is none); bq_gemm_workspace_bytes_cus gives it for a device of
 * `cus` compute units (MI355X: 256).  work must be 16-byte aligned.  Calls
 * that share a workspace must be ordered (one stream, or events): the
 * workspace holds one call's partials at a time.  No counterpart in the
 * reference (its 128x128 GEMM never splits K). */
size_t bq_gemm_workspace_bytes(int rows, int K, int n_total);
size_t bq_gemm_workspace_bytes_cus(int rows, int K, int n_total, int cus);

/* Y_p[M][N_p] for nparts (1..4) Q5_K matrices, 128x128 tiles on int8 MFMA.
 * Replaces try_launch_mmq (bruce.cu:7366-7419).  rows >= 96 (the reference's
 * rule), N_p % 128 == 0, K % 256 == 0, else BQ_UNSUPPORTED.  If every part has
 * rep/rep_min and K % 512 == 0 the W144 kernel runs (k_gemm_mmq_q5k_144
 * :6604-6792, fp16 min term from Dm and xdh; xdh scratch [M][K/32] must be
 * given and is written first, as k_fill_xdh does); otherwise the raw-Q5_K
 * kernel runs (k_gemm_mmq_q5k :6367-6593, fp32 min term) and xdh is unused.
 * ys and xq 16-byte aligned. */
int bq_try_mmq(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
               const int8_t* xq, const float* xd, const int32_t* xsum, uint16_t* xdh,
               void* work, size_t work_bytes, bq_stream_t st);

/* Q6_K prefill GEMM over W160, rows >= 1, N % 128 == 0.  Replaces the
 * k_gemm_mma_q6k_128 arm of launch_gemm_b (bruce.cu:7475-7521; kernel :6943-7063). */
int bq_gemm_q6k_mma(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                    void* work, size_t work_bytes, bq_stream_t st);

/* Prompt-batch dispatcher.  Replaces launch_gemm_b (bruce.cu:7428-7568): rows
 * <= 8 -> the verify / GEMV kernels above; Q5_K (W144 prepack or raw) and
 * Q6_K W160 above 8 rows -> the MFMA GEMMs (a 32- or 128-token tile,
 * whichever a work estimate for the launch's shape favours; the 8-row chunks
 * stream
 * the weights once per chunk); otherwise 8-row chunks of the multi-row
 * kernels.  (The reference sends rows 9..95 to a 64x64 MMA tile.)  The W144
 * tier needs xdh as bq_try_mmq does, but at 9..64 rows its tile forms the
 * min term's half(xd*xsum) itself and xdh is not written.  Never returns
 * BQ_UNSUPPORTED for a Q5_K/Q6_K weight with K % 256 == 0. */
int bq_gemm_b(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
              const int32_t* xsum, uint16_t* xdh, void* work, size_t work_bytes, bq_stream_t st);
/* launch_gemm_b_fused (bruce.cu:7421-7426): one MMQ launch over the parts if
 * possible (row thresholds of bq_gemm_b), otherwise bq_gemm_b per part. */
int bq_gemm_b_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                    const int8_t* xq, const float* xd, const int32_t* xsum, uint16_t* xdh,
                    void* work, size_t work_bytes, bq_stream_t st);

/* Allocation-free variant of bq_gemm_b_fused, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  No counterpart in the reference.  The W144 tier's xdh
 * rows and the K-split workspace live in a 16 MiB static device array of the
 * library (4 MiB for xdh, 12 MiB of workspace), which each GPU the library
 * runs on holds until the process ends; the caller passes only inputs and
 * outputs.  A call that takes the W144 tier (every part Q5_K with
 * rep/rep_min, K % 512 == 0, N_p % 128 == 0, rows > 8) needs
 * rows * (K/32) * 2 <= 4 MiB of xdh, else BQ_ETOOBIG (nothing enqueued), and
 * equals bq_gemm_b_fused given its own xdh and a 12 MiB workspace, bit for
 * bit; any other call uses no xdh and the whole 16 MiB as its workspace, and
 * equals bq_gemm_b_fused given a 16 MiB workspace.  Every call on one GPU
 * shares that GPU's array and it keeps the last call's contents (nothing in it needs clearing: each call
 * writes what it reads): calls that overlap on one GPU (other streams, other
 * host threads, graphs replayed concurrently) race, so order them. */
int bq_gemm_b_fused_noalloc(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                            const int8_t* xq, const float* xd, const int32_t* xsum, bq_stream_t st);
size_t bq_noalloc_scratch_bytes(void);  /* 16 MiB */

/* ---- load-time repacks -----------------------------------------------------
 * Q5_K raw -> W144 + Dm (k_q5k_prepack144, bruce.cu:5747-5789, launched by
 * q5k_prepack_launch :4832-4838).  Bit-exact with the reference. */
int bq_repack_q5k(const void* raw, int K, int N, void* w144, uint16_t* dm, bq_stream_t st);
size_t bq_repack_q5k_bytes(int K, int N);     /* W144 bytes: (K/128)*N*144 */
size_t bq_repack_q5k_min_bytes(int K, int N); /* Dm bytes:   N*(K/32)*2   */
/* Q6_K raw -> W160 on the device (device twin of q6k_repack_host). */
int bq_repack_q6k(const void* raw, int K, int N, void* w160, bq_stream_t st);
/* Host version: q6k_repack_host (bruce.cu:4783-4811), same bytes. */
int bq_repack_q6k_host(const void* raw, int K, int N, void* w160);
size_t bq_repack_q6k_bytes(int K, int N);     /* N*(K/128)*160 */

/* ---- Q8_0 logits head ------------------------------------------------------
 * Q8S layout (bruce.cu:4400-4407): per (row, 256 values) 272 B = 8 fp16 group
 * scales | 256 int8 codes; row-major [N][K/256][272].  K % 256 == 0.
 * The BF16 output matrix is converted once at load and the decode / prompt
 * logits read it with the q8 activations the last norm already produced. */
size_t bq_q8s_bytes(int K, int N);            /* N*(K/256)*272 */
/* BF16 [N][K] (bit patterns) -> Q8S on the device.  Replaces k_bf16_to_q8
 * (bruce.cu:5159-5184).  Per 32 values d = amax*(1/127), id = d>0 ? 1/d : 0,
 * q = clamp(rint(v*id), -127, 127), scale = half_rn(d).  Bit-exact with the
 * reference for finite inputs.  A group with 0 < amax < 127/FLT_MAX has
 * id = inf: its zero values (0 * inf = NaN) give code 0 and its other values
 * +-127, as __float2int_rn does on the device; the reference's host loop
 * leaves that case to lrintf(inf), which differs.  bf16 and dst 16-byte
 * aligned. */
int bq_quantize_q8s(const uint16_t* bf16, int K, int N, void* dst, bq_stream_t st);
/* Host version: q8k_quant_host (bruce.cu:4843-4867), same bytes. */
int bq_quantize_q8s_host(const uint16_t* bf16, int K, int N, void* dst);
/* y[m][n] = rs[n] * sum_g ws[n][g]*xd[m][g]*dot(codes[n][g], xq[m][g]) for
 * m < rows (1..8); rs NULL means 1.  Replaces k_gemm_q8_logits<M,8>
 * (bruce.cu:4409-4449) as launched by launch_logits_b (:7570-7590) and the
 * decode / last-row calls (:8028-8032, :7831-7836).  xq [rows][K] and xd
 * [rows][K/32] as from bq_quantize_q8 (xsum is not used); w and xq 16-byte
 * aligned.  K <= 4096, else BQ_UNSUPPORTED. */
int bq_gemv_q8s(float* y, const void* w, const int8_t* xq, const float* xd, int K, int N, int rows,
                const float* rs, bq_stream_t st);

/* ---- GGUF reader and streaming loader ---------------------------------------
 * Replaces GgufFile (engine/src/gguf.h:146-346: v3 header, key/value metadata,
 * tensor table, pread streaming) and the k-quant part of the streamed weight
 * loader (bruce.cu:4869-5131, bind_weights :5186-5443).  Host calls; the
 * reader needs no GPU.  Strings returned stay valid until bq_gguf_close. */
typedef struct bq_gguf bq_gguf;
typedef struct bq_gguf_tensor {
    const char* name;
    const char* suffix;   /* "attn_q.weight" for "blk.3.attn_q.weight", else "" */
    uint64_t ne[4];       /* ne[0] = K (row length), ne[1] = N (rows) */
    uint64_t offset;      /* absolute file offset of the tensor data */
    uint64_t nbytes;
    uint32_t ggml_type;
    uint32_t ndim;
    int32_t block;        /* N of "blk.N." names, else -1 */
} bq_gguf_tensor;
/* BQ_EINVAL: unreadable file, bad magic, version != 3, unknown value or tensor
 * type, truncated header, or a tensor extending past the end of the file. */
int bq_gguf_open(const char* path, bq_gguf** out);
void bq_gguf_close(bq_gguf* g);
int64_t bq_gguf_n_tensors(const bq_gguf* g);
int64_t bq_gguf_find(const bq_gguf* g, const char* name);  /* -1 if absent */
int bq_gguf_tensor_info(const bq_gguf* g, int64_t i, bq_gguf_tensor* out);
/* numeric (types 0-7, 10-12) and string (type 8) metadata; BQ_UNSUPPORTED if
 * the key is absent or of another type */
int bq_gguf_kv_num(const bq_gguf* g, const char* key, double* out);
int bq_gguf_kv_str(const bq_gguf* g, const char* key, const char** out);
/* n bytes of tensor i from byte `off` of its data into host memory */
int bq_gguf_read(const bq_gguf* g, int64_t i, void* dst, size_t n, uint64_t off);
/* Stream 2-D tensor i into device memory `raw` (nbytes) through two pinned
 * staging slots (file reads overlap the copies), then on the same stream:
 *   Q5_K: rep/rep_min given -> W144 + Dm (bq_repack_q5k);
 *   Q6_K: rep given -> W160 (bq_repack_q6k);
 *   BF16: rep required -> Q8S logits head (bq_quantize_q8s); raw is the BF16
 *         staging buffer and may be reused once the stream has passed it.
 * *w (optional) receives the descriptor: bq_weight of the Q5_K / Q6_K tensor,
 * or for BF16 raw = the Q8S matrix with ggml_type 8 (Q8_0), for bq_gemv_q8s.
 * Returns when the file has been read and the copies are done; the repack is
 * enqueued.  The staging slots (2 x 64 MiB pinned) are allocated on the first
 * call and freed by bq_gguf_close.  BQ_UNSUPPORTED: not 2-D, another type, or
 * K % 256 != 0. */
int bq_gguf_load(bq_gguf* g, int64_t i, void* raw, void* rep, void* rep_min, bq_weight* w, bq_stream_t st);

/* ---- decode step -------------------------------------------------------------
 * The per-token decode launch sequence of the reference's forward_launch
 * (bruce.cu:7902-8037) over a caller's block list, eagerly or as one captured
 * HIP graph (capture_graph :8046-8055, replayed per token as bruce_decode_step
 * does, :8246-8252).  With rows = 2..8 it is the speculative-verify step over
 * `rows` tokens with every row's logits (forward_batch_impl :7610-7843 with
 * all_logits), captured once per row count as capture_verify_graphs does
 * (:7877-7900) and replayed by verify_launch (:7862-7875); the argmax that
 * follows there is the caller's.  With rows = 9..BQ_MAX_STEP_ROWS it is a
 * prompt chunk, forward_batch_impl as bruce_prefill_chunk calls it
 * (:8274-8291; the reference's chunks are at most MBUF = 512 rows, :1058):
 * the projections run on the prefill GEMMs (bq_gemm_b_fused / bq_gemm_b with
 * the step's xdh and work), and only the last row's logits are computed
 * (:7833-7836), into logits [vocab].  Per block, in the reference's order:
 *   norm_before: x = norm(x + input_h) -> q8                      (k_add_norm :7914)
 *   attention block: QKV GEMV over the q8 rows (bq_verify_fused over the Q5_K
 *     parts, single-row / multi-row GEMVs for others), the caller's attention
 *     hook, gate norm of attn_out by attn_gate -> q8, O GEMV -> proj (:7915-7993)
 *   FFN block: gate+up GEMV, silu*mul norm -> q8, down GEMV -> proj (:7994-8012)
 *   x = resid(x, proj, alpha) -> q8                               (k_resid :8017)
 *   norm_after: x = norm(x) -> q8                                 (k_norm :8022)
 *     (on a block with norm_after, its resid and this norm run as one launch,
 *     bit-identical to the two)
 * then the logits of every row: the Q8_0 head (head_q8s, bq_gemv_q8s with
 * head_rs) or a k-quant head (head)                                (:8026-8032).
 * fold = 1 (rows = 1 only; BQ_UNSUPPORTED with more) runs the gate norm
 * inside the O GEMV and the silu*mul inside the gate+up epilogue with its norm
 * inside the down GEMV (bq_gemv_norm_fused, bq_gate_up_silu; 2 launches fewer
 * per block pair, outputs equal to rounding).  fold = 2 (rows = 1 only)
 * also runs the resid -> q8 of each block that an attention block follows
 * inside that block's QKV GEMV (bq_gemv_norm_fused with BQ_OP_RESID over its
 * Q5_K parts; its q8 row is written out for any other part), and an
 * attention block's norm_before the same way (BQ_OP_ADD), which writes
 * the new residual row to the other of x and x_alt; the other updates run as
 * their own launches into x, so x holds the result as in the other modes
 * (needs x_alt; 1 launch fewer per layer than fold = 1).  The attention
 * kernels are the caller's: `attention(user, block, st)` must enqueue them
 * on st (and only there) and write attn_out; NULL leaves attn_out as it is.
 * Every buffer holds `rows` rows, row-major: x, input_h, proj
 * [rows][n_embd]; attn_out, attn_gate [rows][n_attn]; qkv_out[p] [rows][N_p];
 * ffn_g, ffn_u [rows][n_ff] (with fold >= 1 ffn_u, optional, is scratch: when
 * attn_gate is the start of a Q5_K QKV part's output, the QKV launch also
 * writes that part times sgate there, or for a Q5_K O its sigmoid
 * denominator 1 + exp(-gate * sgate), and the O GEMV's gate norm reads it
 * instead of attn_gate and sgate, same results); logits
 * [rows][vocab] (a prompt chunk: [vocab]); xq/xd/xsum hold the q8 rows of the
 * widest operand, rows x max(n_embd, n_attn, n_ff) values.  x is updated in
 * place.  A graph captures the pointers and the row count it is created with:
 * replays read and write the same buffers. */
enum { BQ_BLOCK_ATTN = 0, BQ_BLOCK_FFN = 1 };
typedef struct bq_decode_block {
    int kind;                     /* BQ_BLOCK_ATTN or BQ_BLOCK_FFN */
    int norm_before, norm_after;  /* loop start / end of the reference's recurrence */
    const float* alpha;           /* resid blend [n_embd] */
    /* attention block */
    const bq_weight* qkv; int n_qkv;   /* q, k, gate, v parts (1..4) sharing K = n_embd */
    float* const* qkv_out;
    const float* attn_out;        /* written by the hook; [n_attn] */
    const float* attn_gate;       /* gate pre-activation [n_attn] (usually one of qkv_out) */
    const float* sgate;           /* [n_attn] */
    int n_attn;
    const bq_weight* o;           /* K = n_attn, N = n_embd */
    /* FFN block */
    const bq_weight* gate; const bq_weight* up;   /* K = n_embd, N = n_ff */
    const float* s_gate; const float* s_up;       /* [n_ff] */
    const bq_weight* down;                        /* K = n_ff, N = n_embd */
    int n_ff;
} bq_decode_block;
typedef struct bq_decode_step {
    int n_blocks;
    const bq_decode_block* blocks;
    int n_embd;
    int fold;
    float* x;                     /* residual stream [n_embd]; its q8 row must be current in xq/xd/xsum */
    const float* input_h;         /* for norm_before */
    int8_t* xq; float* xd; int32_t* xsum;
    float* proj; float* ffn_g; float* ffn_u;
    void (*attention)(void* user, int block, bq_stream_t st);
    void* user;
    const void* head_q8s; const float* head_rs; const bq_weight* head;  /* one of the two heads, or neither */
    int vocab;
    float* logits;
    int rows;                     /* tokens per step, 1..BQ_MAX_STEP_ROWS (0 means 1) */
    float* x_alt;                 /* fold = 2: a second residual row [n_embd], not x */
    /* rows > 8: the prefill GEMMs' xdh scratch [rows][max K/32] fp16 and K-split
     * workspace (bq_gemm_b; NULL / 0: the raw-Q5_K tier / no split) */
    uint16_t* xdh;
    void* work;
    size_t work_bytes;
} bq_decode_step;
/* Enqueue one token's launch sequence on st (stream-ordered, allocates nothing). */
int bq_decode_enqueue(const bq_decode_step* s, bq_stream_t st);
/* Capture bq_decode_enqueue into a HIP graph and instantiate it: a set-up
 * call (synchronises st, allocates the graph), outside any capture. */
typedef struct bq_decode_graph bq_decode_graph;
int bq_decode_graph_create(const bq_decode_step* s, bq_stream_t st, bq_decode_graph** g);
int bq_decode_graph_launch(const bq_decode_graph* g, bq_stream_t st);  /* one token */
void bq_decode_graph_destroy(bq_decode_graph* g);

/* ---- tooling ---------------------------------------------------------------
 * No counterpart in the reference (its harnesses bracket launches with
 * cudaEventRecord, tools/gemvbench.cu:360-371).  Times the calling thread's
 * next GEMV/GEMM kernel dispatch: the two hipEvent_t handles are recorded at
 * the dispatch's start and end (hipExtLaunchKernelGGL), so their elapsed time
 * is the kernel's own duration.  Used by the benchmark driver. */
int bq_time_next_launch(void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif
#endif /* BQ_H */
