/*
 * bq_oracle.h -- CPU restatement of the reference's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libbq.so, bq.py) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root; bruce.cu = engine/src/bruce.cu).
 *
 * Parity pinning (how each function is checked independently of itself):
 *   orc_h2f / orc_f2h_rn   exhaustive over all 65536 halves against numpy float16
 *   orc_q8_rows            closed-form invariants + special cases (tests/test_oracle.py)
 *   orc_q5k_scale          hand-built known-answer blocks from the GGUF layout + brute force
 *   orc_dequant_q5k/q6k    hand-built KAT blocks; independent numpy decoder in the tests
 *   orc_gemm_q5k/q6k       integer dots vs brute force over dequantized int codes,
 *                          the mmq_test.cu "y = K" KAT, linearity in xd, dmin = 0 case
 *   orc_repack_*           index-map restatement checked against dequant round trip
 *   orc_gemm_q5k_144       equals orc_gemm_q5k up to the fp16 rounding of the min term
 *   orc_quantize_q8s       codes and scales equal orc_q8_rows on the widened bf16 values
 *                          (scale = half_rn(xd)); hand-built layout KAT with numpy
 *                          float32/float16 arithmetic; round-trip bound |w - s*q| <= s/2
 *   orc_norm_rows          unit-L2 closed form (|v|^2 = ss/(ss+eps)), scale invariance,
 *                          alpha = 0 / 1 / sg = 0 special cases, scipy.special.expit
 *                          restatements of the gate / silu products (tests/test_norm_oracle.py)
 *   orc_gemv_q8s           float64 matmul of the dequantized operands (numpy, built from
 *                          a reshape of the block layout); "y = K" KAT; exact scaling in rs
 * None of the functions is "parity unpinned".
 */
#ifndef BQ_ORACLE_H
#define BQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic synthetic data ---------------------------------------- */
/* splitmix64 stream + Box-Muller; fills n floats N(mean, std). */
void orc_gaussian(uint64_t seed, float mean, float std, float* out, size_t n);

/* ---- fp16 ------------------------------------------------------------------ */
float orc_h2f(uint16_t h);          /* bruce.cu:4768-4781 (denormal-correct) */
uint16_t orc_f2h_rn(float f);       /* IEEE binary16 round-to-nearest-even */

/* ---- activation quantizer (bruce.cu:518-539, :1081-1108) ------------------- */
void orc_q8_rows(const float* x, int M, int K, int8_t* xq, float* xd, int32_t* xsum);
/* xdh = half(xd * xsum)  (bruce.cu:6598-6602) */
void orc_fill_xdh(const float* xd, const int32_t* xsum, size_t n, uint16_t* xdh);

/* ---- k-quant encoders (own design; the reference reads llama.cpp files) ---- */
void orc_quantize_q5k(const float* w, int N, int K, uint8_t* out);   /* 176 B / 256 */
void orc_quantize_q6k(const float* w, int N, int K, uint8_t* out);   /* 210 B / 256 */

/* ---- format decode --------------------------------------------------------- */
/* 6-bit scale/min of sub-block js from the 12 scale bytes (bruce.cu:368-381) */
void orc_q5k_scale(const uint8_t* scales12, int js, int* sc, int* m);
/* 5-bit code u of value k (0..255) in a block (bruce.cu:405-432, gemvbench.cu:390-396) */
int orc_q5k_code(const uint8_t* blk, int k);
/* 6-bit code q (0..63) of value k in a Q6_K block, and its int8 scale (bruce.cu:4795-4807) */
int orc_q6k_code(const uint8_t* blk, int k);
int orc_q6k_sc(const uint8_t* blk, int k);
void orc_dequant_q5k(const uint8_t* raw, int N, int K, float* out);   /* gemvbench.cu:373-403 */
void orc_dequant_q6k(const uint8_t* raw, int N, int K, float* out);   /* ref_np.py:106-123 */

/* ---- integer dots (sub_stats gemvbench.cu:405-430) ------------------------- */
/* dots[m][n][g]: sum over the 32 values of group g of code*xq  (Q5_K: u5, Q6_K: q6-32) */
void orc_dots_q5k(const uint8_t* raw, const int8_t* xq, int M, int N, int K, int32_t* dots);
/* Q6_K per 16-value group: dots16[m][n][K/16] */
void orc_dots16_q6k(const uint8_t* raw, const int8_t* xq, int M, int N, int K, int32_t* dots);

/* ---- GEMM references ------------------------------------------------------- */
/* y[m*N+n] = sum_g xd*(ds*dot - dm*xsum), evaluated in double from the exact fp32
 * ds = d*sc, dm = dmin*m (mmq_test.cu:269-294).  */
void orc_gemm_q5k(const uint8_t* raw, const int8_t* xq, const float* xd, const int32_t* xsum,
                  int M, int N, int K, double* y);
/* same formula in the reference's fp32 serial operation order (mmq_test.cu:283-288) */
void orc_gemm_q5k_f32(const uint8_t* raw, const int8_t* xq, const float* xd, const int32_t* xsum,
                      int M, int N, int K, float* y);
/* Q6_K: y = sum_{16-groups} xd[g32] * (d*sc16) * sum (q-32)*xq  (bruce.cu:4330-4345) */
void orc_gemm_q6k(const uint8_t* raw, const int8_t* xq, const float* xd,
                  int M, int N, int K, double* y);
void orc_gemm_q6k_f32(const uint8_t* raw, const int8_t* xq, const float* xd,
                      int M, int N, int K, float* y);
/* prepacked prefill: y = sum_g (ds*xd)*dot + sum_g f(Dm)*f(xdh)  (bruce.cu:6615-6790) */
void orc_gemm_q5k_144(const uint8_t* w144, const uint16_t* dm, const int8_t* xq, const float* xd,
                      const uint16_t* xdh, int M, int N, int K, double* y);

/* ---- load-time repacks ----------------------------------------------------- */
/* Q5_K -> W144 [K/128][N][144] + Dm [N][K/32] fp16  (bruce.cu:5756-5789) */
void orc_repack_q5k_144(const uint8_t* raw, int K, int N, uint8_t* w144, uint16_t* dm);
/* Q6_K -> [N][K/128][160]  (bruce.cu:4783-4811) */
void orc_repack_q6k_160(const uint8_t* raw, int K, int N, uint8_t* dst);

/* ---- Q8_0 logits head (bruce.cu:4400-4449, 4841-4867, 5159-5184) ---------- */
/* BF16 [N][K] -> Q8S: per (row, 256 values) 8 fp16 group scales (16 B) then
 * 256 int8 codes (256 B) = 272 B.  q8k_quant_host, bruce.cu:4843-4867. */
void orc_quantize_q8s(const uint16_t* bf16, int K, int N, uint8_t* dst);
/* y[m*N+n] = rs[n] * sum_g ws[n][g] * xd[m][g] * dot_g, in double (rs NULL = 1);
 * k_gemm_q8_logits, bruce.cu:4409-4449. */
void orc_gemv_q8s(const uint8_t* w, int K, int N, int M, const int8_t* xq, const float* xd,
                  const float* rs, double* y);

/* ---- q8 producers (bruce.cu:305-307, 541-641, 1110-1228) ------------------ */
/* The fp32 rows v = t * l2_scale(sum t^2, n) of the reference's norm kernels,
 * evaluated in double: op 0 norm(a), 1 norm(a + b), 2 resid (a = x, b = upd,
 * c = alpha[n]), 3 gate (a = aout, b = gate, c = sg[n]), 4 silu*mul (a = g,
 * b = u, c = sg[n], d = su[n]).  The q8 rows are orc_q8_rows of the result. */
void orc_norm_rows(int op, const float* a, const float* b, const float* c, const float* d, int rows, int n,
                   double* out);

#ifdef __cplusplus
}
#endif
#endif
