// bq_internal.hpp -- host-side declarations shared by the libbq translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace bq {

constexpr int kMaxParts = 4;
constexpr int kGemvMaxK = 49152;  // GEMV / multi-row kernels: 16 K slices x 3 steps x 1024

// Up to four matrices that share K and the activation rows, concatenated along
// N (the reference's W0..W3 / Y0..Y3 / N0..N3 kernel arguments, bruce.cu:5815).
// tile0[p] = first tile index of part p; filled by the launcher.
struct PartTable {
    const void* W[kMaxParts];
    const void* aux[kMaxParts];  // per-part side array (Q5_K W144: Dm fp16)
    float* Y[kMaxParts];
    int N[kMaxParts];
    int tile0[kMaxParts];
    int nparts;
    int ntiles;
    int prio = 0;  // GEMV: raise the wave priority during the activation staging
    // one-row GEMV: part sp's outputs also go to ys scaled by ss (ys[row] =
    // y[row] * ss[row]); ys NULL: none
    int sp = 0;
    float* ys = nullptr;
    const float* ss = nullptr;
    int sden = 0;  // ys[row] = 1 + exp(-(y[row] * ss[row])) instead (the gate's sigmoid denominator)
};

enum class GemvKind { Q5K, Q6KRaw, Q6KRep };

// Optional per-launch timing (bq_time_next_launch): when set, the next GEMV /
// GEMM kernel of the calling thread is launched with hipExtLaunchKernelGGL,
// which records the two events at the dispatch's start and end.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchTiming& next_launch_timing();

// Optional scaled copy of one part's output for the calling thread's next
// one-row GEMV launch, the part named by its weight pointer (the decode
// step's attention gate: gate * sg, which the O GEMV's gate-norm producer
// then reads instead of the gate and sg rows).  Consumed by that launch.
struct ScaledCopy {
    const void* w = nullptr;
    float* y = nullptr;
    const float* s = nullptr;
    bool den = false;  // write the sigmoid denominator of the scaled value
};
ScaledCopy& next_scaled_copy();
// O GEMV with the gate norm over precomputed sigmoid denominators (kOpGateDen;
// bq_api.hip): y = W * q8(norm(a / den)); BQ_UNSUPPORTED when not taken
int gemv_gate_den_fused(float* y, const void* w_raw, int K, int N, const float* a, const float* den, void* st);
// CU count of the current device (set by the entry point's init; 256 before any)
int device_cus();

template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
    LaunchTiming& t = next_launch_timing();
    if (t.start) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, t.start, t.stop, 0, args...);
        t = LaunchTiming();
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    }
}

hipError_t launch_quant_q8(const float* x, int rows, int K, int8_t* xq, float* xd, int32_t* xsum,
                           uint16_t* xdh, hipStream_t st);
hipError_t launch_fill_xdh(const float* xd, const int32_t* xsum, int n, uint16_t* xdh, hipStream_t st);

// GEMV K split (bq_gemv.hip): steps per wave capped per shape class, then
// KS = K slices per row and SPS = steps per slice
int sps_cap(GemvKind kind, int K, long long N, int MR, bool fused);
void k_split(int K, int cap, int& KS, int& SPS);
// Fused quantize + GEMV of one fp32 activation row (K % 256 == 0, K <= 49152);
// xq/xd/xsum receive the q8 row when xq != NULL.
bool gemv_fused_supported(int K);
hipError_t launch_gemv_fused_q8(GemvKind kind, PartTable pt, int K, const float* x, int8_t* xq,
                                float* xd, int32_t* xsum, hipStream_t st);
// q8 producer (op as launch_norm_q8, K % 256 == 0, K <= 16384) + GEMV of the
// produced row in one launch; out (the emitted fp32 row) and xq/xd/xsum are
// optional outputs written by workgroup 0.  Bit-identical to launch_norm_q8
// followed by launch_gemv_fused_q8 on its fp32 output.
bool gemv_producer_supported(int K);
hipError_t launch_gemv_producer(GemvKind kind, PartTable pt, int K, int op, float* out, const float* a,
                                const float* b, const float* c, const float* d, int8_t* xq, float* xd,
                                int32_t* xsum, hipStream_t st);
size_t gemv_lds_bytes(GemvKind kind, int rows, int K);
hipError_t launch_gemv_silu_pair(GemvKind kind, PartTable pt, int K, const int8_t* xq, const float* xd,
                                 const int32_t* xsum, const float* sg, const float* su, float* h, hipStream_t st);
hipError_t launch_gemv(GemvKind kind, PartTable pt, int rows, int K, const int8_t* xq,
                       const float* xd, const int32_t* xsum, hipStream_t st);

hipError_t launch_repack_q5k(const void* raw, int K, int N, void* w144, uint16_t* dm, hipStream_t st);
hipError_t launch_repack_q6k(const void* raw, int K, int N, void* w160, hipStream_t st);

// prefill GEMMs (128-row weight tiles, int8 MFMA).  ws / ws_floats: the K-split
// workspace (nullptr: no split); mmq_ksplit gives the split a launch takes
// (stage_units: the raw tier, which splits at 128-value stages; tm: the
// token-tile height, 128 or the W144 kernel's 32).  cus: the CU count of the
// device the launch runs on (the workgroup slots every split choice counts).
int mmq_ksplit(int rows, int K, int ntot, bool stage_units, size_t ws_floats, int tm, int cus);
size_t mmq_tail_ws_floats(int rows, int K, int ntot, int cus);  // workspace of the Q5_K leftover-tile split
hipError_t launch_mmq_q5k_raw(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                              const int32_t* xsum, hipStream_t st, int cus, float* ws = nullptr,
                              size_t ws_floats = 0);
hipError_t launch_mmq_q5k_144(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                              const int32_t* xsum, uint16_t* xdh, hipStream_t st, int cus, float* ws = nullptr,
                              size_t ws_floats = 0);
hipError_t launch_mmq_q6k(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                          hipStream_t st, int cus, float* ws = nullptr, size_t ws_floats = 0);

// Q8_0 logits head (Q8S: 8 fp16 scales + 256 int8 per row and 256 values)
constexpr int kQ8SMaxK = 4096;  // the GEMV keeps K/1024 activation chunks per lane in registers
hipError_t launch_quant_q8s(const uint16_t* src, int K, int N, uint8_t* dst, hipStream_t st);
hipError_t launch_gemv_q8s(const void* W, int K, int N, int rows, const int8_t* xq, const float* xd,
                           const float* rs, float* y, hipStream_t st, int cus);

// q8 producers: elementwise op -> L2 norm -> q8 (op: 0 norm, 1 add, 2 resid,
// 3 gate, 4 silu*mul); n % 32 == 0, n <= kNormMaxN
enum NormOp { kOpNorm = 0, kOpAdd = 1, kOpResid = 2, kOpGate = 3, kOpSilu = 4,
              // resid -> q8 followed by the plain norm of its row in one launch
              // (the decode step's last resid and norm_after; launch_norm_q8 only)
              kOpResidNorm = 5,
              // the attention gate with its sigmoid denominators precomputed:
              // t = a / b (producer-fused GEMV only)
              kOpGateDen = 6 };
constexpr int kNormMaxN = 32768;
hipError_t launch_norm_q8(int op, float* out, const float* a, const float* b, const float* c,
                          const float* d, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
                          hipStream_t st);

}  // namespace bq
