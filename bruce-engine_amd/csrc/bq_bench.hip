// bq_bench.hip -- native timing driver for bench.py (libbq_bench.so).
//
// Runs the decode / prefill steps through libbq's public C ABI in a tight host
// loop on one stream and times them with HIP events: the whole timed region
// (start/end events after a device synchronisation) and, per step, the
// dominant kernels' own durations (bq_time_next_launch: events recorded at the
// dispatch's start and end, the same interval a kernel trace reports).
// The same launch sequence is what the reference's decode loop issues per
// token for one FFN block (bruce.cu:7992-8011): quantize the block input,
// fused gate+up GEMV, quantize the down-projection input, down GEMV.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>
#include <vector>

#include "../../include/bq.h"

namespace {

struct EventPool {
    std::vector<hipEvent_t> ev;
    explicit EventPool(size_t n) : ev(n, nullptr) {
        for (auto& e : ev) (void)hipEventCreate(&e);
    }
    ~EventPool() {
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

float elapsed(hipEvent_t a, hipEvent_t b) {
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, a, b);
    return ms;
}

// Streaming-read probe: every byte of `bytes` read once with 16-byte loads
// (4 per thread, 256 threads per workgroup, consecutive lanes on consecutive
// 16-byte chunks), reduced to nothing (a never-taken store keeps the loads).
__global__ void __launch_bounds__(256) k_stream(const uint4* __restrict__ src, size_t n16, uint32_t* sink) {
    const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t j = base + 256 * i;
        if (j < n16) {
            const uint4 v = src[j];
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// The same bytes read by a persistent grid (gridDim = 4 workgroups per CU):
// workgroup b reads 16 KB chunks b, b + gridDim, ... with 4 loads per thread
// in flight per iteration.  Faster than k_stream at the GEMV launch sizes
// (fewer workgroups to dispatch, every chunk of one round adjacent).
__global__ void __launch_bounds__(256) k_stream_gs(const uint4* __restrict__ src, size_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 1024;
    for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n16; base += stride) {
        uint4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t j = base + 256 * i;
            v[i] = j < n16 ? src[j] : uint4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// A kernel that does nothing: its dispatch-event duration is the fixed cost
// every launch pays (dispatch, wave launch, end-of-kernel completion).
__global__ void __launch_bounds__(256) k_empty(uint32_t* sink) {
    if (threadIdx.x == 1023) sink[0] = 1;  // never true: keeps the kernel
}

// Issue-rate probes: every wave runs `iters` rounds of 4 (matrix) or 8 (VALU)
// independent chains of one instruction (no memory traffic; one operand changes per round), 8 waves
// per CU.  W selects the instruction.
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef int i32x16v __attribute__((ext_vector_type(16)));
typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef float f32x32v __attribute__((ext_vector_type(32)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
template <int W>
__global__ void __launch_bounds__(256) k_inst_rate(int iters, uint32_t* sink) {
    uint32_t t = 0;
    if constexpr (W == 0 || W == 1) {  // int8 32x32x32 / 32x32x16
        i32x4v a = {(int)threadIdx.x, 3, 5, 7}, b = {1, 2, 3, (int)threadIdx.x};
        long a2 = threadIdx.x, b2 = 3;
        i32x16v c[4] = {};
        for (int it = 0; it < iters; ++it) {
            a.x += 1;
            a2 += 1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (W == 0) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
                else c[k] = __builtin_amdgcn_mfma_i32_32x32x16_i8(a2, b2, c[k], 0, 0, 0);
            }
        }
        for (int k = 0; k < 4; ++k)
            for (int i = 0; i < 16; ++i) t ^= (uint32_t)c[k][i];
    } else if constexpr (W == 2) {  // fp16 32x32x16
        f16x8v a = {(_Float16)threadIdx.x, 1, 2, 3, 4, 5, 6, 7}, b = {1, 2, 3, 4, 5, 6, 7, 8};
        f32x16v c0 = {0.f}, c1 = {0.f}, c2 = {0.f}, c3 = {0.f};
        for (int it = 0; it < iters; ++it) {
            a[0] += (_Float16)1;
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
        }
        float f = 0.f;
        for (int i = 0; i < 16; ++i) f += c0[i] + c1[i] + c2[i] + c3[i];
        t = f == 1.2345f ? 0x7fffffffu : 0u;
    } else if constexpr (W == 3) {  // fp32 32x32x1, two blocks (the GEMMs' scale outer product)
        float a = threadIdx.x, b = 3.f;
        f32x32v c0 = {0.f}, c1 = {0.f}, c2 = {0.f}, c3 = {0.f};
        for (int it = 0; it < iters; ++it) {
            a += 1.f;
            c0 = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c3, 0, 0, 0);
        }
        float f = 0.f;
        for (int i = 0; i < 32; ++i) f += c0[i] + c1[i] + c2[i] + c3[i];
        t = f == 1.2345f ? 0x7fffffffu : 0u;
    } else if constexpr (W == 4) {  // int8 4x4x4, 16 blocks (the multi-row GEMV dots)
        int a = threadIdx.x, b = 3;
        i32x4v c[4] = {};
        for (int it = 0; it < iters; ++it) {
            a += 1;
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = __builtin_amdgcn_mfma_i32_4x4x4i8(a, b, c[k], 0, 0, 0);
        }
        for (int k = 0; k < 4; ++k)
            for (int i = 0; i < 4; ++i) t ^= (uint32_t)c[k][i];
    } else if constexpr (W == 5) {  // fp32 FMA (VALU; 8 chains, so latency does not limit)
        float a = threadIdx.x, c[8] = {0.f, 1.f, 2.f, 3.f, 4.f, 5.f, 6.f, 7.f};
        for (int it = 0; it < iters; ++it) {
            a += 1.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) c[k] = __builtin_fmaf(a, 1.0001f, c[k]);
        }
        for (int k = 0; k < 8; ++k) t ^= __builtin_bit_cast(uint32_t, c[k]);
    } else {  // int32 -> fp32 convert (VALU; paired with an add per chain, 8 chains)
        int a = threadIdx.x - 7;
        float c[8] = {0.f, 1.f, 2.f, 3.f, 4.f, 5.f, 6.f, 7.f};
        for (int it = 0; it < iters; ++it) {
            a += 1;
#pragma unroll
            for (int k = 0; k < 8; ++k) c[k] += (float)(a ^ k);
        }
        for (int k = 0; k < 8; ++k) t ^= __builtin_bit_cast(uint32_t, c[k]);
    }
    if (t == 0x7fffffffu) sink[threadIdx.x & 3] = t;
}

}  // namespace

extern "C" {

// Issue rate of one instruction (k_inst_rate<which>): out[0] = the launch's
// duration (ms), out[1] = instructions issued per SIMD.
int bqb_inst_rate(int which, int blocks, int iters, uint32_t* sink, bq_stream_t st, double* out) {
    void (*k)(int, uint32_t*) = nullptr;
    switch (which) {
        case 0: k = k_inst_rate<0>; break;
        case 1: k = k_inst_rate<1>; break;
        case 2: k = k_inst_rate<2>; break;
        case 3: k = k_inst_rate<3>; break;
        case 4: k = k_inst_rate<4>; break;
        case 5: k = k_inst_rate<5>; break;
        case 6: k = k_inst_rate<6>; break;
        default: return -1;
    }
    int cus = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
    hipLaunchKernelGGL(k, dim3(blocks), dim3(256), 0, (hipStream_t)st, iters / 10 + 1, sink);
    EventPool pool(2);
    (void)hipDeviceSynchronize();
    hipExtLaunchKernelGGL(k, dim3(blocks), dim3(256), 0, (hipStream_t)st, pool.ev[0], pool.ev[1], 0, iters, sink);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    // waves per SIMD x rounds x chains (4 for the matrix instructions, 8 for
    // the VALU ones; the convert probe counts convert + add)
    out[1] = (double)blocks * 4 / (4.0 * (cus > 0 ? cus : 256)) * iters * (which == 5 ? 8 : which == 6 ? 16 : 4);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Dispatch-event duration of an empty kernel of `blocks` x 256 threads:
// out[0] = summed over `steps` back-to-back launches, out[1] = summed over
// `steps` launches each after a device synchronisation (ms).
int bqb_empty(int steps, int blocks, uint32_t* sink, bq_stream_t st, double* out) {
    EventPool pool((size_t)steps * 2);
    hipLaunchKernelGGL(k_empty, dim3(blocks), dim3(256), 0, (hipStream_t)st, sink);
    (void)hipDeviceSynchronize();
    for (int i = 0; i < steps; ++i)
        hipExtLaunchKernelGGL(k_empty, dim3(blocks), dim3(256), 0, (hipStream_t)st, pool.ev[2 * i],
                              pool.ev[2 * i + 1], 0, sink);
    (void)hipDeviceSynchronize();
    out[0] = 0;
    for (int i = 0; i < steps; ++i) out[0] += elapsed(pool.ev[2 * i], pool.ev[2 * i + 1]);
    out[1] = 0;
    for (int i = 0; i < steps; ++i) {
        hipExtLaunchKernelGGL(k_empty, dim3(blocks), dim3(256), 0, (hipStream_t)st, pool.ev[0], pool.ev[1], 0, sink);
        (void)hipDeviceSynchronize();
        out[1] += elapsed(pool.ev[0], pool.ev[1]);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The HBM streaming-read ceiling for one launch of `bytes`: `steps` timed
// launches of k_stream (pattern 0) or k_stream_gs (pattern 1) over nbufs
// rotating buffers (so the 256 MB last-level cache cannot serve them), each
// bracketed by dispatch events.  out[0] = summed kernel durations (ms).
int bqb_stream(int pattern, int steps, int warmup, int nbufs, const void* const* bufs, size_t bytes, uint32_t* sink,
               bq_stream_t st, double* out) {
    const size_t n16 = bytes / 16;
    int cus = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
    auto k = pattern == 0 ? k_stream : k_stream_gs;
    const dim3 grid(pattern == 0 ? (unsigned)((n16 + 1023) / 1024)
                                 : (unsigned)std::min<size_t>((n16 + 1023) / 1024, 4 * (size_t)(cus > 0 ? cus : 256)));
    for (int i = 0; i < warmup; ++i)
        hipLaunchKernelGGL(k, grid, dim3(256), 0, (hipStream_t)st, (const uint4*)bufs[i % nbufs], n16, sink);
    EventPool pool((size_t)steps * 2);
    (void)hipDeviceSynchronize();
    for (int i = 0; i < steps; ++i)
        hipExtLaunchKernelGGL(k, grid, dim3(256), 0, (hipStream_t)st, pool.ev[2 * i], pool.ev[2 * i + 1], 0,
                              (const uint4*)bufs[i % nbufs], n16, sink);
    (void)hipDeviceSynchronize();
    double t = 0;
    for (int i = 0; i < steps; ++i) t += elapsed(pool.ev[2 * i], pool.ev[2 * i + 1]);
    out[0] = t;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Dense int8 MFMA throughput: every wave runs `iters` rounds of four
// independent v_mfma_i32_32x32x32_i8 chains (no memory traffic in the loop;
// one operand changes per round so nothing is hoisted), 8 waves per CU.
__global__ void __launch_bounds__(256) k_mfma_peak(int iters, uint32_t* sink) {
    typedef int i32x4v __attribute__((ext_vector_type(4)));
    typedef int i32x16v __attribute__((ext_vector_type(16)));
    i32x4v a = {(int)threadIdx.x, 3, 5, 7}, b = {1, 2, 3, (int)threadIdx.x};
    i32x16v c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    for (int it = 0; it < iters; ++it) {
        a.x += 1;
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    }
    int t = 0;
    for (int i = 0; i < 16; ++i) t += c0[i] ^ c1[i] ^ c2[i] ^ c3[i];
    if (t == 0x7fffffff) sink[threadIdx.x & 3] = (uint32_t)t;
}

// out[0] = the launch's duration (ms, dispatch events), out[1] = int8 ops
// (2 x 32 x 32 x 32 per MFMA)
int bqb_mfma_peak(int blocks, int iters, uint32_t* sink, bq_stream_t st, double* out) {
    hipLaunchKernelGGL(k_mfma_peak, dim3(blocks), dim3(256), 0, (hipStream_t)st, iters / 10 + 1, sink);
    EventPool pool(2);
    (void)hipDeviceSynchronize();
    hipExtLaunchKernelGGL(k_mfma_peak, dim3(blocks), dim3(256), 0, (hipStream_t)st, pool.ev[0], pool.ev[1], 0, iters,
                          sink);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    out[1] = (double)blocks * 4 * iters * 4 * 65536.0;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// One decode FFN step per iteration, weight set s = i % nsets (sets rotate so
// that the working set exceeds the 256 MB last-level cache).
// mode 0: nsets consecutive steps (sets 0..nsets-1) are captured into one
//         HIP graph and the timed region replays it -- the reference replays
//         one captured CUDA graph per decoded token, i.e. per layer stack
//         (bruce.cu:8246-8252).
//         out[0] = timed region (ms, `steps` steps).
// mode 1: direct launches, the two GEMV kernels timed with dispatch events.
//         out[0] = timed region, out[1] / out[2] = summed gate+up / down
//         kernel durations (ms).
// mode | 2: the same step with bq_gemv_q8_fused (each GEMV quantizes its own
//         fp32 input: two launches per step instead of four); the q8 rows are
//         still written out.
int bqb_decode_ffn(int mode, int steps, int warmup, int nsets, const bq_weight* gate, const bq_weight* up,
                   const bq_weight* down, const float* x, const float* t, int8_t* xq, float* xd,
                   int32_t* xs, int8_t* tq, float* td, int32_t* ts, float* yg, float* yu, float* yd,
                   bq_stream_t st, double* out) {
    const int K = gate[0].K, KD = down[0].K;
    const bool fused = (mode & 2) != 0;
    mode &= 1;
    auto step = [&](int i, hipEvent_t g0, hipEvent_t g1, hipEvent_t d0, hipEvent_t d1,
                    bq_stream_t s_) -> int {
        const int s = i % nsets;
        float* ys[2] = {yg, yu};
        const bq_weight* ws[2] = {&gate[s], &up[s]};
        if (fused) {
            if (g0) bq_time_next_launch(g0, g1);
            int r = bq_gemv_q8_fused(ys, ws, 2, x, xq, xd, xs, s_);
            if (r) return r;
            float* yd_[1] = {yd};
            const bq_weight* wd[1] = {&down[s]};
            if (d0) bq_time_next_launch(d0, d1);
            return bq_gemv_q8_fused(yd_, wd, 1, t, tq, td, ts, s_);
        }
        int r = bq_quantize_q8(x, 1, K, xq, xd, xs, nullptr, s_);
        if (r) return r;
        if (g0) bq_time_next_launch(g0, g1);
        r = bq_verify_fused(ys, ws, 2, 1, xq, xd, xs, 0, s_);
        if (r) return r;
        r = bq_quantize_q8(t, 1, KD, tq, td, ts, nullptr, s_);
        if (r) return r;
        if (d0) bq_time_next_launch(d0, d1);
        return bq_gemv(yd, &down[s], tq, td, ts, s_);
    };
    for (int i = 0; i < warmup; ++i)
        if (int r = step(i, nullptr, nullptr, nullptr, nullptr, st)) return r;
    out[0] = out[1] = out[2] = 0.0;
    if (mode == 0) {
        // one graph holds nsets consecutive steps (one per weight set, like a
        // token's layer stack); a second graph holds the steps % nsets tail
        hipStream_t cs;
        if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) return -1;
        auto capture = [&](int n, hipGraphExec_t* ex) -> int {
            *ex = nullptr;
            if (n == 0) return 0;
            hipGraph_t g;
            (void)hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
            int r = 0;
            for (int i = 0; i < n && !r; ++i) r = step(i, nullptr, nullptr, nullptr, nullptr, (bq_stream_t)cs);
            if (hipStreamEndCapture(cs, &g) != hipSuccess || r) return r ? r : -1;
            const hipError_t e = hipGraphInstantiate(ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            return e == hipSuccess ? 0 : -1;
        };
        hipGraphExec_t full, tail;
        if (int r = capture(nsets, &full)) return r;
        if (int r = capture(steps % nsets, &tail)) return r;
        (void)hipGraphLaunch(full, (hipStream_t)st);  // warm the graph
        EventPool pool(2);
        (void)hipDeviceSynchronize();
        (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
        for (int i = 0; i < steps / nsets; ++i) (void)hipGraphLaunch(full, (hipStream_t)st);
        if (tail) (void)hipGraphLaunch(tail, (hipStream_t)st);
        (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
        (void)hipDeviceSynchronize();
        out[0] = elapsed(pool.ev[0], pool.ev[1]);
        (void)hipGraphExecDestroy(full);
        if (tail) (void)hipGraphExecDestroy(tail);
        (void)hipStreamDestroy(cs);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    EventPool pool((size_t)steps * 4 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        hipEvent_t* e = &pool.ev[2 + 4 * (size_t)i];
        if (int r = step(i, e[0], e[1], e[2], e[3], st)) return r;
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    double g = 0, d = 0;
    for (int i = 0; i < steps; ++i) {
        hipEvent_t* e = &pool.ev[2 + 4 * (size_t)i];
        g += elapsed(e[0], e[1]);
        d += elapsed(e[2], e[3]);
    }
    out[1] = g;
    out[2] = d;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Prefill GEMM: `steps` launches of try_launch_mmq over the same inputs (no
// K-split workspace: the config 4 launches fill the GPU unsplit).
//   out[0] = timed region (ms), out[1] = sum of per-launch event times (ms).
// Prefill GEMM timing through bq_try_mmq with the caller's K-split workspace
// (work, work_bytes; NULL / 0: none).  Per call, the GEMM kernel is bracketed
// by its dispatch events and one more event is recorded after the call, so
// out[1] = summed GEMM kernel durations and out[2] = summed call durations
// from the GEMM kernel's start to the end of the call (the leftover-tile sum,
// when the launch splits, included); the fill_xdh pre-pass of the W144 path
// runs before the GEMM kernel and is in neither.  out[0] = the whole region.
int bqb_gemm(int steps, int warmup, const bq_weight* w, int M, const int8_t* xq, const float* xd,
             const int32_t* xs, uint16_t* xdh, float* y, void* work, size_t work_bytes, bq_stream_t st,
             double* out) {
    float* ys[1] = {y};
    const bq_weight* ws[1] = {w};
    for (int i = 0; i < warmup; ++i)
        if (int r = bq_try_mmq(ys, ws, 1, M, xq, xd, xs, xdh, work, work_bytes, st)) return r;
    EventPool pool((size_t)steps * 3 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        hipEvent_t* e = &pool.ev[2 + 3 * (size_t)i];
        bq_time_next_launch(e[0], e[1]);
        if (int r = bq_try_mmq(ys, ws, 1, M, xq, xd, xs, xdh, work, work_bytes, st)) return r;
        (void)hipEventRecord(e[2], (hipStream_t)st);
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    double k = 0, c = 0;
    for (int i = 0; i < steps; ++i) {
        const hipEvent_t* e = &pool.ev[2 + 3 * (size_t)i];
        k += elapsed(e[0], e[1]);
        c += elapsed(e[0], e[2]);
    }
    out[1] = k;
    out[2] = c;
    return 0;
}

// Single-kernel timing helper: `steps` launches of one GEMV entry point with
// rotating weights (gemv over nsets weights, rows activation rows).
int bqb_gemv_rows(int steps, int warmup, int nsets, const bq_weight* w, int rows, const int8_t* xq,
                  const float* xd, const int32_t* xs, float* y, bq_stream_t st, double* out) {
    auto launch = [&](int i) -> int {
        float* ys[1] = {y};
        const bq_weight* wp[1] = {&w[i % nsets]};
        if (w[0].ggml_type == BQ_TYPE_Q5_K) return bq_verify_fused(ys, wp, 1, rows, xq, xd, xs, 0, st);
        if (w[0].rep) return bq_gemm_q6k_dp(y, wp[0], rows, xq, xd, 0, st);
        return bq_gemm_q6k_raw(y, wp[0], rows, xq, xd, 0, st);
    };
    for (int i = 0; i < warmup; ++i)
        if (int r = launch(i)) return r;
    EventPool pool((size_t)steps * 2 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        bq_time_next_launch(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
        if (int r = launch(i)) return r;
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    double k = 0;
    for (int i = 0; i < steps; ++i) k += elapsed(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
    out[1] = k;
    return 0;
}

// Fused quantize + GEMV: `steps` launches of bq_gemv_q8_fused over nparts
// matrices, weight set s = i % nsets (w = [nsets][nparts]); out[1] = sum of
// the kernels' own durations (ms), out[0] = timed region.
int bqb_gemv_fused(int steps, int warmup, int nsets, int nparts, const bq_weight* w, const float* x,
                   float* const* ys, bq_stream_t st, double* out) {
    auto launch = [&](int i) -> int {
        const bq_weight* wp[4];
        for (int p = 0; p < nparts; ++p) wp[p] = &w[(i % nsets) * nparts + p];
        return bq_gemv_q8_fused(ys, wp, nparts, x, nullptr, nullptr, nullptr, st);
    };
    for (int i = 0; i < warmup; ++i)
        if (int r = launch(i)) return r;
    EventPool pool((size_t)steps * 2 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        bq_time_next_launch(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
        if (int r = launch(i)) return r;
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    double k = 0;
    for (int i = 0; i < steps; ++i) k += elapsed(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
    out[1] = k;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Q8_0 logits head: `steps` launches of bq_gemv_q8s, weight copy s = i % nsets.
// out[0] = timed region (ms), out[1] = sum of the kernels' own durations (ms).
int bqb_q8s(int steps, int warmup, int nsets, const void* const* ws, int K, int N, int rows, const int8_t* xq,
            const float* xd, const float* rs, float* y, bq_stream_t st, double* out) {
    for (int i = 0; i < warmup; ++i)
        if (int r = bq_gemv_q8s(y, ws[i % nsets], xq, xd, K, N, rows, rs, st)) return r;
    EventPool pool((size_t)steps * 2 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        bq_time_next_launch(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
        if (int r = bq_gemv_q8s(y, ws[i % nsets], xq, xd, K, N, rows, rs, st)) return r;
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    double k = 0;
    for (int i = 0; i < steps; ++i) k += elapsed(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
    out[1] = k;
    return 0;
}

// q8 producers: `steps` launches of one norm op over `rows` rows of n values
// (op 0 norm, 1 add, 2 resid, 3 gate, 4 silu*mul; buffers a..d as the op
// reads them, out may be NULL).  out_t[0] = timed region (ms), out_t[1] =
// sum of the kernels' own durations (ms).
int bqb_norm(int op, int steps, int warmup, float* out, float* a, const float* b, const float* c,
             const float* d, int rows, int n, int8_t* xq, float* xd, int32_t* xs, bq_stream_t st,
             double* out_t) {
    auto launch = [&]() -> int {
        switch (op) {
            case 0: return bq_norm_q8(out, a, rows, n, xq, xd, xs, st);
            case 1: return bq_add_norm_q8(a, b, rows, n, xq, xd, xs, st);
            case 2: return bq_resid_q8(a, b, c, rows, n, xq, xd, xs, st);
            case 3: return bq_gate_norm_q8(out, a, b, c, rows, n, xq, xd, xs, st);
            default: return bq_silu_mul_norm_q8(out, a, b, c, d, rows, n, xq, xd, xs, st);
        }
    };
    for (int i = 0; i < warmup; ++i)
        if (int r = launch()) return r;
    EventPool pool((size_t)steps * 2 + 2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) {
        bq_time_next_launch(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
        if (int r = launch()) return r;
    }
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out_t[0] = elapsed(pool.ev[0], pool.ev[1]);
    double k = 0;
    for (int i = 0; i < steps; ++i) k += elapsed(pool.ev[2 + 2 * i], pool.ev[3 + 2 * i]);
    out_t[1] = k;
    return 0;
}

// Whole-stack decode weight stream: per token, for each of
// `nlayers` layers, QKV, O, fused gate+up and down GEMVs, then the lm_head --
// each one a bq_gemv_q8_fused launch that quantizes its fp32 input row (the
// q8 rows are written out, as the reference's norm kernels do).  The token's
// launches are captured once into a HIP graph (the reference replays one graph
// per decoded token, bruce.cu:8246-8252) and the timed region replays it
// `steps` times.  w = [nlayers][5] weights (qkv, o, gate, up, down), inputs
// x (K), a (KO), t (FF), outputs y (>= max N), xq/xd/xs scratch for the
// largest K.  out[0] = timed region (ms).
int bqb_stack(int steps, int warmup, int nlayers, const bq_weight* w, const bq_weight* lm_head, const float* x,
              const float* a, const float* t, float* y0, float* y1, int8_t* xq, float* xd, int32_t* xs,
              bq_stream_t st, double* out) {
    hipStream_t cs;
    if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) return -1;
    auto token = [&](bq_stream_t s_) -> int {
        for (int l = 0; l < nlayers; ++l) {
            const bq_weight* lw = w + 5 * l;
            float* ys[2] = {y0, y1};
            const bq_weight* p1[1] = {&lw[0]};
            if (int r = bq_gemv_q8_fused(ys, p1, 1, x, xq, xd, xs, s_)) return r;          // QKV
            const bq_weight* p2[1] = {&lw[1]};
            if (int r = bq_gemv_q8_fused(ys, p2, 1, a, xq, xd, xs, s_)) return r;          // O
            const bq_weight* p3[2] = {&lw[2], &lw[3]};
            if (int r = bq_gemv_q8_fused(ys, p3, 2, x, xq, xd, xs, s_)) return r;          // gate + up
            const bq_weight* p4[1] = {&lw[4]};
            if (int r = bq_gemv_q8_fused(ys, p4, 1, t, xq, xd, xs, s_)) return r;          // down
        }
        float* ys[1] = {y0};
        const bq_weight* pl[1] = {lm_head};
        return bq_gemv_q8_fused(ys, pl, 1, x, xq, xd, xs, s_);                             // lm_head
    };
    for (int i = 0; i < warmup; ++i)
        if (int r = token(st)) return r;
    hipGraph_t g;
    hipGraphExec_t ex;
    (void)hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    const int r = token((bq_stream_t)cs);
    if (hipStreamEndCapture(cs, &g) != hipSuccess || r) return r ? r : -1;
    if (hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess) return -1;
    (void)hipGraphDestroy(g);
    (void)hipGraphLaunch(ex, (hipStream_t)st);
    EventPool pool(2);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(pool.ev[0], (hipStream_t)st);
    for (int i = 0; i < steps; ++i) (void)hipGraphLaunch(ex, (hipStream_t)st);
    (void)hipEventRecord(pool.ev[1], (hipStream_t)st);
    (void)hipDeviceSynchronize();
    out[0] = elapsed(pool.ev[0], pool.ev[1]);
    (void)hipGraphExecDestroy(ex);
    (void)hipStreamDestroy(cs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
