// bq_q8s.hip -- Q8_0 logits head: BF16 -> Q8S load-time conversion and the
// Q8S x q8 GEMV for 1..8 activation rows.
//
// Q8S layout (bruce.cu:4400-4407): per (row, 256 values) 272 bytes = 8 fp16
// group scales (16 B) followed by 256 int8 codes; rows are contiguous, so a
// row is K/256 * 272 bytes and every 16-byte code chunk is 16-byte aligned.
//
// Conversion (k_bf16_to_q8, bruce.cu:5159-5184; host twin q8k_quant_host
// :4843-4867): per 32 values d = amax*(1/127), id = d>0 ? 1/d : 0,
// q = clamp(rint(v*id), -127, 127), scale = half_rn(d).  The arithmetic is the
// activation quantizer's, so the lane-pair q8_quant16 is reused: each lane
// widens 16 bf16 values and writes 16 codes with one 16-byte store.
//
// GEMV (k_gemm_q8_logits, bruce.cu:4409-4449):
//   y[m][n] = rs[n] * sum_g ws[n][g] * xd[m][g] * dot(codes[n][g], xq[m][g]).
// A row has K/16 code chunks of 16 bytes.  Lane l of a wave owns chunks
// l, l+64, l+128, ... of every row, so its activation chunks (xq, xd) are loaded
// once into registers and reused for every row the wave visits.  A wave
// streams R rows per iteration: R*CPL 16-byte weight loads (each wave-wide load
// covers 1 KiB of consecutive code bytes) plus the matching 2-byte scale loads,
// which hit the same cache lines.  Per chunk: four v_dot4_i32_i8, one convert,
// one multiply-add; then a wave64 sum per (row, activation row).
#include <algorithm>

#include "bq_device.hpp"
#include "bq_internal.hpp"

namespace bq {

constexpr int kQ8S = 272;

__global__ void __launch_bounds__(256) k_quant_q8s(const uint16_t* __restrict__ src, int K,
                                                   long long nthreads, uint8_t* __restrict__ dst) {
    const long long tid = (long long)blockIdx.x * 256 + threadIdx.x;
    const bool live = tid < nthreads;
    f32x4 v[4];
    u32x4 a = u32x4{0u, 0u, 0u, 0u}, b = a;
    if (live) {
        a = *(const u32x4*)(src + tid * 16);
        b = *(const u32x4*)(src + tid * 16 + 8);
    }
    // bf16 -> fp32 is exact: the 16 bits become the top half of the word
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] = f32x4{as_float(w[2 * i] << 16), as_float(w[2 * i] & 0xFFFF0000u),
                     as_float(w[2 * i + 1] << 16), as_float(w[2 * i + 1] & 0xFFFF0000u)};
    uint32_t q[4];
    float d;
    int s;
    q8_quant16(v, q, d, s);
    if (!live) return;
    const long long e0 = tid * 16;
    const long long row = e0 / K;
    const int kin = (int)(e0 - row * K);
    uint8_t* blk = dst + (row * (K >> 8) + (kin >> 8)) * kQ8S;
    *(u32x4*)(blk + 16 + (kin & 255)) = u32x4{q[0], q[1], q[2], q[3]};
    if ((tid & 1) == 0) *(uint16_t*)(blk + 2 * ((kin & 255) >> 5)) = f2h_rn(d);
}

// Buffer resource over one row (gfx9 raw buffer: base, stride 0, byte count,
// word 3 = 0x00020000).  A wave-uniform base keeps the descriptor in SGPRs and
// every load is then base + 32-bit lane offset.
BQ_DEV __amdgpu_buffer_rsrc_t row_rsrc(const uint8_t* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

template <int M, int R, int CPL>
__global__ void __launch_bounds__(256)
k_gemv_q8s(const uint8_t* __restrict__ W, int K, int N, const int8_t* __restrict__ xq,
           const float* __restrict__ xd, const float* __restrict__ rs, float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int nchunk = K >> 4, nb = K >> 5;
    const size_t rowb = (size_t)(K >> 8) * kQ8S;
    u32x4 xv[M][CPL];
    float xs[M][CPL];
    // lanes past the row's last chunk (K % 1024 != 0) read chunk 0 of the row
    // (a valid address) and contribute zero: their xq and xd are zero
    uint32_t woff[CPL], soff[CPL];
    bool ok[CPL];  // chunk c of this lane exists
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int cc = c * 64 + lane;
        ok[c] = cc < nchunk;
        const int sb = ok[c] ? cc >> 4 : 0, p = ok[c] ? cc & 15 : 0;
        woff[c] = sb * kQ8S + 16 + p * 16;
        soff[c] = sb * kQ8S + 2 * (p >> 1);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            xv[m][c] = ok[c] ? *(const u32x4*)(xq + (size_t)m * K + cc * 16) : u32x4{0u, 0u, 0u, 0u};
            xs[m][c] = ok[c] ? xd[(size_t)m * nb + (cc >> 1)] : 0.f;
        }
    }
    // the wave index is uniform (readfirstlane), so row bases are scalar
    const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), tw = gridDim.x * 4;
    for (int r0 = gw * R; r0 < N; r0 += tw * R) {
        u32x4 wv[R][CPL];
        uint32_t sv[R][CPL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // a row past N keeps row N-1 as its base and an empty record range:
            // its loads return zero (results are not stored).  No branches, so
            // all R*CPL loads are in flight together.
            const int row = r0 + r;
            const __amdgpu_buffer_rsrc_t rs_ = row_rsrc(W + (size_t)min(row, N - 1) * rowb,
                                                        row < N ? (uint32_t)rowb : 0u);
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                wv[r][c] = __builtin_amdgcn_raw_buffer_load_b128(rs_, woff[c], 0, 0);
                sv[r][c] = __builtin_amdgcn_raw_buffer_load_b16(rs_, soff[c], 0, 0);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float acc[M];
#pragma unroll
            for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                // lanes past the last chunk read the row's group-0 scale (or 0
                // past N) and have xq = xd = 0, so they add exactly zero
                const float ws = h2f(sv[r][c]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    int dt = dot4((int)wv[r][c].x, (int)xv[m][c].x, 0);
                    dt = dot4((int)wv[r][c].y, (int)xv[m][c].y, dt);
                    dt = dot4((int)wv[r][c].z, (int)xv[m][c].z, dt);
                    dt = dot4((int)wv[r][c].w, (int)xv[m][c].w, dt);
                    acc[m] += ws * xs[m][c] * (float)dt;
                }
            }
            const int row = r0 + r;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float s = wave_sum_dpp63(acc[m]);
                if (lane == 63 && row < N) y[(size_t)m * N + row] = rs ? s * rs[row] : s;
            }
        }
    }
}

hipError_t launch_quant_q8s(const uint16_t* src, int K, int N, uint8_t* dst, hipStream_t st) {
    const long long nthreads = (long long)N * K / 16;
    if (nthreads == 0) return hipSuccess;
    const long long blocks = (nthreads + 255) / 256;
    hipLaunchKernelGGL(k_quant_q8s, dim3((unsigned)blocks), dim3(256), 0, st, src, K, nthreads, dst);
    return hipGetLastError();
}

namespace {
template <int M, int CPL>
hipError_t launch_q8s_mc(const uint8_t* W, int K, int N, const int8_t* xq, const float* xd, const float* rs,
                         float* y, hipStream_t st, int cus) {
    // rows per wave iteration: enough 16-byte loads in flight per wave while
    // the activation registers (M*CPL*5 VGPRs) grow with M.  At 7..8 rows the
    // occupancy is 3 waves/SIMD either way and two rows per wave keep more
    // bytes in flight (131072 x 3072: 7 / 8 rows 128 / 140 -> 121 / 131 us);
    // at 5..6 rows two rows per wave cost occupancy (6 rows 102 -> 113 us).
    // Activation rows in LDS instead of registers measured far slower (8 rows
    // 221 us: the per-use LDS reads bound the kernel).
    constexpr int R = M <= 2 ? 4 : (M <= 4 ? 2 : (M <= 6 ? 1 : 2));
    // persistent grid: as many workgroups as are resident at once, so no
    // partial second round of workgroups trails the stream
    static int per_cu = 0;
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv_q8s<M, R, CPL>, 256, 0) != hipSuccess || n < 1)
            n = 2;
        per_cu = n;
    }
    const long long want = ((long long)N + 4 * R - 1) / (4 * R);
    const int blocks = (int)std::min<long long>(want, (long long)cus * per_cu);
    launch_kernel((k_gemv_q8s<M, R, CPL>), dim3(blocks), dim3(256), 0, st, W, K, N, xq, xd, rs, y);
    return hipGetLastError();
}

template <int M>
hipError_t launch_q8s_m(int cpl, const uint8_t* W, int K, int N, const int8_t* xq, const float* xd,
                        const float* rs, float* y, hipStream_t st, int cus) {
    switch (cpl) {
        case 1: return launch_q8s_mc<M, 1>(W, K, N, xq, xd, rs, y, st, cus);
        case 2: return launch_q8s_mc<M, 2>(W, K, N, xq, xd, rs, y, st, cus);
        case 3: return launch_q8s_mc<M, 3>(W, K, N, xq, xd, rs, y, st, cus);
        default: return launch_q8s_mc<M, 4>(W, K, N, xq, xd, rs, y, st, cus);
    }
}
}  // namespace

hipError_t launch_gemv_q8s(const void* W, int K, int N, int rows, const int8_t* xq, const float* xd,
                           const float* rs, float* y, hipStream_t st, int cus) {
    const int cpl = (K / 16 + 63) / 64;
    const uint8_t* w = (const uint8_t*)W;
    switch (rows) {
        case 1: return launch_q8s_m<1>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 2: return launch_q8s_m<2>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 3: return launch_q8s_m<3>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 4: return launch_q8s_m<4>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 5: return launch_q8s_m<5>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 6: return launch_q8s_m<6>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        case 7: return launch_q8s_m<7>(cpl, w, K, N, xq, xd, rs, y, st, cus);
        default: return launch_q8s_m<8>(cpl, w, K, N, xq, xd, rs, y, st, cus);
    }
}

}  // namespace bq
