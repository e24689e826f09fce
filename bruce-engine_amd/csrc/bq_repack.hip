// bq_repack.hip -- load-time repacks of k-quant weights into aligned int8 stages.
//
// Q5_K -> W144 [K/128][N][144] + Dm [N][K/32] fp16 (index map of
//         k_q5k_prepack144, bruce.cu:5747-5789): 128 u8 5-bit codes in natural
//         k order, 4 fp32 ds = d*sc, and Dm = half(-dmin*m).
// Q6_K -> W160 [N][K/128][160] (q6k_repack_host, bruce.cu:4783-4811): 128 int8
//         (code - 32) in natural k order + 8 fp32 d*sc.
// One wave per 256-value super-block; each lane produces one dword of codes.
// Both outputs are bit-exact with the reference (the fp32 products d*sc are
// exact: an 11-bit significand times a 6/8-bit integer).
#include "bq_device.hpp"
#include "bq_internal.hpp"

namespace bq {

__global__ void __launch_bounds__(256)
k_repack_q5k(const uint8_t* __restrict__ raw, int K, int N, uint8_t* __restrict__ w144,
             uint16_t* __restrict__ dm) {
    const int nsb = K >> 8, nb = K >> 5;
    const long long bi = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (bi >= (long long)N * nsb) return;
    const int row = (int)(bi / nsb), sb = (int)(bi % nsb);
    const int lane = threadIdx.x & 63, hh = lane >> 5, w = lane & 31;
    const int j = 4 * hh + (w >> 3), o4 = (w & 7) * 4;
    const uint8_t* b = raw + (size_t)bi * kQ5Bytes;
    const uint32_t qs = *(const uint32_t*)(b + 48 + 32 * (j >> 1) + o4);
    const uint32_t qh = *(const uint32_t*)(b + 16 + o4);
    const uint32_t val = ((qs >> (4 * (j & 1))) & 0x0F0F0F0Fu) | (((qh >> j) & 0x01010101u) << 4);
    uint8_t* out = w144 + ((size_t)(sb * 2 + hh) * N + row) * kW144;
    *(uint32_t*)(out + 4 * w) = val;
    if (w < 4) {
        const int js = 4 * hh + w;
        uint32_t sc, m;
        q5k_scale_min(*(const uint32_t*)(b + 4), *(const uint32_t*)(b + 8), *(const uint32_t*)(b + 12),
                      js, sc, m);
        const float d = h2f(*(const uint16_t*)b), dmin = h2f(*(const uint16_t*)(b + 2));
        ((float*)(out + 128))[w] = d * (float)sc;
        dm[(size_t)row * nb + sb * 8 + js] = f2h_rn(-(dmin * (float)m));
    }
}

__global__ void __launch_bounds__(256)
k_repack_q6k(const uint8_t* __restrict__ raw, int K, int N, uint8_t* __restrict__ w160) {
    const int nsb = K >> 8, nst = K >> 7;
    const long long bi = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (bi >= (long long)N * nsb) return;
    const int row = (int)(bi / nsb), sb = (int)(bi % nsb);
    const int lane = threadIdx.x & 63, h = lane >> 5, w = lane & 31;
    const int u = w >> 3, ll = (w & 7) * 4;
    const uint8_t* b = raw + (size_t)bi * kQ6Bytes;  // 2-byte aligned: byte loads only
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint8_t qlb = b[64 * h + 32 * (u & 1) + ll + i];
        const int lo = (u < 2) ? (qlb & 0xF) : (qlb >> 4);
        const int hi = (b[128 + 32 * h + ll + i] >> (2 * u)) & 3;
        packed |= (uint32_t)((uint8_t)(int8_t)((lo | (hi << 4)) - 32)) << (8 * i);
    }
    uint8_t* out = w160 + ((size_t)row * nst + sb * 2 + h) * kW160;
    *(uint32_t*)(out + 4 * w) = packed;
    if (w < 8) {
        const float d = h2f((uint32_t)b[208] | ((uint32_t)b[209] << 8));
        ((float*)(out + 128))[w] = d * (float)(int8_t)b[192 + 8 * h + w];
    }
}

hipError_t launch_repack_q5k(const void* raw, int K, int N, void* w144, uint16_t* dm, hipStream_t st) {
    const long long nblk = (long long)N * (K >> 8);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q5k, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st,
                       (const uint8_t*)raw, K, N, (uint8_t*)w144, dm);
    return hipGetLastError();
}

hipError_t launch_repack_q6k(const void* raw, int K, int N, void* w160, hipStream_t st) {
    const long long nblk = (long long)N * (K >> 8);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q6k, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st,
                       (const uint8_t*)raw, K, N, (uint8_t*)w160);
    return hipGetLastError();
}

}  // namespace bq
