// bq_quant.hip -- activation int8 quantizer (per-32 scale + integer sum).
//
// Semantics of k_q8_quant / k_q8_rows (bruce.cu:518-539, :1081-1108): per
// 32-value group d = amax*(1/127), id = d > 0 ? 1/d : 0 (IEEE division),
// q = clamp(rint(v*id), -127, 127), xsum = sum(q); optional xdh = half(xd*xsum)
// (k_fill_xdh, bruce.cu:6598-6602) written by the same pass.
//
// Layout on gfx950: x[rows][K] is contiguous and K % 32 == 0, so group g of the
// flattened array is exactly xd[g] -- the kernel ignores row boundaries.  Each
// lane owns 4 consecutive values (one 16-byte load), 8 lanes own a group, a
// wave64 covers 8 groups (1 KiB of fp32 in, 256 B of int8 out, coalesced).
// amax and sum are reduced across the 8 lanes with xor shuffles; max and
// integer sums are order-independent, so the result is bit-exact.
#include "bq_device.hpp"

namespace bq {

__global__ void __launch_bounds__(256) k_quant_q8(const float* __restrict__ x, int ngroups,
                                                  int8_t* __restrict__ xq, float* __restrict__ xd,
                                                  int32_t* __restrict__ xsum,
                                                  uint16_t* __restrict__ xdh) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int g = tid >> 3;
    const bool live = g < ngroups;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (live) v = *(const f32x4*)(x + (size_t)tid * 4);
    float d;
    int s;
    const uint32_t packed = q8_quant4(v, d, s);
    if (!live) return;
    *(uint32_t*)(xq + (size_t)tid * 4) = packed;
    if ((tid & 7) == 0) {
        xd[g] = d;
        xsum[g] = s;
        if (xdh) xdh[g] = f2h_rn(d * (float)s);
    }
}

__global__ void __launch_bounds__(256) k_fill_xdh(const float* __restrict__ xd,
                                                  const int32_t* __restrict__ xsum, int n,
                                                  uint16_t* __restrict__ xdh) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) xdh[i] = f2h_rn(xd[i] * (float)xsum[i]);
}

hipError_t launch_quant_q8(const float* x, int rows, int K, int8_t* xq, float* xd, int32_t* xsum,
                           uint16_t* xdh, hipStream_t st) {
    const long long ngroups = (long long)rows * (K / 32);
    if (ngroups == 0) return hipSuccess;
    const long long threads = ngroups * 8;
    const int blocks = (int)((threads + 255) / 256);
    hipLaunchKernelGGL(k_quant_q8, dim3(blocks), dim3(256), 0, st, x, (int)ngroups, xq, xd, xsum, xdh);
    return hipGetLastError();
}

hipError_t launch_fill_xdh(const float* xd, const int32_t* xsum, int n, uint16_t* xdh, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_xdh, dim3((n + 255) / 256), dim3(256), 0, st, xd, xsum, n, xdh);
    return hipGetLastError();
}

}  // namespace bq
