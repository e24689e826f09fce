// bq_quant.hip -- activation int8 quantizer (per-32 scale + integer sum).
//
// Semantics of k_q8_quant / k_q8_rows (bruce.cu:518-539, :1081-1108): per
// 32-value group d = amax*(1/127), id = d > 0 ? 1/d : 0 (IEEE division),
// q = clamp(rint(v*id), -127, 127), xsum = sum(q); optional xdh = half(xd*xsum)
// (k_fill_xdh, bruce.cu:6598-6602) written by the same pass.
//
// Layout on gfx950: x[rows][K] is contiguous and K % 32 == 0, so group g of the
// flattened array is exactly xd[g] -- the kernel ignores row boundaries.  Each
// lane owns 16 consecutive values (four 16-byte loads), a lane pair owns a
// group, a wave64 covers 32 groups (4 KiB of fp32 in, 1 KiB of int8 out).
// amax and sum are combined across the pair with one DPP move each; max and
// integer sums are order-independent, so the result is bit-exact.  The same
// q8_quant16 runs inside the fused quantize+GEMV kernel.
#include "bq_device.hpp"

namespace bq {

__global__ void __launch_bounds__(256) k_quant_q8(const float* __restrict__ x, int ngroups,
                                                  int8_t* __restrict__ xq, float* __restrict__ xd,
                                                  int32_t* __restrict__ xsum,
                                                  uint16_t* __restrict__ xdh) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int g = tid >> 1;
    const bool live = g < ngroups;
    f32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (live) v[i] = *(const f32x4*)(x + (size_t)tid * 16 + 4 * i);
    }
    uint32_t q[4];
    float d;
    int s;
    q8_quant16(v, q, d, s);
    if (!live) return;
    *(u32x4*)(xq + (size_t)tid * 16) = u32x4{q[0], q[1], q[2], q[3]};
    if ((tid & 1) == 0) {
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
    const long long threads = ngroups * 2;
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
