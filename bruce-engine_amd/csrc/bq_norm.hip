// bq_norm.hip -- the q8 producers: row L2 norms that emit the q8 activations
// the GEMVs consume, in the same pass.
//
// Reference kernels (bruce.cu), all "elementwise op -> L2 norm -> q8_emit":
//   k_norm :541 / k_norm_rows :1110            t = src
//   k_add_norm :556 / k_add_norm_rows :1128     t = x + h                    (in place, x)
//   k_resid :571 / _rows :1146 / _vec4 :1475    a = x*ka, b = upd*kb,
//                                               t = a + (b - a)*alpha        (in place, x)
//   k_gate_norm :602 / _rows :1181 / _vec4      t = aout / (1 + exp(-gate*sg))
//   k_silu_mul_norm :622 / _rows :1205 / _vec4  gv = g*sg, t = gv/(1 + exp(-gv)) * u * su
// then v = t * l2_scale(sum t^2, n), l2_scale(ss, n) = (1/sqrt(ss/n + eps/n)) *
// (1/sqrt(n)) with eps = 1e-6 (:73, :305-307), and q8_emit (:338-366): per 32
// values d = amax*(1/127), q = clamp(rint(v/d)), xsum = sum q.
//
// gfx950 layout: one workgroup per row, a lane holds 16 consecutive values per
// pass (four 16-byte loads per input array), so a lane pair holds exactly one
// 32-value q8 group and the quantizer is q8_quant16, the same code as
// bq_quantize_q8: the q8 row is bit-identical to quantizing the emitted fp32
// row.  blockDim = n/16 rounded up to a wave (<= 1024), so a decode row of up
// to 16384 values is one pass in registers; rows up to 32768 take two.
// Sums of squares: per lane, wave64 butterfly, then one LDS slot per wave.
#include <math.h>

#include <algorithm>

#include "bq_device.hpp"
#include "bq_internal.hpp"

namespace bq {


struct NormArgs {
    float* out;          // fp32 output rows (NULL: not written); for Add/Resid this is x
    const float* a;      // src / x / x / aout / g
    const float* b;      // - / h / upd / gate / u
    const float* c;      // - / - / alpha[n] / sg[n] / sg[n]
    const float* d;      // - / - / - / - / su[n]
    int8_t* xq;
    float* xd;
    int32_t* xsum;
    int n;
};

template <int OP, int CH>
__global__ void __launch_bounds__(1024) k_norm_q8(NormArgs p) {
    __shared__ float red[32];
    const int n = p.n;
    const size_t ro = (size_t)blockIdx.x * n;
    const int stride = blockDim.x * 16;
    f32x4 t[CH][4];
    float ss[1] = {0.f};
    if constexpr (OP == kOpResid || OP == kOpResidNorm) {
        // two row norms first (x and upd), then the blend and its norm
        f32x4 xa[CH][4], ub[CH][4], al[CH][4];
        float s2[2] = {0.f, 0.f};
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i0 = c * stride + threadIdx.x * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xa[c][i] = ub[c][i] = al[c][i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (i0 < n) {
                    xa[c][i] = *(const f32x4*)(p.a + ro + i0 + 4 * i);
                    ub[c][i] = *(const f32x4*)(p.b + ro + i0 + 4 * i);
                    al[c][i] = *(const f32x4*)(p.c + i0 + 4 * i);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s2[0] += xa[c][i][e] * xa[c][i][e];
                    s2[1] += ub[c][i][e] * ub[c][i][e];
                }
            }
        }
        block_sum<2>(s2, red);
        const float ka = l2_scale(s2[0], n), kb = l2_scale(s2[1], n);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i0 = c * stride + threadIdx.x * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = resid_blend(xa[c][i][e], ka, ub[c][i][e], kb, al[c][i][e]);
                    t[c][i][e] = v;
                    ss[0] += v * v;
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i0 = c * stride + threadIdx.x * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
                if (i0 < n) {
                    const f32x4 a = *(const f32x4*)(p.a + ro + i0 + 4 * i);
                    if constexpr (OP == kOpNorm) {
                        v = a;
                    } else if constexpr (OP == kOpAdd) {
                        v = a + *(const f32x4*)(p.b + ro + i0 + 4 * i);
                    } else if constexpr (OP == kOpGate) {
                        const f32x4 gt = *(const f32x4*)(p.b + ro + i0 + 4 * i);
                        // no sg row: the gate row is already scaled (sg = 1)
                        const f32x4 sg = p.c ? *(const f32x4*)(p.c + i0 + 4 * i) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = gate_div(a[e], gt[e], sg[e]);
                    } else {  // kOpSilu
                        const f32x4 u = *(const f32x4*)(p.b + ro + i0 + 4 * i);
                        const f32x4 sg = *(const f32x4*)(p.c + i0 + 4 * i);
                        const f32x4 su = *(const f32x4*)(p.d + i0 + 4 * i);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = silu_mul(a[e], u[e], sg[e], su[e]);
                    }
                }
                t[c][i] = v;
#pragma unroll
                for (int e = 0; e < 4; ++e) ss[0] += v[e] * v[e];
            }
        }
    }
    block_sum<1>(ss, red);
    float k = l2_scale(ss[0], n);
    if constexpr (OP == kOpResidNorm) {
        // the resid's row, then k_norm over it (bruce.cu:8017, :8022): the
        // sums of a separate norm launch over the emitted row, in its order
        float s3[1] = {0.f};
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                t[c][i] = t[c][i] * k;
#pragma unroll
                for (int e = 0; e < 4; ++e) s3[0] += t[c][i][e] * t[c][i][e];
            }
        block_sum<1>(s3, red);
        k = l2_scale(s3[0], n);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i0 = c * stride + threadIdx.x * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) t[c][i] = t[c][i] * k;
        // lane pairs hold whole 32-value groups (n % 32 == 0): both lanes of a
        // pair are inside the row or both outside
        uint32_t q[4];
        float d;
        int s;
        q8_quant16(t[c], q, d, s);
        if (i0 < n) {
            if (p.out)
#pragma unroll
                for (int i = 0; i < 4; ++i) *(f32x4*)(p.out + ro + i0 + 4 * i) = t[c][i];
            *(u32x4*)(p.xq + ro + i0) = u32x4{q[0], q[1], q[2], q[3]};
            if ((threadIdx.x & 1) == 0) {
                const size_t gi = (ro + i0) >> 5;
                p.xd[gi] = d;
                p.xsum[gi] = s;
            }
        }
    }
}

namespace {
template <int OP>
hipError_t launch_op(const NormArgs& a, int rows, hipStream_t st) {
    const int lanes = (a.n + 15) / 16;
    const int threads = std::min(1024, (lanes + 63) / 64 * 64);
    const int ch = (lanes + threads - 1) / threads;
    if (ch == 1)
        launch_kernel((k_norm_q8<OP, 1>), dim3(rows), dim3(threads), 0, st, a);
    else
        launch_kernel((k_norm_q8<OP, 2>), dim3(rows), dim3(threads), 0, st, a);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_norm_q8(int op, float* out, const float* a, const float* b, const float* c,
                          const float* d, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
                          hipStream_t st) {
    const NormArgs args{out, a, b, c, d, xq, xd, xsum, n};
    switch (op) {
        case kOpNorm: return launch_op<kOpNorm>(args, rows, st);
        case kOpAdd: return launch_op<kOpAdd>(args, rows, st);
        case kOpResid: return launch_op<kOpResid>(args, rows, st);
        case kOpGate: return launch_op<kOpGate>(args, rows, st);
        case kOpResidNorm: return launch_op<kOpResidNorm>(args, rows, st);
        default: return launch_op<kOpSilu>(args, rows, st);
    }
}

}  // namespace bq
