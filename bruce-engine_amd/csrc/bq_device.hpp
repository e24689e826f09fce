// bq_device.hpp -- device helpers shared by the gfx950 kernels of libbq.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define BQ_DEV __device__ __forceinline__

namespace bq {

constexpr int kQ5Bytes = 176;  // GGUF Q5_K block (256 values)
constexpr int kQ6Bytes = 210;  // GGUF Q6_K block (256 values)
constexpr int kW144 = 144;     // Q5_K repack stage (128 values)
constexpr int kW160 = 160;     // Q6_K repack stage (128 values)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

BQ_DEV float h2f(uint32_t bits16) {
    // v_cvt_f32_f16: exact, fp16 denormals included
    const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

BQ_DEV uint16_t f2h_rn(float f) {
    // f is first rounded to fp32 (the reference's __float2half(a * b) rounds
    // twice); the empty asm stops the compiler from fusing the producing
    // multiply into a single-rounding mixed-precision v_mad_mix* instruction.
    asm volatile("" : "+v"(f));
    const _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

// bit pattern -> float.  Takes the word by value: __builtin_bit_cast applied
// directly to an ext_vector element reinterprets element 0, not the element.
BQ_DEV float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }

// signed int8x4 dot product with int32 accumulate (v_dot4_i32_i8)
BQ_DEV int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 16-byte load of read-once weight data
BQ_DEV u32x4 ld16(const void* p) { return *(const u32x4*)p; }

// s_waitcnt vmcnt(N) leaving lgkmcnt / expcnt unconstrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
#define BQ_WAIT_VM(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 0xF) | ((((n) >> 4) & 3) << 14) | 0x70 | 0xF00)
// s_waitcnt lgkmcnt(0) only (LDS writes done; vector loads may stay in flight)
#define BQ_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Wave64 sum left in lane 63 with DPP only (no LDS shuffles): row_shr 1, 2,
// 4, 8 scans each 16-lane row (its lane 15 ends with the row's total), then
// row_bcast:15 adds row 0's total into row 1 and row 2's into row 3, and
// row_bcast:31 adds lane 31 (rows 0 + 1) into rows 2 and 3.  Other lanes hold
// partial sums.  Every lane of the wave must be active (DPP reads the other
// lanes' registers).
template <int CTRL, int ROW_MASK, bool BOUND>
BQ_DEV float dpp_f(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, BOUND));
}
BQ_DEV float wave_sum_dpp63(float v) {
    v += dpp_f<0x111, 0xF, true>(v);   // row_shr:1
    v += dpp_f<0x112, 0xF, true>(v);   // row_shr:2
    v += dpp_f<0x114, 0xF, true>(v);   // row_shr:4
    v += dpp_f<0x118, 0xF, true>(v);   // row_shr:8
    v += dpp_f<0x142, 0xA, false>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_f<0x143, 0xC, false>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// b where bit `lane` of the wave mask is set, else a: one v_cndmask_b32.
// (C selects between array elements with a lane-dependent condition let the
// compiler turn the array into a dynamically indexed one: a compare-and-
// select chain over every element per select.)
BQ_DEV float lane_sel(float a, float b, uint64_t mask) {
    float r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
    return r;
}

constexpr int pow2_ceil(int v) { return v <= 1 ? 1 : 2 * pow2_ceil((v + 1) / 2); }

// Sums of V values per lane over the NL lanes lane0 + S*j (j = 0..NL-1) that
// share the other lane bits, all V at once, as a reduce-scatter butterfly:
// each exchange with the lane S*d apart (d = NL/2, NL/4, ... while the lane
// carries more than one value) keeps the half of its values selected by lane
// bit S*d and adds the partner's copy of them; the remaining exchanges are
// plain sums.  Shuffles: P - 1 for the halving exchanges plus one per plain
// one (P = V rounded up to a power of two), against V * log2 NL for V
// separate reductions.  Returns the total of value `idx` (idx >= V:
// padding); the lanes with ((lane / S) & scatter_writers<V, NL>()) == 0 hold
// distinct idx.  Every lane of the wave must be active (ballot, shuffles).
template <int V, int NL, int S>
BQ_DEV float scatter_sum(const float (&acc)[V], int lane, int& idx) {
    constexpr int P = pow2_ceil(V);
    static_assert(P <= NL && NL * S <= 64, "butterfly shape");
    float v[P];
#pragma unroll
    for (int k = 0; k < P; ++k) v[k] = k < V ? acc[k] : 0.f;
    idx = 0;
    int d = NL / 2;
#pragma unroll
    for (int h = P / 2; h >= 1; h >>= 1, d >>= 1) {
        const bool up = (lane & (S * d)) != 0;
        const uint64_t um = __builtin_amdgcn_ballot_w64(up);
#pragma unroll
        for (int k = 0; k < h; ++k) {
            const float keep = lane_sel(v[k], v[k + h], um);
            const float send = lane_sel(v[k + h], v[k], um);
            v[k] = keep + __shfl_xor(send, S * d, 64);
        }
        idx += up ? h : 0;
    }
#pragma unroll
    for (; d >= 1; d >>= 1) v[0] += __shfl_xor(v[0], S * d, 64);
    return v[0];
}

template <int V, int NL>
BQ_DEV constexpr int scatter_writers() {
    constexpr int P = pow2_ceil(V);  // evaluated at compile time
    return NL / P - 1;
}

// q8 quantization of one 32-value group held by a lane pair (lanes 2i, 2i+1,
// 16 consecutive values each; both lanes of the pair must execute it).
// Semantics of k_q8_quant (bruce.cu:518-539): d = amax*(1/127),
// id = d > 0 ? 1/d : 0 (IEEE division), q = clamp(rint(v*id), -127, 127),
// s = sum q.  The rounding is exact: c = clamp(v*id) is in [-127, 127] and
// c + 1.5*2^23 lands in [2^23, 2^24) where the float spacing is 1, so the
// addition rounds c to the nearest integer (ties to even, 1.5*2^23 being
// even) and the low byte of the sum's bit pattern is that integer in two's
// complement.  The codes of the lane's 16 values are returned in q[0..3]
// (little-endian bytes, value order).
// A group with 0 < amax < 127 * 2^-128 has a denormal d and id = 1/d = inf.
// The reference's __float2int_rn (PTX cvt.rni.s32.f32) turns v * id = NaN
// (v = 0) into 0 and +-inf into +-INT_MAX, clamped to +-127; that group-wide
// case is redone explicitly after the fast path (never taken otherwise).
BQ_DEV void q8_quant16(const f32x4 (&v)[4], uint32_t (&q)[4], float& d, int& s) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    // partner lane (xor 1) via DPP quad_perm [1,0,3,2]
    amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
    d = amax * (1.f / 127.f);
    const float id = d > 0.f ? 1.f / d : 0.f;
    constexpr float kMagic = 12582912.f;  // 1.5 * 2^23
    int acc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float c0 = __builtin_amdgcn_fmed3f(v[i].x * id, -127.f, 127.f) + kMagic;
        const float c1 = __builtin_amdgcn_fmed3f(v[i].y * id, -127.f, 127.f) + kMagic;
        const float c2 = __builtin_amdgcn_fmed3f(v[i].z * id, -127.f, 127.f) + kMagic;
        const float c3 = __builtin_amdgcn_fmed3f(v[i].w * id, -127.f, 127.f) + kMagic;
        const uint32_t lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, c1), __builtin_bit_cast(uint32_t, c0), 0x0C0C0400u);
        const uint32_t hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, c3), __builtin_bit_cast(uint32_t, c2), 0x0C0C0400u);
        q[i] = lo | (hi << 16);
    }
    if (__builtin_expect(id > 3.402823466e38f, 0)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = v[i][e];
                const uint32_t c = x > 0.f ? 0x7Fu : (x < 0.f ? 0x81u : 0u);
                w |= c << (8 * e);
            }
            q[i] = w;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_sdot4((int)q[i], 0x01010101, acc, false);
    s = acc + __builtin_amdgcn_mov_dpp(acc, 0xB1, 0xF, 0xF, false);
}

// Row L2 norm helpers shared by the q8 producers and the producer-fused
// GEMV (one definition, so both produce identical bits).
constexpr float kEpsL2 = 1e-6f;

// l2_scale (bruce.cu:305-307), IEEE division and square root
BQ_DEV float l2_scale(float ss, int n) {
    return (1.0f / sqrtf(ss / (float)n + kEpsL2 / (float)n)) * (1.0f / sqrtf((float)n));
}

// Workgroup sum of one (X = 1) or two (X = 2) floats; every thread gets the totals.
template <int X>
BQ_DEV void block_sum(float (&v)[X], float* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int i = 0; i < X; ++i) v[i] = wave_sum_dpp63(v[i]);
    __syncthreads();  // red may still be read by a previous reduction
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < X; ++i) red[i * 16 + w] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < X; ++i) {
        float t = 0.f;
        for (int k = 0; k < nw; ++k) t += red[i * 16 + k];
        v[i] = t;
    }
}

// 1 + exp(-x) with the fast exponential (v_exp_f32 of x * log2(e)), as the
// reference's __expf (bruce.cu:611, :632): the silu*mul producer has a fifth
// fewer VALU instructions than with the accurate expf, which shortens the
// producer in front of the fused down GEMV (decode chain 1.5-2% faster)
BQ_DEV float sigmoid_den(float x) { return 1.f + __expf(-x); }

// The elementwise parts of the q8 producers (one definition each, so the
// standalone producers and the GEMV-fused ones compile to the same arithmetic).
// The quotient by the sigmoid denominator is a product with its reciprocal
// (v_rcp_f32, 1 ulp) instead of the correctly rounded division (a dozen
// instructions): within an ulp or two of the reference's division, next to
// the few ulps of its __expf; the decode chain's producers run 1% faster.
BQ_DEV float over_den(float a, float den) { return a * __builtin_amdgcn_rcpf(den); }
// gate: aout / (1 + exp(-gate*sg))  (k_gate_norm, bruce.cu:602)
BQ_DEV float gate_div(float a, float gate, float sg) { return over_den(a, sigmoid_den(gate * sg)); }
// silu(g*sg) * u * su  (k_silu_mul_norm, bruce.cu:622)
BQ_DEV float silu_mul(float g, float u, float sg, float su) {
    const float gv = g * sg;
    return over_den(gv, sigmoid_den(gv)) * u * su;
}
// resid: a = x*ka, b = upd*kb, a + (b - a)*alpha  (k_resid, bruce.cu:571)
BQ_DEV float resid_blend(float x, float ka, float u, float kb, float al) {
    const float an = x * ka, bn = u * kb;
    return an + (bn - an) * al;
}

// 6-bit scale and min of Q5_K sub-block j from the three scale words
// (s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11]); GGUF layout:
// j < 4: sc = s[j] & 63, m = s[j+4] & 63; j >= 4: low nibbles from s[j+4],
// top two bits from s[j-4] / s[j].  Branch-free for divergent j.
BQ_DEV void q5k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t& sc, uint32_t& m) {
    const int sh = 8 * (j & 3);
    const uint32_t a = (s0 >> sh) & 0xFF, b = (s1 >> sh) & 0xFF, c = (s2 >> sh) & 0xFF;
    const uint32_t lo_sc = a & 63, lo_m = b & 63;
    const uint32_t hi_sc = (c & 0xF) | ((a >> 6) << 4);
    const uint32_t hi_m = (c >> 4) | ((b >> 6) << 4);
    sc = j < 4 ? lo_sc : hi_sc;
    m = j < 4 ? lo_m : hi_m;
}

}  // namespace bq
