// bq_gemv.hip -- k-quant x q8 decode GEMV / multi-row (1..8 rows) kernels for gfx950.
//
// Reference semantics (engine/src/bruce.cu):
//   Q5_K  y[n] = sum_g xd[g] * (ds[n,g]*dot[n,g] - dm[n,g]*xsum[g])
//         k_gemv_q5k :384-440, k_gemv_q5k_fused :5815-5887, k_gemm_tc_verify_q5k :5889-6076
//   Q6_K  y[n] = sum_{16-groups} xd[g32] * (d*sc16) * sum (q-32)*xq
//         k_gemm_q6k :4282-4362 (raw 210 B), k_gemv_q6k_dp :4452-4513 (160 B repack)
//
// MI355X design (one decode GEMV is 6-40 MB: about one HBM latency x
// bandwidth product, so every load is issued up front and consumed in order):
//   * Lane task = 64 consecutive weight values of one row (two Q5_K sub-blocks,
//     half a Q6_K repack stage, or a 4 x 16 slice of a raw Q6_K block); a row
//     has K/64 tasks.
//   * One weight row per 16-lane DPP row: a wave owns 4 rows ("tile"), lanes
//     16g..16g+15 walk the tasks of row g, 16 per step, at most 3 steps per
//     wave (longer rows are split over KS waves of one workgroup).  Row sums
//     are reduced with four DPP row shifts; K slices are combined through LDS.
//   * Activations are copied to LDS with direct-to-LDS DMA loads issued before
//     the weight loads; each wave then waits only for its own DMA (vmcnt =
//     number of weight loads issued after it) before the workgroup barrier, so
//     all weight bytes are in flight before any wave waits, and step s is
//     computed as soon as its loads have returned.
#include "bq_device.hpp"
#include "bq_internal.hpp"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace bq {

constexpr int kRowsPerTile = 4;    // one row per 16-lane DPP row
// Q5_K multi-row: dot products (and, since the scale products moved to
// v_mfma_f32_4x4x1f32, the epilogue's scale products) on the matrix cores
// from this many activation rows up.  The matrix-core lane map (4 lanes = one
// task across the 4 rows) loses the address merging of the per-block header /
// qh loads that the dot4 map gets (4 lanes of one row read the same 16
// bytes).  Measured with 40 rotating copies (dot4 -> matrix cores, us):
// 9216 x 3072 4 / 5 rows 7.95 / 8.84 -> 7.2 / 8.45, 18432 x 3072 12.1 / 14.7
// -> 10.0 / 12.6, 3072 x 3072 5.1 / 5.6 -> 4.5 / 5.0; at 2 / 3 rows dot4
// stays ahead or level (9216 x 3072 2 rows 6.4 vs 6.7-6.8).
constexpr int kQ5kMfmaMinRows = 4;
// Q6_K (W160 and raw) from 3 rows: no per-block header is shared between the
// lanes of a row there (W160), or only 2 of 8 loads (raw), and the dot4 path
// needs two dot4 per dword for the -32 offset (raw).  Measured 3072 x 9216,
// rows 3 / 4 / 8: W160 11.5 / 12.7 / 17.1 -> 11.0 / 11.7 / 14.8 us, raw
// 10.0 / 11.2 / 16.1 -> 9.8 / 10.5 / 13.9 us; at 2 rows equal (W160) or
// slower (raw 8.7 -> 9.2).
constexpr int kQ6RepMfmaMinRows = 3;
constexpr int kQ6RawMfmaMinRows = 3;
constexpr int kTasksPerStep = 16;  // tasks of one row per step

BQ_DEV int find_part(const PartTable& pt, int tile) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxParts; ++i)
        if (i < pt.nparts && tile >= pt.tile0[i]) p = i;
    return p;
}

// sum over the 16 lanes of a DPP row; lane 15 of the row ends with the total
BQ_DEV float row16_sum(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true));  // row_shr:1
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true));  // row_shr:2
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true));  // row_shr:4
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true));  // row_shr:8
    return v;
}

// 4 bytes of 5-bit codes of Q5_K sub-block j: low/high nibble (hi) of qs with
// bit j of each qh byte as bit 4.  alignbit(qh, qh, j - 4) rotates bit j of
// every byte onto bit 4 of the same byte.
BQ_DEV uint32_t q5_codes(uint32_t qs, uint32_t qh, int j, bool hi) {
    const uint32_t nib = (hi ? (qs >> 4) : qs) & 0x0F0F0F0Fu;
    const uint32_t rot = __builtin_amdgcn_alignbit(qh, qh, (uint32_t)(j - 4) & 31u);
    return (rot & 0x10101010u) | nib;
}

// Row stride of the staged int8 activation rows: with several rows, K + 16,
// so that the lanes of a multi-row block (lane = 4 * task + row), which read
// the same 16 bytes of 4 rows, reach 4 different bank groups.  Unpadded, the
// rows (K a multiple of 256) start on the same bank and every such read is a
// 4-way conflict.
__host__ __device__ constexpr int act_row_stride(int rows, int K) { return rows > 1 ? K + 16 : K; }

struct ActLds {            // activations of MR rows staged in LDS
    const int8_t* x;       // [MR][xr] int8 codes (row stride act_row_stride)
    const float* xd;       // [MR][K/32]
    const int32_t* xs;     // Q5_K only: xsum [MR][K/32]
    int xr;                // row stride of x
};

// ---------------------------------------------------------------------------
// Weight-format policies: Task = registers one lane loads for one 64-value
// task; load() issues them, dot() adds the task's contribution to each
// activation row.
// ---------------------------------------------------------------------------
struct FmtQ5K {
    static constexpr int kLoads = 5;  // VMEM instructions per task
    struct Task { u32x4 hdr, qh0, qh1, qs0, qs1; };
    // task t: super-block t >> 2, sub-block pair t & 3
    static BQ_DEV void load(Task& a, const uint8_t* row, int t) {
        const uint8_t* blk = row + (t >> 2) * kQ5Bytes;
        const int jp = t & 3;
        a.hdr = ld16(blk);
        a.qh0 = ld16(blk + 16);
        a.qh1 = ld16(blk + 32);
        a.qs0 = ld16(blk + 48 + 32 * jp);
        a.qs1 = ld16(blk + 64 + 32 * jp);
    }
    // 6-bit scales / mins of the task's sub-blocks j0 = 2jp, j1 = 2jp + 1 from
    // the header words (y = scales[0..3], z = scales[4..7], w = scales[8..11]),
    // packed as bytes [sc0, sc1, m0, m1]:
    //   jp < 2:  sc = y.byte(j) & 63, m = z.byte(j) & 63
    //   jp >= 2: sc = (w.byte(j-4) & 15) | (y.byte(j-4) >> 6) << 4,
    //            m  = (w.byte(j-4) >> 4) | (z.byte(j-4) >> 6) << 4
    // Bytes i0 = 2(jp & 1), i0 + 1 of y/z/w are gathered with v_perm_b32.
    static BQ_DEV uint32_t scale_min4(const u32x4& hdr, int jp) {
        const bool odd = jp & 1;
        const uint32_t q = __builtin_amdgcn_perm(hdr.z, hdr.y, odd ? 0x07060302u : 0x05040100u);  // y_i0 y_i1 z_i0 z_i1
        const uint32_t lo = q & 0x3F3F3F3Fu;
        const uint32_t ww = __builtin_amdgcn_perm(hdr.w, hdr.w, odd ? 0x03020302u : 0x01000100u); // w_i0 w_i1 w_i0 w_i1
        const uint32_t wn = ((ww >> 4) & 0x0F0F0000u) | (ww & 0x00000F0Fu);
        const uint32_t hi = wn | ((q >> 2) & 0x30303030u);
        return jp >= 2 ? hi : lo;
    }
    template <int MR>
    static BQ_DEV void dot(const Task& a, const uint8_t*, int t, const ActLds& act, int K, float (&acc)[MR]) {
        const int jp = t & 3, j0 = 2 * jp, j1 = j0 + 1;
        const uint32_t sm = scale_min4(a.hdr, jp);
        const float d = h2f(a.hdr.x & 0xFFFF), dmin = h2f(a.hdr.x >> 16);
        const float ds0 = d * (float)(sm & 0xFF), ds1 = d * (float)((sm >> 8) & 0xFF);
        const float dm0 = dmin * (float)((sm >> 16) & 0xFF), dm1 = dmin * (float)(sm >> 24);
        uint32_t u0[8], u1[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u0[i] = q5_codes(a.qs0[i], a.qh0[i], j0, false);
            u0[i + 4] = q5_codes(a.qs1[i], a.qh1[i], j0, false);
            u1[i] = q5_codes(a.qs0[i], a.qh0[i], j1, true);
            u1[i + 4] = q5_codes(a.qs1[i], a.qh1[i], j1, true);
        }
        const int nb = K >> 5;
        const int g0 = (t >> 2) * 8 + j0;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int8_t* xp = act.x + m * act.xr + 32 * g0;
            const u32x4 x0 = *(const u32x4*)(xp), x1 = *(const u32x4*)(xp + 16);
            const u32x4 x2 = *(const u32x4*)(xp + 32), x3 = *(const u32x4*)(xp + 48);
            int s0 = 0, s1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s0 = dot4((int)u0[i], (int)x0[i], s0);
                s0 = dot4((int)u0[i + 4], (int)x1[i], s0);
                s1 = dot4((int)u1[i], (int)x2[i], s1);
                s1 = dot4((int)u1[i + 4], (int)x3[i], s1);
            }
            const float2 xdv = *(const float2*)(act.xd + m * nb + g0);
            const int2 xsv = *(const int2*)(act.xs + m * nb + g0);
            acc[m] += xdv.x * (ds0 * (float)s0 - dm0 * (float)xsv.x) + xdv.y * (ds1 * (float)s1 - dm1 * (float)xsv.y);
        }
    }
};

// Multi-row dot products of FmtQ5K on the matrix cores: v_mfma_i32_4x4x4i8
// runs 16 independent 4x4x4 blocks per instruction; block b (lanes 4b..4b+3)
// gives C[i][j] = sum_k A(lane 4b+i)[k] * B(lane 4b+j)[k] and lane 4b+j holds
// C[0..3][j] (measured on gfx950).  With the multi-row lane map (lane = 4 *
// task + row, kMmLanes) block b is one task across the wave's 4 weight rows:
// lane 4b+r feeds weight row r's code dword as B and activation row 4ms+r's
// dword as A, so after 8 instructions per 32-value sub-block the lane holds
// the exact integer dots of its weight row with activation rows 4ms..4ms+3.
// The float epilogue runs its scale products on the matrix cores as well (below).
template <int MR>
BQ_DEV void q5k_dot_mm(const FmtQ5K::Task& a, int t, const ActLds& act, int K, float (&acc)[MR], int lane) {
    const int jp = t & 3, j0 = 2 * jp, j1 = j0 + 1;
    const uint32_t sm = FmtQ5K::scale_min4(a.hdr, jp);
    const float d = h2f(a.hdr.x & 0xFFFF), dmin = h2f(a.hdr.x >> 16);
    const float ds0 = d * (float)(sm & 0xFF), ds1 = d * (float)((sm >> 8) & 0xFF);
    const float dm0 = dmin * (float)((sm >> 16) & 0xFF), dm1 = dmin * (float)(sm >> 24);
    uint32_t u0[8], u1[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u0[i] = q5_codes(a.qs0[i], a.qh0[i], j0, false);
        u0[i + 4] = q5_codes(a.qs1[i], a.qh1[i], j0, false);
        u1[i] = q5_codes(a.qs0[i], a.qh0[i], j1, true);
        u1[i + 4] = q5_codes(a.qs1[i], a.qh1[i], j1, true);
    }
    const int nb = K >> 5;
    const int g0 = (t >> 2) * 8 + j0;
    const int r = lane & 3;
#pragma unroll
    for (int ms = 0; ms < (MR + 3) / 4; ++ms) {
        const int m = 4 * ms + r;  // activation row fed as A by this lane
        const int8_t* xp = act.x + (m < MR ? m : MR - 1) * act.xr + 32 * g0;
        u32x4 x0 = *(const u32x4*)(xp), x1 = *(const u32x4*)(xp + 16);
        u32x4 x2 = *(const u32x4*)(xp + 32), x3 = *(const u32x4*)(xp + 48);
        // one accumulator chain per sub-block (split chains measured slower)
        i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int xa = (int)(k < 4 ? x0[k] : x1[k - 4]), xb = (int)(k < 4 ? x2[k] : x3[k - 4]);
            c0 = __builtin_amdgcn_mfma_i32_4x4x4i8(xa, (int)u0[k], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_4x4x4i8(xb, (int)u1[k], c1, 0, 0, 0);
        }
        // Scales on the matrix cores too (v_mfma_f32_4x4x1f32, same block
        // layout): lane 4b+r feeds activation row 4ms+r's xd (and xd * xsum)
        // as A and its weight row's ds (dm) as B, so lane 4b+r receives
        // xd[4ms+q] * ds[r] for q = 0..3 -- the scale products -- and the
        // min terms (xd * xsum)[4ms+q] * dm[r].  The epilogue is then one
        // convert and one FMA per activation row and sub-block:
        // sum_j (ds_j * xd) * dot_j - dm_j * (xd * xsum), the reference
        // verify kernel's form (bruce.cu:6007-6010).
        const float2 xdv = *(const float2*)(act.xd + (m < MR ? m : MR - 1) * nb + g0);
        const int2 xsv = *(const int2*)(act.xs + (m < MR ? m : MR - 1) * nb + g0);
        const f32x4 zf = {0.f, 0.f, 0.f, 0.f};
        const f32x4 s0 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.x, ds0, zf, 0, 0, 0);
        const f32x4 s1 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.y, ds1, zf, 0, 0, 0);
        f32x4 mn = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.x * (float)xsv.x, dm0, zf, 0, 0, 0);
        mn = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.y * (float)xsv.y, dm1, mn, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int mm = 4 * ms + q;
            if (mm < MR)
                acc[mm] += __builtin_fmaf(s1[q], (float)c1[q], __builtin_fmaf(s0[q], (float)c0[q], -mn[q]));
        }
    }
}

// The MR rows' sums over the 16 task lanes 4i + (lane & 3) of the multi-row
// lane map at once, as a reduce-scatter butterfly: each exchange with the
// lane 4d apart (d = 8, 4, 2 while the lane carries more than one row) keeps
// the half of its rows selected by bit d of i and adds the partner's copy of
// them, so a lane ends with one row m = rows_of(i), which the remaining
// exchanges (plain sums) complete.  P = MR rounded up to a power of two
// shuffles instead of 4 per row: 8 for 5..8 rows against 32.  Lanes with
// (i & (16 / P - 1)) == 0 hold distinct rows; m >= MR are padding.
struct FmtQ6KRep {
    static constexpr int kLoads = 5;
    struct Task { u32x4 c[4]; f32x4 sc; };
    // task t: stage t >> 1, half t & 1 (64 codes + the 4 scales of their 16-value groups)
    static BQ_DEV void load(Task& a, const uint8_t* row, int t) {
        const uint8_t* st = row + (t >> 1) * kW160;
        const int hf = t & 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) a.c[i] = ld16(st + 64 * hf + 16 * i);
        a.sc = *(const f32x4*)(st + 128 + 16 * hf);
    }
    template <int MR>
    static BQ_DEV void dot(const Task& a, const uint8_t*, int t, const ActLds& act, int K, float (&acc)[MR]) {
        const int k0 = 64 * t, nb = K >> 5;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            int s[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const u32x4 x = *(const u32x4*)(act.x + m * act.xr + k0 + 16 * g);
                int v = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) v = dot4((int)a.c[g][i], (int)x[i], v);
                s[g] = v;
            }
            const float2 xdv = *(const float2*)(act.xd + m * nb + (k0 >> 5));
            acc[m] += xdv.x * (a.sc.x * (float)s[0] + a.sc.y * (float)s[1]) +
                      xdv.y * (a.sc.z * (float)s[2] + a.sc.w * (float)s[3]);
        }
    }
};

// Multi-row dot products of FmtQ6KRep (W160: signed codes q-32, one fp32
// scale per 16 values) on v_mfma_i32_4x4x4i8, with the lane map and block
// layout of q5k_dot_mm: per 16-value group 4 instructions into one
// accumulator; the float epilogue is FmtQ6KRep::dot's expression.
template <int MR>
BQ_DEV void q6rep_dot_mm(const FmtQ6KRep::Task& a, int t, const ActLds& act, int K, float (&acc)[MR], int lane) {
    const int k0 = 64 * t, nb = K >> 5;
    const int r = lane & 3;
#pragma unroll
    for (int ms = 0; ms < (MR + 3) / 4; ++ms) {
        const int m = 4 * ms + r;  // activation row fed as A by this lane
        const int8_t* xp = act.x + (m < MR ? m : MR - 1) * act.xr + k0;
        i32x4 c[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const u32x4 x = *(const u32x4*)(xp + 16 * g);
            c[g] = i32x4{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) c[g] = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x[i], (int)a.c[g][i], c[g], 0, 0, 0);
        }
        // scale products xd[4ms+q] * (d*sc)[g] on v_mfma_f32_4x4x1f32 (see q5k_dot_mm)
        const float2 xdv = *(const float2*)(act.xd + (m < MR ? m : MR - 1) * nb + (k0 >> 5));
        const f32x4 zf = {0.f, 0.f, 0.f, 0.f};
        const f32x4 s0 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.x, a.sc.x, zf, 0, 0, 0);
        const f32x4 s1 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.x, a.sc.y, zf, 0, 0, 0);
        const f32x4 s2 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.y, a.sc.z, zf, 0, 0, 0);
        const f32x4 s3 = __builtin_amdgcn_mfma_f32_4x4x1f32(xdv.y, a.sc.w, zf, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int mm = 4 * ms + q;
            if (mm < MR)
                acc[mm] += __builtin_fmaf(s3[q], (float)c[3][q],
                                          __builtin_fmaf(s2[q], (float)c[2][q],
                                                         __builtin_fmaf(s1[q], (float)c[1][q], s0[q] * (float)c[0][q])));
        }
    }
}

// round a pointer down to 4 bytes, keeping it a (global) pointer
BQ_DEV const uint8_t* align4(const uint8_t* p) { return p - ((uintptr_t)p & 3); }

struct FmtQ6KRaw {
    // task t: super-block t >> 2, half h = (t >> 1) & 1, positions l0 = 16*(t & 1):
    // values 128h + 32u + l0 .. +15 of the four quarters u (both ql nibbles used).
    // Blocks are 2-byte aligned: every field is read as whole dwords from a
    // 4-byte aligned window inside the block and funnel-shifted into place.
    static constexpr int kLoads = 8;  // VMEM instructions per task
    struct Task { u32x4 qlA, qlB, qh; uint32_t qlA4, qlB4, qh4, d; uint32_t sc[3]; };
    static BQ_DEV void load(Task& a, const uint8_t* row, int t) {
        const uint8_t* blk = row + (t >> 2) * kQ6Bytes;
        const int h = (t >> 1) & 1, l0 = 16 * (t & 1);
        const uint8_t* pa = align4(blk + 64 * h + l0);
        const uint8_t* pb = align4(blk + 64 * h + 32 + l0);
        const uint8_t* ph = align4(blk + 128 + 32 * h + l0);
        // scales 192 + 8h .. +7: 12-byte window ending at most at byte 210
        const uint8_t* ps = align4(blk + 192 + 8 * h - 2);
        a.qlA = *(const u32x4*)pa;
        a.qlA4 = *(const uint32_t*)(pa + 16);
        a.qlB = *(const u32x4*)pb;
        a.qlB4 = *(const uint32_t*)(pb + 16);
        a.qh = *(const u32x4*)ph;
        a.qh4 = *(const uint32_t*)(ph + 16);
        __builtin_memcpy(a.sc, ps, 12);
        a.d = *(const uint16_t*)(blk + 208);
    }
    static BQ_DEV u32x4 shift16(const u32x4& v, uint32_t v4, uint32_t sh) {
        u32x4 r;
        r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
        r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
        r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
        r.w = __builtin_amdgcn_alignbyte(v4, v.w, sh);
        return r;
    }
    template <int MR>
    static BQ_DEV void dot(const Task& a, const uint8_t* row, int t, const ActLds& act, int K, float (&acc)[MR]) {
        const int h = (t >> 1) & 1, l0 = 16 * (t & 1);
        const uint8_t* blk = row + (t >> 2) * kQ6Bytes;
        const uint32_t sh = (uint32_t)(uintptr_t)blk & 2;  // 0 or 2 bytes
        const u32x4 qlA = shift16(a.qlA, a.qlA4, sh), qlB = shift16(a.qlB, a.qlB4, sh);
        const u32x4 qh = shift16(a.qh, a.qh4, sh);
        // the scale window starts 4 (aligned block) or 2 bytes before byte 192 + 8h
        const uint32_t s0 = sh ? __builtin_amdgcn_alignbyte(a.sc[1], a.sc[0], 2) : a.sc[1];
        const uint32_t s1 = sh ? __builtin_amdgcn_alignbyte(a.sc[2], a.sc[1], 2) : a.sc[2];
        const float d = h2f(a.d);
        float sc[4];
        uint32_t q[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int gi = 2 * u + (l0 >> 4);  // byte of the 8 scale bytes of this half
            const uint32_t w = gi < 4 ? s0 : s1;
            sc[u] = d * (float)(int8_t)(w >> (8 * (gi & 3)));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ql = (u & 1) ? qlB[i] : qlA[i];
                const uint32_t nib = ((u >= 2) ? (ql >> 4) : ql) & 0x0F0F0F0Fu;
                q[u][i] = nib | (((qh[i] >> (2 * u)) & 0x03030303u) << 4);
            }
        }
        const int kb = (t >> 2) * 256 + 128 * h + l0, nb = K >> 5;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = kb + 32 * u;
                const u32x4 x = *(const u32x4*)(act.x + m * act.xr + k);
                int s = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s = dot4((int)q[u][i], (int)x[i], s);
                    s = dot4((int)0xE0E0E0E0u, (int)x[i], s);  // codes are q in 0..63: add -32*x
                }
                v += act.xd[m * nb + (k >> 5)] * sc[u] * (float)s;
            }
            acc[m] += v;
        }
    }
    // the same on v_mfma_i32_4x4x4i8 (block layout of q5k_dot_mm): the codes
    // become signed q - 32 per byte, ((q | 0x80) - 0x20) ^ 0x80 with no
    // carry between bytes, then 4 instructions per 16-value quarter
    template <int MR>
    static BQ_DEV void dot_mm(const Task& a, const uint8_t* row, int t, const ActLds& act, int K, float (&acc)[MR],
                              int lane) {
        const int h = (t >> 1) & 1, l0 = 16 * (t & 1);
        const uint8_t* blk = row + (t >> 2) * kQ6Bytes;
        const uint32_t sh = (uint32_t)(uintptr_t)blk & 2;
        const u32x4 qlA = shift16(a.qlA, a.qlA4, sh), qlB = shift16(a.qlB, a.qlB4, sh);
        const u32x4 qh = shift16(a.qh, a.qh4, sh);
        const uint32_t s0 = sh ? __builtin_amdgcn_alignbyte(a.sc[1], a.sc[0], 2) : a.sc[1];
        const uint32_t s1 = sh ? __builtin_amdgcn_alignbyte(a.sc[2], a.sc[1], 2) : a.sc[2];
        const float d = h2f(a.d);
        float sc[4];
        uint32_t q[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int gi = 2 * u + (l0 >> 4);
            const uint32_t w = gi < 4 ? s0 : s1;
            sc[u] = d * (float)(int8_t)(w >> (8 * (gi & 3)));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ql = (u & 1) ? qlB[i] : qlA[i];
                const uint32_t nib = ((u >= 2) ? (ql >> 4) : ql) & 0x0F0F0F0Fu;
                const uint32_t code = nib | (((qh[i] >> (2 * u)) & 0x03030303u) << 4);
                q[u][i] = ((code | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            }
        }
        const int kb = (t >> 2) * 256 + 128 * h + l0, nb = K >> 5;
        const int r = lane & 3;
#pragma unroll
        for (int ms = 0; ms < (MR + 3) / 4; ++ms) {
            const int m = 4 * ms + r;
            const int8_t* xp = act.x + (m < MR ? m : MR - 1) * act.xr + kb;
            i32x4 c[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const u32x4 x = *(const u32x4*)(xp + 32 * u);
                c[u] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < 4; ++i) c[u] = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x[i], (int)q[u][i], c[u], 0, 0, 0);
            }
            // scale products xd[4ms+qq] * (d*sc)[u] on v_mfma_f32_4x4x1f32 (the
            // block layout of the int8 dots; see q5k_dot_mm)
            const int ma = m < MR ? m : MR - 1;
            const f32x4 zf = {0.f, 0.f, 0.f, 0.f};
            f32x4 sx[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                sx[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(act.xd[ma * nb + ((kb + 32 * u) >> 5)], sc[u], zf, 0, 0, 0);
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int mm = 4 * ms + qq;
                if (mm < MR) {
                    float v = sx[0][qq] * (float)c[0][qq];
#pragma unroll
                    for (int u = 1; u < 4; ++u) v = __builtin_fmaf(sx[u][qq], (float)c[u][qq], v);
                    acc[mm] += v;
                }
            }
        }
    }
};

template <class F> struct RowBytes;
template <> struct RowBytes<FmtQ5K> { static BQ_DEV size_t of(int K) { return (size_t)(K / 256) * kQ5Bytes; } };
template <> struct RowBytes<FmtQ6KRaw> { static BQ_DEV size_t of(int K) { return (size_t)(K / 256) * kQ6Bytes; } };
template <> struct RowBytes<FmtQ6KRep> { static BQ_DEV size_t of(int K) { return (size_t)(K / 128) * kW160; } };

// LDS bytes: MR staged activation rows + the K-slice partial sums
template <class F>
__host__ __device__ inline size_t act_lds_bytes(int rows, int K) {
    size_t b = (size_t)rows * act_row_stride(rows, K) + (size_t)rows * (K / 32) * 4;
    if (std::is_same<F, FmtQ5K>::value) b += (size_t)rows * (K / 32) * 4;
    return b;
}


// Copy `bytes` (multiple of 16) from global to LDS with direct-to-LDS loads:
// one 64-lane instruction moves 1 KiB into consecutive LDS.
BQ_DEV void dma_to_lds(uint8_t* lds, const void* src, int bytes, int wave, int waves, int lane) {
    const int n = bytes >> 4;
    for (int b = wave * 64; b < n; b += 64 * waves) {
        if (b + lane < n)
            __builtin_amdgcn_global_load_lds((const uint8_t*)src + 16 * (b + lane),
                                             (__attribute__((address_space(3))) void*)(lds + 16 * b), 16, 0, 0);
    }
}

// Fused-quantizer arguments: the fp32 activation row and optional q8 outputs
// (written by workgroup 0 only; NULL = not written).  With a q8 producer
// (QN == kQnProducer) x is the producer's first input, b/c/d the others (as
// in bq_norm_q8 .. bq_silu_mul_norm_q8) and out (optional, workgroup 0)
// receives the fp32 row the producer emits.
struct FusedQ8 {
    const float* x;
    int8_t* xq;
    float* xd;
    int32_t* xsum;
    int op = 0;             // NormOp of the producer
    float* out = nullptr;
    const float* b = nullptr;
    const float* c = nullptr;
    const float* d = nullptr;
};
constexpr int kQnProducer = -1;  // QN value of the producer-fused instances
// fused quantizer limit: 16 waves x 3 chunks of 1024 values in registers
constexpr int kFusedMaxK = kGemvMaxK;
constexpr int kProducerMaxK = 16 * 1024;  // one 1024-value chunk per wave, 16 waves
constexpr int kChunk = 1024;       // values one wave quantizes at a time (16 per lane)

// Fused quantizer, part 1: issue the fp32 loads of this wave's chunks (chunk c
// of the row belongs to wave c % waves).  K % 256 == 0 keeps lane pairs whole.
template <int QN>
BQ_DEV void fq_load(f32x4 (&xv)[QN][4], const float* x, int K, int wave, int waves, int lane) {
#pragma unroll
    for (int c = 0; c < QN; ++c) {
        const int v0 = (wave + waves * c) * kChunk + 16 * lane;
        if (v0 < K) {
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[c][i] = *(const f32x4*)(x + v0 + 4 * i);
        }
    }
}

// Fused quantizer, part 2 (after the loads have returned): q8_quant16 per lane
// pair, codes / xd / (XS) xsum into the LDS activation row, and the q8 row to
// global memory from workgroup 0 when requested.  Ends with the LDS writes
// complete (lgkmcnt 0); the caller's barrier publishes them.
template <int QN, bool XS>
BQ_DEV void fq_quantize(const f32x4 (&xv)[QN][4], uint8_t* smem, int K, int wave, int waves, int lane,
                        const FusedQ8& fq) {
    uint8_t* lx = smem;
    float* lxd = (float*)(smem + K);
    int32_t* lxs = (int32_t*)(lxd + (K >> 5));
    const bool out = blockIdx.x == 0 && fq.xq;
#pragma unroll
    for (int c = 0; c < QN; ++c) {
        const int v0 = (wave + waves * c) * kChunk + 16 * lane;
        if (v0 < K) {
            uint32_t q[4];
            float d;
            int s;
            q8_quant16(xv[c], q, d, s);
            const int gi = v0 >> 5;
            *(u32x4*)(lx + v0) = u32x4{q[0], q[1], q[2], q[3]};
            if ((lane & 1) == 0) {
                lxd[gi] = d;
                if constexpr (XS) lxs[gi] = s;
            }
            if (out) {
                *(u32x4*)(fq.xq + v0) = u32x4{q[0], q[1], q[2], q[3]};
                if ((lane & 1) == 0) {
                    fq.xd[gi] = d;
                    fq.xsum[gi] = s;
                }
            }
        }
    }
    asm volatile("" ::: "memory");
    BQ_WAIT_LGKM0();
}

// q8 producer fused into the GEMV (QN == kQnProducer): the row is cut into
// 1024-value chunks, chunk c belongs to wave c (one chunk per wave, K <=
// 16384) and lane l holds values 1024c + 16l .. +15 -- exactly the lane
// layout of k_norm_q8 (bq_norm.hip) for one row of that length, whose thread
// 64c + l holds the same 16 values and whose wave c is this wave.  The sums of
// squares therefore follow the same order: per lane over the 16 values, the
// same wave64 butterfly, then the per-wave totals in wave order; the
// elementwise ops are the same shared functions.  The emitted row and its q8
// codes are bit-identical to the standalone producer's.
// Part 1: issue the loads of this wave's chunk (zeros outside the row).
BQ_DEV void fp_load(f32x4 (&in)[4][4], const FusedQ8& fq, int K, int wave, int lane) {
    const int v0 = wave * kChunk + 16 * lane;
    const int op = fq.op;
#pragma unroll
    for (int i = 0; i < 4; ++i) in[0][i] = in[1][i] = in[2][i] = in[3][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (v0 < K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            in[0][i] = *(const f32x4*)(fq.x + v0 + 4 * i);
            if (op != kOpNorm) in[1][i] = *(const f32x4*)(fq.b + v0 + 4 * i);
            // gate with no sg row: the gate row is already scaled (sg = 1)
            if (op >= kOpResid && op != kOpGateDen)
                in[2][i] = fq.c ? *(const f32x4*)(fq.c + v0 + 4 * i) : f32x4{1.f, 1.f, 1.f, 1.f};
            if (op == kOpSilu) in[3][i] = *(const f32x4*)(fq.d + v0 + 4 * i);
        }
    }
}

// Workgroup sum of per-wave values over the first nch waves, wave order.  Uses
// only LDS waits and s_barrier (no wait on vector memory: the weight loads
// stay in flight).  Every wave of the workgroup must call it.
template <int X>
BQ_DEV void chunk_sum(float (&v)[X], float* red, int wave, int lane, int nch) {
#pragma unroll
    for (int i = 0; i < X; ++i) v[i] = wave_sum_dpp63(v[i]);
    if (lane == 63 && wave < nch)
#pragma unroll
        for (int i = 0; i < X; ++i) red[i * 16 + wave] = v[i];
    asm volatile("" ::: "memory");
    BQ_WAIT_LGKM0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < X; ++i) {
        float t = 0.f;
        for (int k = 0; k < nch; ++k) t += red[i * 16 + k];
        v[i] = t;
    }
}

// Part 2 (after the loads have returned): the producer's row, its L2 norm and
// q8 codes into the LDS activation row (+ workgroup 0's optional outputs).
// red: 48 floats of LDS.  Ends with the LDS writes complete.
template <bool XS>
BQ_DEV void fp_produce(const f32x4 (&in)[4][4], uint8_t* smem, float* red, int K, int wave, int lane,
                       const FusedQ8& fq) {
    const int op = fq.op, nch = (K + kChunk - 1) / kChunk;
    const int v0 = wave * kChunk + 16 * lane;
    f32x4 t[4];
    if (op == kOpResid) {
        float s2[2] = {0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s2[0] += in[0][i][e] * in[0][i][e];
                s2[1] += in[1][i][e] * in[1][i][e];
            }
        chunk_sum<2>(s2, red, wave, lane, nch);
        const float ka = l2_scale(s2[0], K), kb = l2_scale(s2[1], K);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) t[i][e] = resid_blend(in[0][i][e], ka, in[1][i][e], kb, in[2][i][e]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (op == kOpNorm) {
                t[i] = in[0][i];
            } else if (op == kOpAdd) {
                t[i] = in[0][i] + in[1][i];
            } else if (op == kOpGate) {
#pragma unroll
                for (int e = 0; e < 4; ++e) t[i][e] = gate_div(in[0][i][e], in[1][i][e], in[2][i][e]);
            } else if (op == kOpGateDen) {
#pragma unroll
                for (int e = 0; e < 4; ++e) t[i][e] = over_den(in[0][i][e], in[1][i][e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) t[i][e] = silu_mul(in[0][i][e], in[1][i][e], in[2][i][e], in[3][i][e]);
            }
        }
    }
    float ss[1] = {0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss[0] += t[i][e] * t[i][e];
    chunk_sum<1>(ss, red + 32, wave, lane, nch);
    const float k = l2_scale(ss[0], K);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = t[i] * k;
    uint32_t q[4];
    float d;
    int s;
    q8_quant16(t, q, d, s);
    if (v0 < K) {
        uint8_t* lx = smem;
        float* lxd = (float*)(smem + K);
        int32_t* lxs = (int32_t*)(lxd + (K >> 5));
        const int gi = v0 >> 5;
        *(u32x4*)(lx + v0) = u32x4{q[0], q[1], q[2], q[3]};
        if ((lane & 1) == 0) {
            lxd[gi] = d;
            if constexpr (XS) lxs[gi] = s;
        }
        if (blockIdx.x == 0) {
            if (fq.out)
#pragma unroll
                for (int i = 0; i < 4; ++i) *(f32x4*)(fq.out + v0 + 4 * i) = t[i];
            if (fq.xq) {
                *(u32x4*)(fq.xq + v0) = u32x4{q[0], q[1], q[2], q[3]};
                if ((lane & 1) == 0) {
                    fq.xd[gi] = d;
                    fq.xsum[gi] = s;
                }
            }
        }
    }
    asm volatile("" ::: "memory");
    BQ_WAIT_LGKM0();
}

// The scaled copy of a one-row GEMV output: v * s, or (den) the sigmoid
// denominator of that product, 1 + exp(-(v * s)), the value the gate norm
// forms from it (gate_div with sg = 1); the product is rounded to fp32 first,
// as it is when stored and read back
BQ_DEV float scaled_out(float v, float s, int den) {
    float x = v * s;
    if (!den) return x;
    asm("" : "+v"(x));
    return sigmoid_den(x);
}

// ---------------------------------------------------------------------------
// The kernel: blockDim.x / 64 = KS * RT waves per workgroup, a wave owns (tile
// of 4 rows, K slice ks of KS), SPS steps of 16 tasks per row; MR activation
// rows.
// QN > 0: the workgroup quantizes one fp32 activation row itself (q8_quant16,
// bit-exact with k_quant_q8) instead of copying q8 activations.  The row is cut
// into 1024-value chunks, chunk c belongs to wave c % waves (QN = most chunks
// of one wave); the fp32 loads are issued before the weight loads and the
// codes go from registers into LDS.
// QN == kQnProducer: the same with a q8 producer (norm / add / resid / gate /
// silu*mul, then the row L2 norm) in front of the quantizer, one chunk per
// wave (fp_load / fp_produce).
// ---------------------------------------------------------------------------
// Wave priority during the activation staging: the staging loads of a wave
// that starts late queue behind the weight loads other waves of the CU have
// already issued (per-wave timestamps, fused gate+up: the fp32 row landed at
// a median 3.75 us, p90 6.2 us, into a ~9 us kernel).  s_setprio(3) from the
// staging loads through the quantization and the workgroup barrier lets them
// win the issue arbitration; measured (kernel-event medians) gate+up 8.75 ->
// 8.3-8.5 us, QKV 5.6 -> 5.2-5.4, O 5.0 -> 4.7-4.8, decode FFN step 17.66 ->
// 17.12 us.  Raising it only around the loads (1) gained about half of that.
// Large grids (several rounds of workgroups: the 131072-row lm_head at 2..8
// rows) lose with it (54.9 -> 58.0 us at 2 rows), so the launch sets it only
// up to kPrioMaxBlocks workgroups.
constexpr int kPrioMaxBlocks = 4096;

// K slices of a compile-time-K instance with SPS steps per wave
__host__ __device__ constexpr int kc_ks(int K, int sps) { return ((K + 1023) / 1024 + sps - 1) / sps; }

// PAIR: gate and up rows of the same index in one wave (parts 0 and 1, equal
// N): DPP rows 0, 1 take gate rows 2t, 2t+1 and rows 2, 3 the up rows of the
// same indices; the epilogue writes h = silu(g * sg) * u * su (fq.out, with
// sg = fq.c, su = fq.d) instead of the two outputs.  The sums of each row are
// the plain kernel's, so h is bit-identical to silu_mul on its outputs.
template <class F, int MR, int SPS, int QN, int LB, int KC = 0, bool PAIR = false>
__global__ void __launch_bounds__(LB)
k_gemv(PartTable pt, int K_, int KS_, const int8_t* __restrict__ xq, const float* __restrict__ xd,
       const int32_t* __restrict__ xsum, FusedQ8 fq) {
    static_assert(QN == 0 || MR == 1, "fused quantizer / producer: one activation row");
    static_assert(!PAIR || (MR == 1 && QN == 0), "paired silu epilogue: one q8 activation row");
    // KC > 0: the row length, and with it the K split (kc_ks) and the workgroup
    // (LB / 64 waves), is a compile-time constant -- the decode shapes get
    // their own instances
    const int K = KC ? KC : K_;
    const int KS = KC ? kc_ks(KC, SPS) : KS_;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // multi-row Q5_K from kQ5kMfmaMinRows rows: dot products on the matrix
    // cores, lane = 4 * task + row
    constexpr bool kMmLanes = (MR >= kQ5kMfmaMinRows && std::is_same<F, FmtQ5K>::value) ||
                              (MR >= kQ6RepMfmaMinRows && std::is_same<F, FmtQ6KRep>::value) ||
                              (MR >= kQ6RawMfmaMinRows && std::is_same<F, FmtQ6KRaw>::value);
    const int lane = threadIdx.x & 63;
    const int g = kMmLanes ? (lane & 3) : (lane >> 4), li = kMmLanes ? (lane >> 2) : (lane & 15);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
    const int waves = KC ? LB / 64 : blockDim.x >> 6;
    const int nb = K >> 5;
    // ---- 1. activations -> LDS (asynchronous), or this wave's fp32 chunks -> registers
    ActLds act;
    constexpr int kXr0 = act_row_stride(MR, 0);  // 0 or 16: padding per row
    const int xr = K + kXr0;
    act.x = (const int8_t*)smem;
    act.xr = xr;
    act.xd = (const float*)(smem + MR * xr);
    act.xs = (const int32_t*)(act.xd + MR * nb);
    float* part_sums = (float*)(smem + act_lds_bytes<F>(MR, K));  // [waves][MR][4]
    constexpr int QA = QN > 0 ? QN : 1;
    f32x4 xv[QA][4];
    [[maybe_unused]] f32x4 pin[QN < 0 ? 4 : 1][4];
    if (pt.prio) __builtin_amdgcn_s_setprio(3);
    if constexpr (QN > 0) {
        fq_load<QA>(xv, fq.x, K, wave, waves, lane);
    } else if constexpr (QN < 0) {
        fp_load(pin, fq, K, wave, lane);
    } else {
        if constexpr (kXr0 == 0) {
            dma_to_lds(smem, xq, MR * K, wave, waves, lane);
        } else {
#pragma unroll
            for (int r = 0; r < MR; ++r) dma_to_lds(smem + r * xr, xq + (size_t)r * K, K, wave, waves, lane);
        }
        dma_to_lds(smem + MR * xr, xd, MR * nb * 4, wave, waves, lane);
        if constexpr (std::is_same<F, FmtQ5K>::value)
            dma_to_lds(smem + MR * xr + MR * nb * 4, xsum, MR * nb * 4, wave, waves, lane);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's weight loads, all issued now (addresses clamped so the
    //         instruction count is fixed; results of clamped lanes are unused)
    const int RT = waves / KS;  // waves beyond RT * KS only help with the staging
    const int tile = blockIdx.x * RT + wave / KS, ks = wave % KS;
    const bool active = wave < RT * KS && tile < pt.ntiles;
    const int tl = active ? tile : 0;
    // PAIR in the K = 3072 decode instance (one K slice): wave w of the
    // workgroup takes 4 consecutive rows of one matrix (gate for even tiles,
    // up for odd), as the plain two-output launch reads them, and the pair's
    // h comes from both waves through LDS (folded decode chain fold 1 / 2
    // 1.240 / 1.173 -> 1.231 / 1.167 ms/token against 2 gate + 2 up rows
    // per wave); the sums are the same, so h is unchanged
    constexpr bool kSplit = PAIR && KC == 3072 && SPS == 3;
    const int p = PAIR ? 0 : find_part(pt, tl);
    const int Nloc = pt.N[p];
    const int row = kSplit ? (tl >> 1) * kRowsPerTile + g : PAIR ? 2 * tl + (g & 1) : (tl - pt.tile0[p]) * kRowsPerTile + g;
    const int tpr = K >> 6;
    const void* wbase = kSplit ? pt.W[tl & 1] : PAIR ? ((g >> 1) ? pt.W[1] : pt.W[0]) : pt.W[p];
    const uint8_t* rowp = (const uint8_t*)wbase + (size_t)min(row, Nloc - 1) * RowBytes<F>::of(K);
    typename F::Task w[SPS];
    // The fused quantizer's fp32 row comes from memory that the whole grid's
    // weight stream is also queueing on: issued together, the row lands only
    // after several microseconds (measured: median 3.5-4 us, p90 5-6 us, with
    // the compute waiting for it).  With a 9216-value row (36 KB of fp32 per
    // workgroup: the down projection) every wave therefore stages and
    // quantizes first and issues its weight loads after the barrier.  With the
    // 3072 / 4096-value rows of the compile-time-K decode instances the row is
    // a third of that and issuing the weights first measured faster (gate+up
    // 10.3 -> 9.8 us, whole stack 1.008 -> 0.998 ms/token, interleaved A/B).
    // q8 staging (DMA of a row the previous kernel just wrote) stays ahead of
    // the weight loads.  (Issuing all of them early for the 9216-value row
    // measured slower: down 7.4 -> 8.0-8.2 us.)  A q8 producer (QN < 0) reads
    // two or three rows and runs its reductions before any dot, so it takes
    // the late issue at every K.
    constexpr bool kLate = QN < 0 || (QN > 0 && KC != 3072 && KC != 4096);
    // Steps whose loads go out before the staging wait.  With the late issue
    // the first step's loads still go out before it (of two or more steps):
    // for the fused quantizer (down, 2 steps per wave: kernel-event medians
    // 8.19 -> 7.97 us) and for a producer (decode chain, fold = 2: the QKV
    // GEMV with the residual update and the O GEMV with the gate norm 1.291 ->
    // 1.266 ms/token against all steps first, 1.275 with two steps early; the
    // down GEMV with the norm of the silu*mul row 1.256 -> 1.242 against no
    // step early).
    constexpr int kEarly = kLate ? (1 < SPS - 1 ? 1 : SPS - 1) : SPS;
    auto issue_weights = [&](int s0, int s1) {
#pragma unroll
        for (int s = 0; s < SPS; ++s) {
            if (s < s0 || s >= s1) continue;
            const int t = (ks * SPS + s) * kTasksPerStep + li;
            F::load(w[s], rowp, min(t, tpr - 1));
            // keep the steps' loads in step order, so that step s waits only
            // for its own loads (left alone, the scheduler interleaves them)
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    // PAIR: the epilogue's sg and su of the row are loaded now, ahead of the
    // weights, rather than after the last dot (folded decode chain, fold 1
    // 1.237 -> 1.234 ms/token; the same for the scaled gate copy's ss delays
    // a producer's staging wait: fold 2 1.172 -> 1.187)
    [[maybe_unused]] float pre_sg = 0.f, pre_su = 0.f;
    if constexpr (PAIR) {
        const int rr = min(row, Nloc - 1);
        pre_sg = fq.c[rr];
        pre_su = fq.d[rr];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kEarly > 0) issue_weights(0, kEarly);

    // ---- 3. own DMA / fp32 loads done (only the weight loads may still be outstanding)
    BQ_WAIT_VM(F::kLoads * kEarly);
    if constexpr (QN > 0) fq_quantize<QA, std::is_same<F, FmtQ5K>::value>(xv, smem, K, wave, waves, lane, fq);
    if constexpr (QN < 0)
        fp_produce<std::is_same<F, FmtQ5K>::value>(pin, smem, part_sums + waves * MR * 4, K, wave, lane, fq);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_setprio(0);
    if constexpr (kEarly < SPS) issue_weights(kEarly, SPS);

    // ---- 4. compute, step by step as the loads return
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    const bool rowok = active && row < Nloc;
#pragma unroll
    for (int s = 0; s < SPS; ++s) {
        const int t = (ks * SPS + s) * kTasksPerStep + li;
        if constexpr (kMmLanes) {
            // every lane of the block takes part in the matrix instruction;
            // the lane's own contribution is dropped afterwards if not valid
            float tmp[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) tmp[m] = 0.f;
            if constexpr (std::is_same<F, FmtQ5K>::value) q5k_dot_mm<MR>(w[s], min(t, tpr - 1), act, K, tmp, lane);
            if constexpr (std::is_same<F, FmtQ6KRep>::value)
                q6rep_dot_mm<MR>(w[s], min(t, tpr - 1), act, K, tmp, lane);
            if constexpr (std::is_same<F, FmtQ6KRaw>::value)
                FmtQ6KRaw::template dot_mm<MR>(w[s], rowp, min(t, tpr - 1), act, K, tmp, lane);
            if (rowok && t < tpr)
#pragma unroll
                for (int m = 0; m < MR; ++m) acc[m] += tmp[m];
        } else {
            if (rowok && t < tpr) F::template dot<MR>(w[s], rowp, t, act, K, acc);
        }
    }
    // ---- 5. row sums; K slices combined through LDS
    float* Y = pt.Y[p];
    if (KS == 1) {
        if constexpr (kSplit) {
            // tiles 2j, 2j + 1 (gate, up rows 4j..4j+3) are waves 2i, 2i + 1
            const float v = row16_sum(acc[0]);
            if (li == 15) part_sums[wave * 4 + g] = v;
            __syncthreads();
            if ((wave & 1) == 0 && li == 15 && rowok)
                fq.out[row] = silu_mul(v, part_sums[(wave + 1) * 4 + g], pre_sg, pre_su);
            return;
        }
        if constexpr (PAIR) {
            const float v = row16_sum(acc[0]);
            const float u = __shfl(v, lane + 32, 64);  // DPP rows 0, 1 <- 2, 3
            if (g < 2 && li == 15 && rowok)
                fq.out[row] = silu_mul(v, u, pre_sg, pre_su);
            return;
        }
        if constexpr (kMmLanes) {
            // the 16 task lanes 4i + g of a weight row, all MR rows at once
            int m;
            const float v = scatter_sum<MR, 16, 4>(acc, lane, m);
            if ((li & scatter_writers<MR, 16>()) == 0 && m < MR && rowok) Y[(size_t)m * Nloc + row] = v;
        } else {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float v = row16_sum(acc[m]);
                if (li == 15 && rowok) {
                    Y[(size_t)m * Nloc + row] = v;
                    if (MR == 1 && pt.ys && p == pt.sp) pt.ys[row] = scaled_out(v, pt.ss[row], pt.sden);
                }
            }
        }
        return;
    }
    if constexpr (kMmLanes) {
        int m;
        const float v = scatter_sum<MR, 16, 4>(acc, lane, m);
        if ((li & scatter_writers<MR, 16>()) == 0 && m < MR) part_sums[(wave * MR + m) * 4 + g] = v;
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float v = row16_sum(acc[m]);
            if (li == 15) part_sums[(wave * MR + m) * 4 + g] = v;
        }
    }
    __syncthreads();
    if constexpr (PAIR) {
        if (ks == 0 && g < 2 && rowok && li == 15) {
            float v = 0.f, u = 0.f;
            for (int k = 0; k < KS; ++k) {
                v += part_sums[(wave + k) * 4 + g];
                u += part_sums[(wave + k) * 4 + g + 2];
            }
            fq.out[row] = silu_mul(v, u, pre_sg, pre_su);
        }
        return;
    }
    if (ks == 0 && rowok && li == 15) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v = 0.f;
            for (int k = 0; k < KS; ++k) v += part_sums[((wave + k) * MR + m) * 4 + g];
            Y[(size_t)m * Nloc + row] = v;
            if (MR == 1 && pt.ys && p == pt.sp) pt.ys[row] = scaled_out(v, pt.ss[row], pt.sden);
        }
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
static void build_tiles(PartTable& pt, int rows_per_tile = kRowsPerTile) {
    int acc = 0;
    for (int p = 0; p < pt.nparts; ++p) {
        pt.tile0[p] = acc;
        acc += (pt.N[p] + rows_per_tile - 1) / rows_per_tile;
    }
    for (int p = pt.nparts; p < kMaxParts; ++p) pt.tile0[p] = acc;
    pt.ntiles = acc;
}

// K split: ceil(K/1024) steps per row, at most `cap` per wave.  The cap
// decides how many waves share a row (KS = steps / cap) and so the workgroup
// shape and count.  It is chosen per shape class from interleaved sweeps of
// caps 1 / 2 / 3 (kernel-event medians, us; N*K = weight values):
//   fused quantize + GEMV: K > 4096 (down 3072 x 9216): 2 (8.10 -> 7.83);
//     else 3 from 20M values (gate+up 2 x 9216 x 3072: 12.07 -> 9.02), else
//     1 (QKV 5120 x 3072: 5.66 -> 5.40; O 3072 x 4096: 4.84 -> 4.70)
//   Q5_K, q8 input (9216 x 3072 = 28M, 18432 x 3072 = 57M, 3072 x 4096 = 12.6M):
//     4..8 rows (matrix-core dots): 3 from 20M (28M, 8 rows 11.0 -> 9.6; 57M
//       18.9 -> 14.6, 4 rows 13.2 -> 9.7), else 1 (12.6M, 8 rows 8.9 -> 8.3)
//     1..3 rows: 3 from 40M (57M: 1 row 9.4 -> 8.5, 2 rows 10.0 -> 9.4), else
//       1 (12.6M, 2 rows 5.2 -> 4.5; 5120 x 3072, 1 row 5.15 -> 4.97); below
//       12M values 1..2 rows keep 3 (3072 x 3072 tie)
//   Q6_K: 2 once rows * K staged activation bytes per workgroup are large
//     (want several row tiles per workgroup), else 3:
//     raw 3072 x 9216: 3 up to 5 rows (4 rows 10.6 -> 10.2), 2 from 6 rows
//       (rows * K >= 48K; 8 rows 26.7 -> 13.9); 131072 x 3072 (the lm_head):
//       3 for 2..8 rows (8 rows 115 -> 85), 1 row 2 (60.0 -> 57.5)
//     W160 3072 x 9216: 3 up to 2 rows (2 rows 10.2 -> 9.7), else 2 (rows * K
//       >= 27K); 131072 x 3072: 3 for all rows (8 rows 121.6 -> 99)
int sps_cap(GemvKind kind, int K, long long N, int MR, bool fused) {
    if (fused) return K > 4096 ? 2 : (N * K >= (20ll << 20) ? 3 : 1);
    // Q6_K: the staged activation bytes per workgroup (rows * K) decide
    if (kind == GemvKind::Q6KRaw) return MR == 1 ? (K <= 4096 ? 2 : 3) : (MR * K >= 48 * 1024 ? 2 : 3);
    if (kind == GemvKind::Q6KRep) return MR * K >= 3 * 9216 ? 2 : 3;
    const long long nk = N * K;
    if (MR >= kQ5kMfmaMinRows) return nk >= (20ll << 20) ? 3 : 1;
    if (nk >= (40ll << 20)) return 3;
    if (nk < (12ll << 20) && MR <= 2) return 3;
    return 1;
}

void k_split(int K, int cap, int& KS, int& SPS) {
    const int spt = (K / 64 + kTasksPerStep - 1) / kTasksPerStep;
    cap = std::min(3, std::max(cap, (spt + 15) / 16));  // at most 16 slices (K <= 49152)
    KS = (spt + cap - 1) / cap;
    SPS = (spt + KS - 1) / KS;
}

// Workgroup size: 4 waves while K needs at most 4 slices, else 16; the
// workgroup holds RT = waves / KS row tiles and any remaining waves only share
// the activation staging.
static int gemv_waves(int KS) { return KS <= 4 ? 4 : 16; }

// Row tiles per workgroup of a producer-fused one-row GEMV: the launch takes
// about as long as its busiest CU, so take the candidate with the fewest row
// tiles there, ceil(ceil(ntiles / rt) / cus) * rt (the first of equals).  At
// config 5 that is one workgroup per CU: QKV 5120 x 3072 5 tiles (256
// workgroups of 5 waves instead of 320 of 4, 64 CUs holding two), O 3072 x
// 4096 3 tiles x 2 K slices (256 of 6 instead of 384 of 4); the folded
// decode chain, alternated in one process, fold 1 / 2 1.244 / 1.198 -> 1.235 /
// 1.163 ms/token.  Every workgroup still runs the producer over the whole row
// in the same chunk and wave order, so the results are unchanged.  (Sizing
// the q8 / fused-quantizer gate+up to 6 tiles, 3 workgroups per CU, measured
// 8.5 -> 10.2 us: without a producer the 4-wave workgroups stay.)
static int pick_rt(int ntiles, int cus, const int* rts, int n) {
    int best = rts[0];
    long long bc = -1;
    for (int i = 0; i < n; ++i) {
        const long long nb = (ntiles + rts[i] - 1) / rts[i];
        const long long c = (nb + cus - 1) / cus * rts[i];
        if (bc < 0 || c < bc) {
            bc = c;
            best = rts[i];
        }
    }
    return best;
}
template <class F, int MR, int SPS, int QN = 0, bool PAIR = false>
static hipError_t launch_fmt(const PartTable& pt, int K, int KS, const int8_t* xq, const float* xd,
                             const int32_t* xsum, hipStream_t st, FusedQ8 fq = {}) {
    int waves = gemv_waves(KS);
    // the producer needs a wave per 1024-value chunk
    if (QN < 0 && waves < (K + kChunk - 1) / kChunk) waves = 16;
    const int RT = waves / KS;  // the kernel derives the same from blockDim
    const size_t lds = act_lds_bytes<F>(MR, K) + (size_t)waves * MR * 4 * sizeof(float) +
                       (QN != 0 ? 48 * sizeof(float) : 0);
    const int blocks = (pt.ntiles + RT - 1) / RT;
    PartTable ptl = pt;
    ptl.prio = blocks <= kPrioMaxBlocks;
    if (MR == 1 && !PAIR) {
        ScaledCopy& sc = next_scaled_copy();
        for (int q = 0; sc.y && q < pt.nparts; ++q)
            if (pt.W[q] == sc.w) {  // consumed by the launch that holds the part
                ptl.sp = q;
                ptl.ys = sc.y;
                ptl.ss = sc.s;
                ptl.sden = sc.den ? 1 : 0;
                sc = ScaledCopy();
            }
    }
    // the launch-bounds class sets the compiler's occupancy target; the
    // single-row decode shapes run compile-time-K instances
    if constexpr (SPS == 3 && (MR == 1 || QN == 0)) {
        if (waves == 4 && K == 3072 && KS == kc_ks(K, SPS)) {
            if constexpr (MR == 1 && QN < 0) {
                // three 1024-value steps per wave (KS = 1): 4, 5 or 6 row tiles per
                // workgroup (8 never does better than 4 under the rule)
                static constexpr int kRts[] = {4, 5, 6};
                const int rt = pick_rt(pt.ntiles, device_cus(), kRts, 3);
                const int nb = (pt.ntiles + rt - 1) / rt;
                const size_t lr = act_lds_bytes<F>(MR, K) + (size_t)rt * MR * 4 * sizeof(float) + 48 * sizeof(float);
                switch (rt) {
                    case 5: launch_kernel((k_gemv<F, MR, SPS, QN, 320, 3072, PAIR>), dim3(nb), dim3(320), lr, st, ptl, K,
                                          KS, xq, xd, xsum, fq);
                            return hipGetLastError();
                    case 6: launch_kernel((k_gemv<F, MR, SPS, QN, 384, 3072, PAIR>), dim3(nb), dim3(384), lr, st, ptl, K,
                                          KS, xq, xd, xsum, fq);
                            return hipGetLastError();
                    default: break;
                }
            }
            launch_kernel((k_gemv<F, MR, SPS, QN, 256, 3072, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K, KS, xq, xd,
                          xsum, fq);
            return hipGetLastError();
        }
    }
    if constexpr (SPS == 3 && MR == 1) {
        if (waves == 4 && K == 9216 && KS == kc_ks(K, SPS)) {
            launch_kernel((k_gemv<F, MR, SPS, QN, 256, 9216, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K, KS, xq, xd,
                          xsum, fq);
            return hipGetLastError();
        }
    }
    if constexpr (MR == 1 && SPS == 2) {
        if (waves == 4 && K == 4096 && KS == kc_ks(K, SPS)) {
            if constexpr (QN < 0) {
                // two 2048-value steps per wave, 2 K slices: 2 or 3 row tiles per
                // workgroup (4 never does better than 2 under the rule)
                static constexpr int kRts[] = {2, 3};
                const int rt = pick_rt(pt.ntiles, device_cus(), kRts, 2);
                const int nb = (pt.ntiles + rt - 1) / rt;
                const size_t lr = act_lds_bytes<F>(MR, K) + (size_t)2 * rt * MR * 4 * sizeof(float) + 48 * sizeof(float);
                switch (rt) {
                    case 3: launch_kernel((k_gemv<F, MR, SPS, QN, 384, 4096, PAIR>), dim3(nb), dim3(384), lr, st, ptl, K,
                                          KS, xq, xd, xsum, fq);
                            return hipGetLastError();
                    default: break;
                }
            }
            launch_kernel((k_gemv<F, MR, SPS, QN, 256, 4096, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K, KS, xq, xd,
                          xsum, fq);
            return hipGetLastError();
        }
    }
    // one step per wave (the cap-1 K split of the small decode GEMVs: QKV, O,
    // config 3).  K = 3072 splits 3 ways, so a 4-wave workgroup holds one row
    // tile and a wave that only helps the staging: 3-wave workgroups instead
    // (9216 x 3072 at one row: 2304 workgroups, 9216 -> 6912 waves, within one
    // dispatch round of 8 per SIMD; same K split, so the same sums; measured
    // alternating in one process, medians of 12: 5.87 -> 5.73 us, 3072 x 3072
    // level).  A producer keeps 4 waves (one 1024-value chunk per wave).
    if constexpr (MR == 1 && SPS == 1 && QN <= 1) {
        if (waves == 4 && KS == kc_ks(K, SPS) && (K == 3072 || K == 4096)) {
            if (K == 3072 && QN >= 0)
                launch_kernel((k_gemv<F, MR, SPS, QN, 192, 3072, PAIR>), dim3(blocks), dim3(192), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            else if (K == 3072)
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 3072, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            else
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 4096, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            return hipGetLastError();
        }
    }
    // Q5_K verify rows 2..8 at K = 3072 / 4096 (cap-1 / cap-2 K splits)
    if constexpr (QN == 0 && !PAIR && MR > 1 && SPS < 3 && std::is_same<F, FmtQ5K>::value) {
        if (waves == 4 && KS == kc_ks(K, SPS) && (K == 3072 || K == 4096)) {
            // one step per wave at K = 3072: 3-wave workgroups, as for one
            // row (rows 2 / 3 at 9216 x 3072 5.75 -> 5.61 / 6.54 -> 6.24 us,
            // 8 rows at 5120 x 3072 6.06 -> 5.55, 4 rows level; the Q6_K
            // 9216-value rows keep their fourth wave: 3 waves measured 5%
            // slower at 1 and 2 rows, the wave shares a 9 KB staging per row)
            if (K == 3072 && SPS == 1)
                launch_kernel((k_gemv<F, MR, SPS, QN, 192, 3072, PAIR>), dim3(blocks), dim3(192), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            else if (K == 3072)
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 3072, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            else
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 4096, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
            return hipGetLastError();
        }
    }
    // Q6_K (raw and W160) at the down (K = 9216, verify rows) and lm_head
    // (K = 3072, one row) shapes
    if constexpr (QN == 0 && !PAIR && !std::is_same<F, FmtQ5K>::value) {
        if constexpr (SPS == 3 && MR > 1) {
            if (waves == 4 && K == 9216 && KS == kc_ks(K, SPS)) {
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 9216, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
                return hipGetLastError();
            }
        }
        if constexpr (SPS == 2 && MR == 1) {
            if (waves == 4 && K == 3072 && KS == kc_ks(K, SPS)) {
                launch_kernel((k_gemv<F, MR, SPS, QN, 256, 3072, PAIR>), dim3(blocks), dim3(256), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
                return hipGetLastError();
            }
        }
        if constexpr (SPS == 2 && MR > 1) {
            if (waves == 16 && K == 9216 && KS == kc_ks(K, SPS)) {
                launch_kernel((k_gemv<F, MR, SPS, QN, 1024, 9216, PAIR>), dim3(blocks), dim3(1024), lds, st, ptl, K,
                              KS, xq, xd, xsum, fq);
                return hipGetLastError();
            }
        }
    }
    // the fused / producer-fused 9216-value row over 16-wave workgroups (the down projection)
    if constexpr (MR == 1 && SPS == 2 && QN != 0 && !PAIR) {
        if (waves == 16 && K == 9216 && KS == kc_ks(K, SPS)) {
            launch_kernel((k_gemv<F, MR, SPS, QN, 1024, 9216, PAIR>), dim3(blocks), dim3(1024), lds, st, ptl, K, KS,
                          xq, xd, xsum, fq);
            return hipGetLastError();
        }
    }
    if (waves <= 4)
        launch_kernel((k_gemv<F, MR, SPS, QN, 256, 0, PAIR>), dim3(blocks), dim3(64 * waves), lds, st, ptl, K, KS,
                      xq, xd, xsum, fq);
    else
        launch_kernel((k_gemv<F, MR, SPS, QN, 1024, 0, PAIR>), dim3(blocks), dim3(64 * waves), lds, st, ptl, K, KS,
                      xq, xd, xsum, fq);
    return hipGetLastError();
}

template <class F> struct KindOf;
template <> struct KindOf<FmtQ5K> { static constexpr GemvKind v = GemvKind::Q5K; };
template <> struct KindOf<FmtQ6KRaw> { static constexpr GemvKind v = GemvKind::Q6KRaw; };
template <> struct KindOf<FmtQ6KRep> { static constexpr GemvKind v = GemvKind::Q6KRep; };

template <class F, int MR>
static hipError_t dispatch_mr(const PartTable& pt, int K, const int8_t* xq, const float* xd,
                              const int32_t* xsum, hipStream_t st) {
    int KS, SPS;
    k_split(K, sps_cap(KindOf<F>::v, K, (long long)pt.ntiles * kRowsPerTile, MR, false), KS, SPS);
    if (KS > 16) return hipErrorInvalidValue;  // K > 49152
    switch (SPS) {
        case 1: return launch_fmt<F, MR, 1>(pt, K, KS, xq, xd, xsum, st);
        case 2: return launch_fmt<F, MR, 2>(pt, K, KS, xq, xd, xsum, st);
        default: return launch_fmt<F, MR, 3>(pt, K, KS, xq, xd, xsum, st);
    }
}

template <class F>
static hipError_t dispatch_rows(int rows, const PartTable& pt, int K, const int8_t* xq, const float* xd,
                                const int32_t* xsum, hipStream_t st) {
    switch (rows) {
        case 1: return dispatch_mr<F, 1>(pt, K, xq, xd, xsum, st);
        case 2: return dispatch_mr<F, 2>(pt, K, xq, xd, xsum, st);
        case 3: return dispatch_mr<F, 3>(pt, K, xq, xd, xsum, st);
        case 4: return dispatch_mr<F, 4>(pt, K, xq, xd, xsum, st);
        case 5: return dispatch_mr<F, 5>(pt, K, xq, xd, xsum, st);
        case 6: return dispatch_mr<F, 6>(pt, K, xq, xd, xsum, st);
        case 7: return dispatch_mr<F, 7>(pt, K, xq, xd, xsum, st);
        case 8: return dispatch_mr<F, 8>(pt, K, xq, xd, xsum, st);
        default: return hipErrorInvalidValue;
    }
}

size_t gemv_lds_bytes(GemvKind kind, int rows, int K) {
    const size_t partials = (size_t)16 * rows * 4 * sizeof(float);
    switch (kind) {
        case GemvKind::Q5K: return act_lds_bytes<FmtQ5K>(rows, K) + partials;
        case GemvKind::Q6KRaw: return act_lds_bytes<FmtQ6KRaw>(rows, K) + partials;
        default: return act_lds_bytes<FmtQ6KRep>(rows, K) + partials;
    }
}

// rows 1..8 activation rows starting at xq/xd/xsum (already offset)
hipError_t launch_gemv(GemvKind kind, PartTable pt, int rows, int K, const int8_t* xq,
                       const float* xd, const int32_t* xsum, hipStream_t st) {
    build_tiles(pt);
    if (pt.ntiles == 0) return hipSuccess;
    switch (kind) {
        case GemvKind::Q5K: return dispatch_rows<FmtQ5K>(rows, pt, K, xq, xd, xsum, st);
        case GemvKind::Q6KRaw: return dispatch_rows<FmtQ6KRaw>(rows, pt, K, xq, xd, xsum, st);
        default: return dispatch_rows<FmtQ6KRep>(rows, pt, K, xq, xd, xsum, st);
    }
}

// gate and up of one q8 row with the silu*mul epilogue (PAIR): parts 0 and 1
// of pt (equal N), h / sg / su in fq.out / fq.c / fq.d.  The K split is the
// one launch_gemv picks for the two parts, so each row's sum is the same.
template <class F>
static hipError_t dispatch_pair(const PartTable& pt, int K, const int8_t* xq, const float* xd,
                                const int32_t* xsum, const FusedQ8& fq, hipStream_t st) {
    int KS, SPS;
    k_split(K, sps_cap(KindOf<F>::v, K, (long long)pt.ntiles * kRowsPerTile, 1, false), KS, SPS);
    if (KS > 16) return hipErrorInvalidValue;
    switch (SPS) {
        case 1: return launch_fmt<F, 1, 1, 0, true>(pt, K, KS, xq, xd, xsum, st, fq);
        case 2: return launch_fmt<F, 1, 2, 0, true>(pt, K, KS, xq, xd, xsum, st, fq);
        default: return launch_fmt<F, 1, 3, 0, true>(pt, K, KS, xq, xd, xsum, st, fq);
    }
}

hipError_t launch_gemv_silu_pair(GemvKind kind, PartTable pt, int K, const int8_t* xq, const float* xd,
                                 const int32_t* xsum, const float* sg, const float* su, float* h, hipStream_t st) {
    if (pt.nparts != 2 || pt.N[0] != pt.N[1] || pt.N[0] % 4 != 0) return hipErrorInvalidValue;
    build_tiles(pt);
    if (pt.ntiles == 0) return hipSuccess;
    FusedQ8 fq{};
    fq.out = h;
    fq.c = sg;
    fq.d = su;
    switch (kind) {
        case GemvKind::Q5K: return dispatch_pair<FmtQ5K>(pt, K, xq, xd, xsum, fq, st);
        case GemvKind::Q6KRaw: return dispatch_pair<FmtQ6KRaw>(pt, K, xq, xd, xsum, fq, st);
        default: return dispatch_pair<FmtQ6KRep>(pt, K, xq, xd, xsum, fq, st);
    }
}

// fused quantizer: QN = most 1024-value chunks one wave quantizes (<= 3: the
// K split gives KS >= chunks / 3 and waves >= KS)
template <class F, int SPS>
static hipError_t dispatch_fused_qn(const PartTable& pt, int K, int KS, const FusedQ8& fq, hipStream_t st) {
    const int waves = gemv_waves(KS);
    const int qn = (K / kChunk + waves - 1) / waves;
    switch (qn) {
        case 0:
        case 1: return launch_fmt<F, 1, SPS, 1>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
        case 2: return launch_fmt<F, 1, SPS, 2>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
        default: return launch_fmt<F, 1, SPS, 3>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
    }
}

template <class F>
static hipError_t dispatch_fused(const PartTable& pt, int K, const FusedQ8& fq, hipStream_t st) {
    int KS, SPS;
    k_split(K, sps_cap(KindOf<F>::v, K, (long long)pt.ntiles * kRowsPerTile, 1, true), KS, SPS);
    if (K > kFusedMaxK || KS > 16) return hipErrorInvalidValue;
    switch (SPS) {
        case 1: return dispatch_fused_qn<F, 1>(pt, K, KS, fq, st);
        case 2: return dispatch_fused_qn<F, 2>(pt, K, KS, fq, st);
        default: return dispatch_fused_qn<F, 3>(pt, K, KS, fq, st);
    }
}

bool gemv_fused_supported(int K) { return K > 0 && K % 256 == 0 && K <= kFusedMaxK; }
bool gemv_producer_supported(int K) { return K > 0 && K % 256 == 0 && K <= kProducerMaxK; }

template <class F>
static hipError_t dispatch_producer(const PartTable& pt, int K, const FusedQ8& fq, hipStream_t st) {
    // every workgroup redoes the producer, so the split keeps the fewest
    // workgroups (the fused quantizer's cap 1 for small GEMVs measured slower
    // here: folded decode chain 1.51 -> 1.68 ms/token; with the current
    // producers, fold = 2 at cap 3 / 2 / 1 for K <= 4096: 1.199-1.200 /
    // 1.270-1.272 / 1.326-1.327 ms/token)
    int KS, SPS;
    k_split(K, K > 4096 ? 2 : 3, KS, SPS);
    switch (SPS) {
        case 1: return launch_fmt<F, 1, 1, kQnProducer>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
        case 2: return launch_fmt<F, 1, 2, kQnProducer>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
        default: return launch_fmt<F, 1, 3, kQnProducer>(pt, K, KS, nullptr, nullptr, nullptr, st, fq);
    }
}

// q8 producer (op) + GEMV of its one row, fused; out / xq.. optional
hipError_t launch_gemv_producer(GemvKind kind, PartTable pt, int K, int op, float* out, const float* a,
                                const float* b, const float* c, const float* d, int8_t* xq, float* xd,
                                int32_t* xsum, hipStream_t st) {
    if (!gemv_producer_supported(K)) return hipErrorInvalidValue;
    build_tiles(pt);
    if (pt.ntiles == 0)  // no weight rows: the producer's outputs are still written
        return launch_norm_q8(op, out, a, b, c, d, 1, K, xq, xd, xsum, st);
    FusedQ8 fq{a, xq, xd, xsum};
    fq.op = op;
    fq.out = out;
    fq.b = b;
    fq.c = c;
    fq.d = d;
    switch (kind) {
        case GemvKind::Q5K: return dispatch_producer<FmtQ5K>(pt, K, fq, st);
        case GemvKind::Q6KRaw: return dispatch_producer<FmtQ6KRaw>(pt, K, fq, st);
        default: return dispatch_producer<FmtQ6KRep>(pt, K, fq, st);
    }
}

// one fp32 activation row x[K], quantized inside the GEMV; q8 outputs optional
hipError_t launch_gemv_fused_q8(GemvKind kind, PartTable pt, int K, const float* x, int8_t* xq,
                                float* xd, int32_t* xsum, hipStream_t st) {
    if (!gemv_fused_supported(K)) return hipErrorInvalidValue;
    build_tiles(pt);
    const FusedQ8 fq{x, xq, xd, xsum};
    if (pt.ntiles == 0) {
        // no weight rows: the q8 outputs are still produced
        return xq ? launch_quant_q8(x, 1, K, xq, xd, xsum, nullptr, st) : hipSuccess;
    }
    switch (kind) {
        case GemvKind::Q5K: return dispatch_fused<FmtQ5K>(pt, K, fq, st);
        case GemvKind::Q6KRaw: return dispatch_fused<FmtQ6KRaw>(pt, K, fq, st);
        default: return dispatch_fused<FmtQ6KRep>(pt, K, fq, st);
    }
}

}  // namespace bq
