// bq_gemm.hip -- 128x128-tile int8 MFMA prefill GEMMs for gfx950.
//
// Reference semantics (engine/src/bruce.cu):
//   k_gemm_mmq_q5k_144 :6604-6792  Y = sum_g (ds*xd)*dot + sum_g f16(Dm)*f16(xdh)
//   k_gemm_mmq_q5k     :6367-6593  Y = sum_g fma(ds*xd, dot, -dm*(xd*xsum))   (fp32 min term)
//   k_gemm_mma_q6k_128 :6943-7063  Y = sum_g32 xd * (s_lo*dot16_lo + s_hi*dot16_hi)
//
// MI355X design:
//   * Workgroup = 4 waves, tile = 128 weight rows x 128 tokens, each wave a
//     64x64 sub-tile of 2x2 v_mfma_i32_32x32x32_i8 (K = 32 = one Q5_K scale
//     group per instruction, so the per-group scale is applied once per MFMA).
//     Each kernel also has a 32-token tile (4 waves of 32x32, three
//     workgroups per CU), chosen per launch by a work estimate.
//   * K advances in 128-value stages.  The raw tier stages a stage in LDS
//     with a 144-byte row stride (128 codes + 16 B pad: 4-dword bank offset
//     per row, conflict-free 128-bit reads) and prefetches the next stage into
//     registers while the current one is computed; the W144 and Q6_K kernels
//     copy stages with direct-to-LDS loads (below).
//   * The k order inside an MFMA operand is irrelevant to the sum as long as A
//     and B use the same order, so each lane simply loads 16 contiguous bytes.
//   * Scales are staged q-major (sWs[q][row]) so a lane's 4 consecutive
//     accumulator rows read their scales with one ds_read_b128.
//   * Min term: W144 path -- fp16 v_mfma_f32_32x32x16_f16 over (Dm, xdh), once
//     per tile before the main loop (the reference's fp16 semantics); raw path
//     -- exact fp32 v_mfma_f32_32x32x2_f32 on (dmin*m, -(xd*xsum)) per stage.
//   * Blocks are mapped XCD-major: block b runs on XCD b % 8, and each XCD gets
//     a contiguous range of tiles (token tiles fastest) so the tiles that share
//     a weight panel share one L2.
#include "bq_device.hpp"
#include "bq_internal.hpp"

#include <stdlib.h>

#include <algorithm>

namespace bq {

constexpr int kTN = 128;   // weight rows per tile
constexpr int kRS = 144;   // LDS row stride (bytes)
constexpr int kXcds = 8;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct TileMap {
    int mt, nt;  // token tile, weight-row tile (over concatenated parts)
};

BQ_DEV bool map_tile(int b, int ntm, int ntn, TileMap& t) {
    const int ntiles = ntm * ntn;
    const int per = (ntiles + kXcds - 1) / kXcds;
    const int idx = (b % kXcds) * per + b / kXcds;
    if (idx >= ntiles) return false;
    t.mt = idx % ntm;
    t.nt = idx / ntm;
    return true;
}

// Leftover-tile K split.  A launch of T tiles on C CUs runs for as long as its
// busiest CU, which gets ceil(T / C) tiles; with T = q * C + L (0 < L < C)
// every CU but L of them idles for the last tile's duration.  The tail split
// runs the first q * C tiles whole and cuts each of the L leftover tiles into
// k K slices, so the leftover work spreads over L * k pieces; the slices'
// partial tiles go to the caller's workspace [slice][leftover tile][TM][128]
// and k_sum_tail adds them in slice order.  k == 1: no tail split (the
// uniform K split, blockIdx.y, or no split at all).
struct TailSplit {
    int k = 1;        // slices per leftover tile
    int nfull = 0;    // tiles run whole (tile indices 0 .. nfull-1)
    int gridfull = 0; // blocks of the whole tiles (a multiple of the XCD count)
    int nleft = 0;    // leftover tiles (indices nfull .. nfull+nleft-1)
};

// Block -> (tile, slice, slices).  Returns false for a block with no work.
// XCD-major over the whole tiles as map_tile; a leftover tile's k slices are
// consecutive blocks.
BQ_DEV bool map_tile_tail(int b, int ntm, int ntn, const TailSplit& ts, TileMap& t, int& kc, int& ks, int& left) {
    left = -1;
    if (ts.k <= 1) {
        kc = blockIdx.y;
        return map_tile(b, ntm, ntn, t);
    }
    if (b < ts.gridfull) {
        const int per = ts.gridfull / kXcds;
        const int idx = (b % kXcds) * per + b / kXcds;
        if (idx >= ts.nfull) return false;
        t.mt = idx % ntm;
        t.nt = idx / ntm;
        kc = 0;
        ks = 1;
        return true;
    }
    const int j = b - ts.gridfull;
    if (j >= ts.nleft * ts.k) return false;
    left = j / ts.k;
    kc = j % ts.k;
    ks = ts.k;
    const int idx = ts.nfull + left;
    t.mt = idx % ntm;
    t.nt = idx / ntm;
    return true;
}

// offset of slice kc, part p in the K-split workspace [slice][part][rows][N[part]]
BQ_DEV size_t split_offset(const PartTable& pt, int p, int kc, int rows) {
    size_t ntot = 0, off = 0;
#pragma unroll
    for (int i = 0; i < kMaxParts; ++i) {
        if (i < pt.nparts) ntot += pt.N[i];
        if (i < p) off += pt.N[i];
    }
    return ((size_t)kc * ntot + off) * rows;
}

BQ_DEV int part_of_ntile(const PartTable& pt, int& nbase) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxParts; ++i)
        if (i < pt.nparts && nbase >= pt.N[p]) { nbase -= pt.N[p]; p = i; }
    return p;
}

// Token-tile height TM of the prefill kernels (128 or 32, chosen per launch
// by mmq_tile_rows): the weight tile stays 128 rows, the
// four waves form a WN x WM grid of (NT x 32) x (MT x 32) sub-tiles (TM 128:
// 2 x 2 waves of 64 x 64; TM 32: 4 x 1 waves of 32 x 32).
template <int TM>
struct TileGeo {
    static constexpr int WN = TM == 32 ? 4 : 2, WM = 4 / WN;
    static constexpr int NT = kTN / (32 * WN), MT = TM / (32 * WM);
    static_assert(NT * WN * 32 == kTN && MT * WM * 32 == TM && MT >= 1, "tile geometry");
};

// Operands of one group pair (2qp, 2qp+1): this lane's 16 code bytes of each
// weight tile / token tile for both groups.
template <int NT, int MT>
struct PairOps {
    i32x4 a[NT][2], b[MT][2];  // [nt|mt][group of the pair]
};

// int32 -> fp32 on the matrix core.  An int8 dot accumulated onto the bit
// pattern of -1.5 * 2^23 (0xCB400000) is, read as a float, -(12582912 + D)
// for |D| < 2^22 (a 32-value group: |D| <= 32 * 31 * 127 = 125984): adding D
// to the bits moves the value by D units of the binade [2^23, 2^24), whose
// spacing is 1.  One bf16 MFMA whose A and B are the same register r, with
// r[k] = 2048 for k = 0, 1, 2 (lanes 0-31, elements 0-2) and 0 elsewhere, adds
// sum_k r[k] * r[k] = 3 * 2^22 = 12582912 and returns -D, exactly (every term
// is an integer below 2^24).  This replaces the 16 v_cvt_f32_i32 per 32 x 32
// tile and group with one MFMA, which (unlike an fp32 MFMA) runs alongside
// VALU work; the epilogue negates the scale.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
struct MfmaCvt {
    i32x16 bias;
    bf16x8 r;
};
BQ_DEV MfmaCvt mfma_cvt_init(int lane) {
    MfmaCvt c;
#pragma unroll
    for (int i = 0; i < 16; ++i) c.bias[i] = (int)0xCB400000u;
    const __bf16 v = lane < 32 ? (__bf16)2048.f : (__bf16)0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) c.r[i] = i < 3 ? v : (__bf16)0.f;
    return c;
}
// -D as fp32 from the biased int8 dot
BQ_DEV f32x16 mfma_cvt_neg(const MfmaCvt& c, const i32x16& d) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(c.r, c.r, __builtin_bit_cast(f32x16, d), 0, 0, 0);
}

// One 128-value stage (two group pairs) of a wave's 2 x 2 tiles of 32 x 32,
// as eight (group pair, tile) units u.  A unit issues its two int8 dots onto
// the conversion bias, the two-block fp32 outer product of its scales (lanes
// 0-31: group 2qp, lanes 32-63: group 2qp+1) and the two conversions, then
// one FMA per output and group.  The two waves per SIMD overlap each other's
// matrix and VALU work (a software-pipelined form that also issued unit u + 1's
// dots before unit u's FMAs needs more than the 256 registers two waves per
// SIMD allow, and spilled).
//   load_ops(PairOps<2, 2>&, qp)  reads a pair's operands from LDS;
//   scale(qp, nt, mt, lh) -> float2 {ds, xd} for the lane's group of the pair.
template <class LoadOps, class Scale>
BQ_DEV void stage_units_2x2(f32x16 (&acc)[2][2], int lh, const MfmaCvt& cv, LoadOps&& load_ops, Scale&& scale) {
    PairOps<2, 2> o;
    const f32x32 zf = {0.f};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int qp = u >> 2, nt = (u >> 1) & 1, mt = u & 1;
        if ((u & 3) == 0) load_ops(o, qp);
        __builtin_amdgcn_sched_barrier(0);
        const i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[nt][0], o.b[mt][0], cv.bias, 0, 0, 0);
        const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[nt][1], o.b[mt][1], cv.bias, 0, 0, 0);
        const float2 sv = scale(qp, nt, mt, lh);
        const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sv.x, sv.y, zf, 0, 0, 0);
        const f32x16 f0 = mfma_cvt_neg(cv, d0);
        const f32x16 f1 = mfma_cvt_neg(cv, d1);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            acc[nt][mt][r] = __builtin_fmaf(-sc[r], f0[r], acc[nt][mt][r]);
            acc[nt][mt][r] = __builtin_fmaf(-sc[16 + r], f1[r], acc[nt][mt][r]);
        }
    }
}

// LDS layout for one stage
template <int TM>
struct Smem {
    uint8_t w[kTN * kRS];      // weight codes, row stride 144
    uint8_t x[TM * kRS];       // token codes, row stride 144
    float ws[4 * kTN];         // ds   [q][row]
    float xs[4 * TM];          // xd   [q][tok]
    float wm[4 * kTN];         // raw: dmin*m      [q][row]
    float xm[4 * TM];          // raw: -(xd*xsum)  [q][tok]
};

template <int TM>
__global__ void __launch_bounds__(256, TM == 32 ? 3 : 2)
k_mmq_q5k_raw(PartTable pt, int ntm, int ntn, int rows, int K, const int8_t* __restrict__ xq,
              const float* __restrict__ xd, const int32_t* __restrict__ xsum, int ksplit,
              float* __restrict__ part, TailSplit ts) {
    using G = TileGeo<TM>;
    __shared__ __attribute__((aligned(16))) Smem<TM> sm;
    TileMap tm;
    int kc, left;
    if (!map_tile_tail(blockIdx.x, ntm, ntn, ts, tm, kc, ksplit, left)) return;
    int nbase = tm.nt * kTN;
    const int p = part_of_ntile(pt, nbase);
    const int Nloc = pt.N[p];
    const uint8_t* __restrict__ W = (const uint8_t*)pt.W[p];
    const int m0 = tm.mt * TM;
    const int nb = K >> 5, nst = K >> 7, nsb = K >> 8;
    // K split (slice kc of ksplit): stages [s0, s1) of this slice
    const int s0 = kc * nst / ksplit, s1 = (kc + 1) * nst / ksplit;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = (wave / G::WM) * G::NT * 32, t0 = (wave % G::WM) * G::MT * 32;
    const int l32 = lane & 31, lh = lane >> 5;

    f32x16 acc[G::NT][G::MT];
#pragma unroll
    for (int a = 0; a < G::NT; ++a)
#pragma unroll
        for (int b = 0; b < G::MT; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    // ---- register prefetch of one stage -------------------------------------
    // tokens: 8 TM chunks of 16 B (tok = c >> 3, part = c & 7), TM / 32 per
    // thread; token scales: threads 0..TM-1 load xd[tok][4s..4s+3] and xsum.
    u32x4 px[TM / 32];
    f32x4 pxd;
    i32x4 pxs;
    // weights, raw: thread -> (row = tid >> 1, 64-value half hv = tid & 1)
    u32x4 rqs0, rqs1, rqh0, rqh1, rhdr;

    auto load_stage = [&](int s) {
#pragma unroll
        for (int i = 0; i < TM / 32; ++i) {
            const int c = tid + 256 * i, tok = c >> 3, part = c & 7;
            const int m = m0 + tok;
            if (m < rows) px[i] = ld16(xq + (size_t)m * K + 128 * s + 16 * part);
            else px[i] = (u32x4){0, 0, 0, 0};
        }
        if (tid < TM) {
            const int m = m0 + tid;
            if (m < rows) {
                pxd = *(const f32x4*)(xd + (size_t)m * nb + 4 * s);
                pxs = *(const i32x4*)(xsum + (size_t)m * nb + 4 * s);
            } else {
                pxd = (f32x4){0.f, 0.f, 0.f, 0.f};
                pxs = (i32x4){0, 0, 0, 0};
            }
        }
        {
            const int row = tid >> 1, hv = tid & 1;
            const uint8_t* blk = W + ((size_t)(nbase + row) * nsb + (s >> 1)) * kQ5Bytes;
            const int j0 = 4 * (s & 1) + 2 * hv;  // sub-blocks j0, j0 + 1
            rhdr = ld16(blk);
            rqh0 = ld16(blk + 16);
            rqh1 = ld16(blk + 32);
            rqs0 = ld16(blk + 48 + 32 * (j0 >> 1));
            rqs1 = ld16(blk + 64 + 32 * (j0 >> 1));
        }
    };

    auto store_stage = [&](int s) {
#pragma unroll
        for (int i = 0; i < TM / 32; ++i) {
            const int c = tid + 256 * i, tok = c >> 3, part = c & 7;
            *(u32x4*)(sm.x + tok * kRS + 16 * part) = px[i];
        }
        if (tid < TM) {
#pragma unroll
            for (int q = 0; q < 4; ++q) sm.xs[q * TM + tid] = pxd[q];
#pragma unroll
            for (int q = 0; q < 4; ++q) sm.xm[q * TM + tid] = -(pxd[q] * (float)pxs[q]);
        }
        {
            const int row = tid >> 1, hv = tid & 1;
            const int j0 = 4 * (s & 1) + 2 * hv;
            // codes of sub-blocks j0 (low nibbles) and j0+1 (high nibbles), 32 each
            u32x4 lo0, lo1, hi0, hi1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo0[i] = (rqs0[i] & 0x0F0F0F0Fu) | (((rqh0[i] >> j0) & 0x01010101u) << 4);
                lo1[i] = (rqs1[i] & 0x0F0F0F0Fu) | (((rqh1[i] >> j0) & 0x01010101u) << 4);
                hi0[i] = ((rqs0[i] >> 4) & 0x0F0F0F0Fu) | (((rqh0[i] >> (j0 + 1)) & 0x01010101u) << 4);
                hi1[i] = ((rqs1[i] >> 4) & 0x0F0F0F0Fu) | (((rqh1[i] >> (j0 + 1)) & 0x01010101u) << 4);
            }
            uint8_t* dst = sm.w + row * kRS + 64 * hv;
            *(u32x4*)(dst + 0) = lo0;
            *(u32x4*)(dst + 16) = lo1;
            *(u32x4*)(dst + 32) = hi0;
            *(u32x4*)(dst + 48) = hi1;
            const float d = h2f(rhdr.x & 0xFFFF), dmin = h2f(rhdr.x >> 16);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                uint32_t sc, mm;
                q5k_scale_min(rhdr.y, rhdr.z, rhdr.w, j0 + e, sc, mm);
                const int q = 2 * hv + e;
                sm.ws[q * kTN + row] = d * (float)sc;
                sm.wm[q * kTN + row] = dmin * (float)mm;
            }
        }
    };

    load_stage(s0);
    const MfmaCvt cv = mfma_cvt_init(lane);
    for (int s = s0; s < s1; ++s) {
        __syncthreads();  // everyone is done reading the previous stage
        store_stage(s);
        __syncthreads();
        if (s + 1 < s1) load_stage(s + 1);

        // Per group pair (q0, q0+1) and tile: the scale products ds[n] * xd[m]
        // of both groups come from one fp32 outer-product MFMA (32x32x1, two
        // blocks: lanes 0-31 feed group q0, lanes 32-63 group q0+1), so the
        // VALU epilogue is one convert and one FMA per output and group.
#pragma unroll
        for (int qp = 0; qp < 2; ++qp) {
            i32x4 a[G::NT][2], b[G::MT][2];  // [tile][group of the pair]
            float wsv[G::NT], xsv[G::MT];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int q = 2 * qp + e;
#pragma unroll
                for (int nt = 0; nt < G::NT; ++nt)
                    a[nt][e] = *(const i32x4*)(sm.w + (n0 + nt * 32 + l32) * kRS + 32 * q + 16 * lh);
#pragma unroll
                for (int mt = 0; mt < G::MT; ++mt)
                    b[mt][e] = *(const i32x4*)(sm.x + (t0 + mt * 32 + l32) * kRS + 32 * q + 16 * lh);
            }
#pragma unroll
            for (int nt = 0; nt < G::NT; ++nt) wsv[nt] = sm.ws[(2 * qp + lh) * kTN + n0 + nt * 32 + l32];
#pragma unroll
            for (int mt = 0; mt < G::MT; ++mt) xsv[mt] = sm.xs[(2 * qp + lh) * TM + t0 + mt * 32 + l32];
#pragma unroll
            for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
                for (int mt = 0; mt < G::MT; ++mt) {
                    const f32x32 zero32 = {0.f};
                    const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(wsv[nt], xsv[mt], zero32, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        if constexpr (TM == 32) {
                            // matrix-core conversion (mfma_cvt_neg): the 32-token
                            // tile has the registers for it (M = 512: 94-96 ->
                            // 90-91 us); the 128-token tile would spill
                            const i32x16 dd =
                                __builtin_amdgcn_mfma_i32_32x32x32_i8(a[nt][e], b[mt][e], cv.bias, 0, 0, 0);
                            const f32x16 ff = mfma_cvt_neg(cv, dd);
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[nt][mt][r] = __builtin_fmaf(-sc[16 * e + r], ff[r], acc[nt][mt][r]);
                        } else {
                            const i32x16 zero = {0};
                            const i32x16 dd = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[nt][e], b[mt][e], zero, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[nt][mt][r] = __builtin_fmaf(sc[16 * e + r], (float)dd[r], acc[nt][mt][r]);
                        }
                    }
                }
        }
        {
            // exact fp32 min term of the stage's four groups: two K=2 MFMAs per tile
#pragma unroll
            for (int qp = 0; qp < 2; ++qp) {
                const int q = 2 * qp + lh;
                float a[G::NT], b[G::MT];
#pragma unroll
                for (int nt = 0; nt < G::NT; ++nt) a[nt] = sm.wm[q * kTN + n0 + nt * 32 + l32];
#pragma unroll
                for (int mt = 0; mt < G::MT; ++mt) b[mt] = sm.xm[q * TM + t0 + mt * 32 + l32];
#pragma unroll
                for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
                    for (int mt = 0; mt < G::MT; ++mt)
                        acc[nt][mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[nt], b[mt], acc[nt][mt], 0, 0, 0);
            }
        }
    }

    // ---- epilogue: Y[m][n], lane owns token column l32, rows 8*rg + 4*lh + 0..3
    // K split: slice kc's partial sums go to part[kc][part p: rows x N[p]];
    // a leftover tile's slice to its own [TM][128] block of the workspace
    float* __restrict__ Y = pt.Y[p];
    size_t ld = (size_t)Nloc;
    int mo = 0, no = nbase;
    if (left >= 0) {
        Y = part + ((size_t)kc * ts.nleft + left) * (size_t)(kTN * TM);
        ld = kTN;
        mo = m0;
        no = 0;
    } else if (ksplit > 1) {
        Y = part + split_offset(pt, p, kc, rows);
    }
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt) {
        const int m = m0 + t0 + mt * 32 + l32;
        if (m >= rows) continue;
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int n = no + n0 + nt * 32 + 8 * rg + 4 * lh;
                const f32x4 v = {acc[nt][mt][4 * rg], acc[nt][mt][4 * rg + 1], acc[nt][mt][4 * rg + 2],
                                 acc[nt][mt][4 * rg + 3]};
                *(f32x4*)(Y + (size_t)(m - mo) * ld + n) = v;
            }
    }
}

// ---------------------------------------------------------------------------
// W144 prefill GEMM (the k_gemm_mmq_q5k_144 semantics above), DMA-staged.
//   * A stage (128 K values = 4 scale groups) is copied global -> LDS with
//     direct-to-LDS loads (64 lanes x 16 B = 1 KB per instruction, no VGPRs):
//     the 128 W144 rows of the tile are contiguous in global memory and land
//     verbatim (row = 128 codes + 4 fp32 ds, 144-byte stride: conflict-free
//     128-bit reads); token rows land 128 B apart with slot p of token t at
//     p ^ (t & 7), so the 8 lanes of each LDS read phase hit 8 different bank
//     groups; xd lands token-major [tok][4].
//   * Two stage buffers (two LDS objects, the stage loop unrolled by two): the
//     DMA of stage s+1 runs while stage s is computed, one barrier per stage.
//   * Per group pair and 32x32 tile: two v_mfma_i32_32x32x32_i8 dots, the
//     scale products ds[n]*xd[m] of both groups from one two-block fp32
//     outer-product MFMA, then one convert + one FMA per output and group
//     (the 128-token tile converts on the matrix core instead: mfma_cvt_neg).
//     (Measured on gfx950: int8 and bf16 MFMAs overlap independent VALU work,
//     fp32 MFMAs do not, so the outer product costs VALU time; a one-block-
//     per-group variant with the MFMAs of the next unit issued ahead was slower.)
// ---------------------------------------------------------------------------
constexpr int kXS = 128;  // token row stride in LDS (bytes)

template <int TM>
struct SmemStage {
    uint8_t w[kTN * kW144];  // 18432 B: W144 rows verbatim
    uint8_t x[TM * kXS];     // token codes, swizzled 16-byte slots
    float xs[TM * 4];        // xd[tok][q]
};

// Direct-to-LDS 16-byte load: lane i's 16 bytes from gbase + voff land at
// LDS address lds + 16 * i.  Issued through asm so that the compiler does not
// treat LDS reads of the other stage buffer, or the min term's global loads,
// as dependent on it (with __builtin_amdgcn_global_load_lds it waits for
// vmcnt(0) before them: 9216 x 3072 at M = 512 / 2048 / 8192 took 75 / 202 /
// 765 us against 66 / 198 / 750 us with this asm); the kernel orders the
// copies itself (vmcnt(0) + barrier before a buffer is read).  An untracked
// VMEM op can only make the compiler's own vmcnt waits stricter, never looser.
// m0 is written here; the compiler warns that it reserves m0 and will not
// preserve it around the asm, which is safe because no other instruction of
// these kernels reads or writes m0 (LDS instructions do not on gfx9; the
// kernels have no other direct-to-LDS loads, s_sendmsg, or relative register
// indexing).  tests/test_isa_m0.py checks that on the built code object.
BQ_DEV void dma16(const void* gbase, uint32_t voff, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(gbase), "s"(m0)
                 : "m0", "memory");
}

// One stage's DMA; every wave issues instructions c = wave + 4i.  Per-lane
// offsets are loop invariant (token slot swizzle: tok & 7 == lane >> 3), the
// rest is wave-uniform.  Token rows past `rows` are skipped (their LDS slots
// keep stale bytes; those outputs are never stored).
struct Mmq144Dma {
    uint32_t w_off, x_off, xd_off;  // per lane
    int tok_hi;                     // lane >> 3
};

template <int TM>
BQ_DEV void mmq144_dma(SmemStage<TM>& sb, const uint8_t* wsrc, const int8_t* xq, const float* xd,
                       const Mmq144Dma& o, int m0, int rows, int K, int nb, int s, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int c = wave + 4 * i;
        if (c < 18) dma16(wsrc + 1024 * c, o.w_off, sb.w + 1024 * c);
    }
    const int8_t* xs0 = xq + (size_t)m0 * K + 128 * s;
#pragma unroll
    for (int i = 0; i < TM / 32; ++i) {
        const int c = wave + 4 * i;
        if (m0 + 8 * c + o.tok_hi < rows) dma16(xs0 + (size_t)(8 * c) * K, o.x_off, sb.x + 1024 * c);
    }
    if (wave < (TM + 63) / 64 && 64 * wave + lane < TM && m0 + 64 * wave + lane < rows)
        dma16(xd + (size_t)(m0 + 64 * wave) * nb + 4 * s, o.xd_off, (uint8_t*)sb.xs + 1024 * wave);
}

template <int TM>
BQ_DEV void mmq144_ops(PairOps<TileGeo<TM>::NT, TileGeo<TM>::MT>& o, const SmemStage<TM>& sb, int qp, int n0,
                       int t0, int l32, int lh) {
    using G = TileGeo<TM>;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int g = 2 * qp + e;
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
            o.a[nt][e] = *(const i32x4*)(sb.w + (n0 + nt * 32 + l32) * kW144 + 32 * g + 16 * lh);
#pragma unroll
        for (int mt = 0; mt < G::MT; ++mt) {
            const int tok = t0 + mt * 32 + l32;
            o.b[mt][e] = *(const i32x4*)(sb.x + tok * kXS + 16 * ((2 * g + lh) ^ (tok & 7)));
        }
    }
}

// One stage.  Per group pair and tile: the scale products of both groups come
// from one two-block fp32 outer-product MFMA (lanes 0-31 feed group 2qp,
// lanes 32-63 group 2qp+1), the two dots from two int8 MFMAs, then one convert
// and one FMA per output and group.  The next pair's operands are read from
// LDS while this pair is computed.  n0 / t0: the wave's first weight row /
// token in the tile.
template <int TM>
BQ_DEV void mmq144_stage(const SmemStage<TM>& sb, f32x16 (&acc)[TileGeo<TM>::NT][TileGeo<TM>::MT], int n0,
                         int t0, int l32, int lh) {
    using G = TileGeo<TM>;
    f32x4 wsq[G::NT], xsq[G::MT];  // the stage's four scales per weight row / token: one 16-byte read each
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) wsq[nt] = *(const f32x4*)(sb.w + (n0 + nt * 32 + l32) * kW144 + 128);
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt) xsq[mt] = *(const f32x4*)(sb.xs + 4 * (t0 + mt * 32 + l32));
    PairOps<G::NT, G::MT> cur;
    mmq144_ops<TM>(cur, sb, 0, n0, t0, l32, lh);
#pragma unroll 1
    for (int qp = 0; qp < 2; ++qp) {
        PairOps<G::NT, G::MT> nxt;
        mmq144_ops<TM>(nxt, sb, 1, n0, t0, l32, lh);  // qp = 1: harmless reread
        float wsv[G::NT], xsv[G::MT];
#pragma unroll
        for (int t = 0; t < G::NT; ++t) wsv[t] = qp ? (lh ? wsq[t][3] : wsq[t][2]) : (lh ? wsq[t][1] : wsq[t][0]);
#pragma unroll
        for (int t = 0; t < G::MT; ++t) xsv[t] = qp ? (lh ? xsq[t][3] : xsq[t][2]) : (lh ? xsq[t][1] : xsq[t][0]);
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < G::MT; ++mt) {
                const f32x32 zf = {0.f};
                const i32x16 zi = {0};
                const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(wsv[nt], xsv[mt], zf, 0, 0, 0);
                const i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[nt][0], cur.b[mt][0], zi, 0, 0, 0);
                const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[nt][1], cur.b[mt][1], zi, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[nt][mt][r] = __builtin_fmaf(sc[r], (float)d0[r], acc[nt][mt][r]);
                    acc[nt][mt][r] = __builtin_fmaf(sc[16 + r], (float)d1[r], acc[nt][mt][r]);
                }
            }
        cur = nxt;
    }
}

// The same stage for the 2 x 2 tiles of a 128-token tile's wave, through
// stage_units_2x2 (matrix-core conversions).  The scales are read once per
// stage, 16 bytes per weight row and token (conflict-free; per-unit 4-byte
// reads at the 144-byte row stride hit 8 banks: 4-way conflicts, measured
// 2-3% slower), and narrowed to the lane half's groups lh and lh + 2.
template <int TM>
BQ_DEV void mmq144_stage_units(const SmemStage<TM>& sb, f32x16 (&acc)[TileGeo<TM>::NT][TileGeo<TM>::MT], int n0,
                               int t0, int l32, int lh, const MfmaCvt& cv) {
    using G = TileGeo<TM>;
    static_assert(G::NT == 2 && G::MT == 2, "four tiles per wave");
    // the stage's four scales per weight row / token as one 16-byte read
    // each, narrowed at once to the lane half's two groups (lh, lh + 2)
    float2 ws2[2], xs2[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const f32x4 w4 = *(const f32x4*)(sb.w + (n0 + t * 32 + l32) * kW144 + 128);
        const f32x4 x4 = *(const f32x4*)(sb.xs + 4 * (t0 + t * 32 + l32));
        ws2[t] = make_float2(lh ? w4[1] : w4[0], lh ? w4[3] : w4[2]);
        xs2[t] = make_float2(lh ? x4[1] : x4[0], lh ? x4[3] : x4[2]);
    }
    stage_units_2x2(
        acc, lh, cv, [&](PairOps<2, 2>& o, int qp) { mmq144_ops<TM>(o, sb, qp, n0, t0, l32, lh); },
        [&](int qp, int nt, int mt, int) {
            return make_float2(qp ? ws2[nt].y : ws2[nt].x, qp ? xs2[mt].y : xs2[mt].x);
        });
}

// The 128-token tile takes stage_units_2x2 (with its matrix-core conversions
// measured 1-2% faster than converts on the VALU at M = 2048 / 8192); the
// 32-token tile has one tile per wave.
template <int TM>
BQ_DEV void mmq144_stage_any(const SmemStage<TM>& sb, f32x16 (&acc)[TileGeo<TM>::NT][TileGeo<TM>::MT], int n0,
                             int t0, int l32, int lh, const MfmaCvt& cv) {
    if constexpr (TileGeo<TM>::NT * TileGeo<TM>::MT == 4)
        mmq144_stage_units<TM>(sb, acc, n0, t0, l32, lh, cv);
    else
        mmq144_stage<TM>(sb, acc, n0, t0, l32, lh);
}

// Eight consecutive xdh values half(xd * xsum) of one token row.  The
// product is rounded to fp32 first: the empty asm keeps the compiler from
// fusing the multiply and the fp16 conversion into one single-rounding
// v_fma_mix, and, not being volatile, it does not order the batch's loads.
BQ_DEV f16x8 xdh8(const float* __restrict__ xd, const int32_t* __restrict__ xs) {
    const f32x4 d0 = *(const f32x4*)xd, d1 = *(const f32x4*)(xd + 4);
    const i32x4 s0 = *(const i32x4*)xs, s1 = *(const i32x4*)(xs + 4);
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float p = (i < 4 ? d0[i] : d1[i - 4]) * (float)(i < 4 ? s0[i] : s1[i - 4]);
        asm("" : "+v"(p));
        h[i] = (_Float16)p;
    }
    return h;
}

// XI: the tile forms xdh itself from xd and xsum (32-token tile only)
template <int TM, bool XI = false>
__global__ void __launch_bounds__(256, TM == 32 ? 3 : 2)
k_mmq_w144(PartTable pt, int ntm, int ntn, int rows, int K, const int8_t* __restrict__ xq,
           const float* __restrict__ xd, const int32_t* __restrict__ xsum, const uint16_t* __restrict__ xdh,
           int ksplit, float* __restrict__ part, TailSplit ts) {
    using G = TileGeo<TM>;
    __shared__ __attribute__((aligned(16))) SmemStage<TM> sm0;
    __shared__ __attribute__((aligned(16))) SmemStage<TM> sm1;
    TileMap tm;
    int kc, left;
    if (!map_tile_tail(blockIdx.x, ntm, ntn, ts, tm, kc, ksplit, left)) return;
    int nbase = tm.nt * kTN;
    const int p = part_of_ntile(pt, nbase);
    const int Nloc = pt.N[p];
    const uint8_t* __restrict__ W = (const uint8_t*)pt.W[p];
    const int m0 = tm.mt * TM;
    const int nb = K >> 5, nst = K >> 7;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = (wave / G::WM) * G::NT * 32, t0 = (wave % G::WM) * G::MT * 32;
    const int l32 = lane & 31, lh = lane >> 5;
    auto wsrc = [&](int s) { return W + ((size_t)s * Nloc + nbase) * kW144; };
    // K split (slice kc of ksplit): stage pairs [s0, s1) of this slice
    const int s0 = 2 * (kc * (nst / 2) / ksplit), s1 = 2 * ((kc + 1) * (nst / 2) / ksplit);
    Mmq144Dma dof;
    dof.tok_hi = lane >> 3;
    dof.w_off = 16 * lane;
    dof.x_off = (uint32_t)(lane >> 3) * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
    dof.xd_off = (uint32_t)lane * (uint32_t)(nb * 4);

    mmq144_dma<TM>(sm0, wsrc(s0), xq, xd, dof, m0, rows, K, nb, s0, wave, lane);
    const MfmaCvt cv = mfma_cvt_init(lane);

    f32x16 acc[G::NT][G::MT];
#pragma unroll
    for (int a = 0; a < G::NT; ++a)
#pragma unroll
        for (int b = 0; b < G::MT; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
    // min term: sum_g f16(Dm[n][g]) * f16(xdh[m][g]) on fp16 MFMA, K/32 % 16 == 0
    // (the first K slice only).  xdh is filled by k_fill_xdh before the
    // launch, except for calls of at most kXdhInlineRows rows (32-token tile
    // only, XI), where that launch is a tenth of the call: there each
    // tile forms xdh[m][g] = half(xd * xsum) itself, rounded as k_fill_xdh
    // rounds it (bruce.cu:6598-6602: to fp32, then to fp16).  The
    // operands of up to kMinBatch 16-group chunks are loaded before the first
    // of their MFMAs, so a tile waits for one global-load latency per batch
    // instead of one per chunk (the MFMA order, and so the sum, is the chunk
    // order either way).
    if (kc == 0) {
        constexpr int kMinBatch = 6;
        const uint16_t* __restrict__ Dm = (const uint16_t*)pt.aux[p];
        for (int g0 = 0; g0 < nb; g0 += 16 * kMinBatch) {
            f16x8 a[kMinBatch][G::NT], b[kMinBatch][G::MT];
#pragma unroll
            for (int c = 0; c < kMinBatch; ++c) {
                const int g = min(g0 + 16 * c, nb - 16);
#pragma unroll
                for (int nt = 0; nt < G::NT; ++nt) {
                    const int n = nbase + n0 + nt * 32 + l32;
                    a[c][nt] = *(const f16x8*)(Dm + (size_t)n * nb + g + 8 * lh);
                }
#pragma unroll
                for (int mt = 0; mt < G::MT; ++mt) {
                    const int m = min(m0 + t0 + mt * 32 + l32, rows - 1);
                    if constexpr (XI)
                        b[c][mt] = xdh8(xd + (size_t)m * nb + g + 8 * lh, xsum + (size_t)m * nb + g + 8 * lh);
                    else
                        b[c][mt] = *(const f16x8*)(xdh + (size_t)m * nb + g + 8 * lh);
                }
            }
#pragma unroll
            for (int c = 0; c < kMinBatch; ++c) {
                if (g0 + 16 * c >= nb) break;
#pragma unroll
                for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
                    for (int mt = 0; mt < G::MT; ++mt)
                        acc[nt][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c][nt], b[c][mt], acc[nt][mt], 0, 0, 0);
            }
        }
    }

    for (int s = s0; s < s1; s += 2) {
        BQ_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 1 < s1) mmq144_dma<TM>(sm1, wsrc(s + 1), xq, xd, dof, m0, rows, K, nb, s + 1, wave, lane);
        mmq144_stage_any<TM>(sm0, acc, n0, t0, l32, lh, cv);
        if (s + 1 >= s1) break;
        BQ_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 2 < s1) mmq144_dma<TM>(sm0, wsrc(s + 2), xq, xd, dof, m0, rows, K, nb, s + 2, wave, lane);
        mmq144_stage_any<TM>(sm1, acc, n0, t0, l32, lh, cv);
    }

    // K split: slice kc's partial sums go to part[kc][part p: rows x N[p]];
    // a leftover tile's slice to its own [TM][128] block of the workspace
    float* __restrict__ Y = pt.Y[p];
    size_t ld = (size_t)Nloc;
    int mo = 0, no = nbase;
    if (left >= 0) {
        Y = part + ((size_t)kc * ts.nleft + left) * (size_t)(kTN * TM);
        ld = kTN;
        mo = m0;
        no = 0;
    } else if (ksplit > 1) {
        Y = part + split_offset(pt, p, kc, rows);
    }
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt) {
        const int m = m0 + t0 + mt * 32 + l32;
        if (m >= rows) continue;
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int n = no + n0 + nt * 32 + 8 * rg + 4 * lh;
                const f32x4 v = {acc[nt][mt][4 * rg], acc[nt][mt][4 * rg + 1], acc[nt][mt][4 * rg + 2],
                                 acc[nt][mt][4 * rg + 3]};
                *(f32x4*)(Y + (size_t)(m - mo) * ld + n) = v;
            }
    }
}

// y of the leftover tiles = the sum of their k slices (fixed slice order), one
// float4 per thread: thread i -> tile i / (TM * 32), token row, 4 columns
template <int TM>
__global__ void __launch_bounds__(256) k_sum_tail(const float* __restrict__ ws, PartTable pt, int ntm, int rows,
                                                  TailSplit ts) {
    const size_t per = (size_t)TM * (kTN / 4);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= per * ts.nleft) return;
    const int left = (int)(i / per);
    const int e = (int)(i % per), ml = e / (kTN / 4), c4 = e % (kTN / 4);
    const int idx = ts.nfull + left;
    const int m = (idx % ntm) * TM + ml;
    if (m >= rows) return;
    int nbase = (idx / ntm) * kTN;
    const int p = part_of_ntile(pt, nbase);
    const size_t slice = (size_t)ts.nleft * kTN * TM;
    const f32x4* src = (const f32x4*)(ws + (size_t)left * kTN * TM) + e;
    f32x4 v = src[0];
    for (int k = 1; k < ts.k; ++k) v = v + src[k * (slice / 4)];
    *(f32x4*)(pt.Y[p] + (size_t)m * pt.N[p] + nbase + 4 * c4) = v;
}

// ---------------------------------------------------------------------------
// Q6_K over W160 (k_gemm_mma_q6k_128 semantics: one K = 16 MFMA per 16-value
// scale group), DMA-staged like k_mmq_w144.
//   * W160 is row-major ([N][K/128][160]), so a stage's 128 rows are 160 B
//     apart only within a row: the codes (bytes 0..127 of a row's stage) land
//     128 B apart with 16-byte slot p of row r at p ^ f(r), f(r) = (r >> 1) & 7
//     (the 8-byte operand reads of 32 rows then hit each bank pair at most
//     twice, as with the old 144-byte stride), and the eight d*sc floats
//     (bytes 128..159) land [row][8].  Tokens as the codes, xd as [tok][4].
//   * 16 + 4 + 16 + 2 direct-to-LDS instructions per stage, two stage buffers
//     (2 x 38 KB: two workgroups per CU), one barrier per stage.
// ---------------------------------------------------------------------------
template <int TM>
struct SmemQ6Stage {
    uint8_t w[kTN * 128];  // 16384 B: codes, swizzled 16-byte slots
    uint8_t x[TM * 128];   // token codes, same swizzle
    float ws[kTN * 8];     //  4096 B: d*sc [row][g16]
    float xs[TM * 4];      // xd [tok][q]
};

BQ_DEV int q6_swz(int r) { return (r >> 1) & 7; }

struct Q6Dma {
    uint32_t w_off;   // codes, per lane (a wave issues instructions c = wave + 4i: c & 1 = wave & 1)
    uint32_t s_off;   // scales, per lane
    uint32_t x_off;   // tokens, per lane
    uint32_t xd_off;
    int tok_hi;         // lane >> 3
};

template <int TM>
BQ_DEV void q6_dma(SmemQ6Stage<TM>& sb, const uint8_t* wstage, uint32_t row_bytes, const int8_t* xq, const float* xd,
                   const Q6Dma& o, int m0, int rows, int K, int nb, int s, int wave, int lane) {
    // weight codes: instruction c = rows 8c..8c+7
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = wave + 4 * i;
        dma16(wstage + (size_t)(8 * c) * row_bytes, o.w_off, sb.w + 1024 * c);
    }
    // weight scales: instruction c = rows 32c..32c+31 (one per wave)
    dma16(wstage + (size_t)(32 * wave) * row_bytes, o.s_off, (uint8_t*)sb.ws + 1024 * wave);
    // tokens: instruction c = tokens 8c..8c+7 (rows past `rows` skipped)
    const int8_t* xs0 = xq + (size_t)m0 * K + 128 * s;
#pragma unroll
    for (int i = 0; i < TM / 32; ++i) {
        const int c = wave + 4 * i;
        if (m0 + 8 * c + o.tok_hi < rows) dma16(xs0 + (size_t)(8 * c) * K, o.x_off, sb.x + 1024 * c);
    }
    if (wave < (TM + 63) / 64 && 64 * wave + lane < TM && m0 + 64 * wave + lane < rows)
        dma16(xd + (size_t)(m0 + 64 * wave) * nb + 4 * s, o.xd_off, (uint8_t*)sb.xs + 1024 * wave);
}

// One stage: per 32-group q and tile, the two-block fp32 outer product of the
// scales of the 16-groups 2q (lanes 0-31) and 2q+1 (lanes 32-63), the two
// int8 K=16 dots onto the conversion bias and their matrix-core conversions,
// then one FMA per output and 16-group (measured against converts on the
// VALU: 3072 x 9216 at M = 2048, 359-369 -> 335-355 us).
// n0 / t0: the wave's first weight row / token in the tile.
template <int TM>
BQ_DEV void q6_stage(const SmemQ6Stage<TM>& sb, f32x16 (&acc)[TileGeo<TM>::NT][TileGeo<TM>::MT], int n0, int t0,
                     int l32, int lh, const MfmaCvt& cv) {
    using G = TileGeo<TM>;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        long a[G::NT][2], b[G::MT][2];  // [tile][16-group half]
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int nt = 0; nt < G::NT; ++nt) {
                const int r = n0 + nt * 32 + l32;
                a[nt][h] = *(const long*)(sb.w + r * 128 + 16 * ((2 * q + h) ^ q6_swz(r)) + 8 * lh);
            }
#pragma unroll
            for (int mt = 0; mt < G::MT; ++mt) {
                const int t = t0 + mt * 32 + l32;
                b[mt][h] = *(const long*)(sb.x + t * 128 + 16 * ((2 * q + h) ^ q6_swz(t)) + 8 * lh);
            }
        }
        float wsv[G::NT], xsv[G::MT];
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt) wsv[nt] = sb.ws[8 * (n0 + nt * 32 + l32) + 2 * q + lh];
#pragma unroll
        for (int mt = 0; mt < G::MT; ++mt) xsv[mt] = sb.xs[4 * (t0 + mt * 32 + l32) + q];
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < G::MT; ++mt) {
                const f32x32 zero32 = {0.f};
                const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(wsv[nt], xsv[mt], zero32, 0, 0, 0);
                // 16-value dots: |D| <= 16 * 32 * 127 < 2^22, so the biased
                // dot converts on the matrix core exactly (mfma_cvt_neg)
                const i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a[nt][0], b[mt][0], cv.bias, 0, 0, 0);
                const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a[nt][1], b[mt][1], cv.bias, 0, 0, 0);
                const f32x16 f0 = mfma_cvt_neg(cv, d0);
                const f32x16 f1 = mfma_cvt_neg(cv, d1);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[nt][mt][r] = __builtin_fmaf(-sc[r], f0[r], acc[nt][mt][r]);
                    acc[nt][mt][r] = __builtin_fmaf(-sc[16 + r], f1[r], acc[nt][mt][r]);
                }
            }
    }
}

template <int TM>
__global__ void __launch_bounds__(256, TM == 32 ? 3 : 2)
k_mmq_q6k_dma(PartTable pt, int ntm, int ntn, int rows, int K, const int8_t* __restrict__ xq,
              const float* __restrict__ xd, int ksplit, float* __restrict__ part) {
    using G = TileGeo<TM>;
    __shared__ __attribute__((aligned(16))) SmemQ6Stage<TM> sm0;
    __shared__ __attribute__((aligned(16))) SmemQ6Stage<TM> sm1;
    TileMap tm;
    if (!map_tile(blockIdx.x, ntm, ntn, tm)) return;
    int nbase = tm.nt * kTN;
    const int p = part_of_ntile(pt, nbase);
    const int Nloc = pt.N[p];
    const uint8_t* __restrict__ W = (const uint8_t*)pt.W[p];
    const int m0 = tm.mt * TM;
    const int nb = K >> 5, nst = K >> 7;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = (wave / G::WM) * G::NT * 32, t0 = (wave % G::WM) * G::MT * 32;
    const int l32 = lane & 31, lh = lane >> 5;
    const uint32_t row_bytes = (uint32_t)nst * kW160;
    auto wstage = [&](int s) { return W + (size_t)nbase * row_bytes + (size_t)s * kW160; };
    Q6Dma o;
    o.tok_hi = lane >> 3;
    // codes: lane -> row (lane >> 3) of the instruction, LDS slot lane & 7,
    // global slot (lane & 7) ^ f(8c + (lane >> 3)); f depends on c only via
    // c & 1, which is wave & 1 for every instruction of this wave
    {
        const uint32_t sw = q6_swz(8 * (wave & 1) + (lane >> 3));
        o.w_off = (uint32_t)(lane >> 3) * row_bytes + 16u * ((lane & 7) ^ sw);
        o.x_off = (uint32_t)(lane >> 3) * (uint32_t)K + 16u * ((lane & 7) ^ sw);
    }
    o.s_off = (uint32_t)(lane >> 1) * row_bytes + 128u + 16u * (uint32_t)(lane & 1);
    o.xd_off = (uint32_t)lane * (uint32_t)(nb * 4);

    // K split (blockIdx.y of ksplit): stage pairs [s0, s1) of this slice
    const int kc = blockIdx.y;
    const int s0 = 2 * (kc * (nst / 2) / ksplit), s1 = 2 * ((kc + 1) * (nst / 2) / ksplit);
    q6_dma<TM>(sm0, wstage(s0), row_bytes, xq, xd, o, m0, rows, K, nb, s0, wave, lane);
    const MfmaCvt cv = mfma_cvt_init(lane);

    f32x16 acc[G::NT][G::MT];
#pragma unroll
    for (int a = 0; a < G::NT; ++a)
#pragma unroll
        for (int b = 0; b < G::MT; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    for (int s = s0; s < s1; s += 2) {
        BQ_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 1 < s1) q6_dma<TM>(sm1, wstage(s + 1), row_bytes, xq, xd, o, m0, rows, K, nb, s + 1, wave, lane);
        q6_stage<TM>(sm0, acc, n0, t0, l32, lh, cv);
        if (s + 1 >= s1) break;
        BQ_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 2 < s1) q6_dma<TM>(sm0, wstage(s + 2), row_bytes, xq, xd, o, m0, rows, K, nb, s + 2, wave, lane);
        q6_stage<TM>(sm1, acc, n0, t0, l32, lh, cv);
    }

    // K split: slice kc's partial sums go to part[kc][part p: rows x N[p]]
    float* __restrict__ Y = ksplit > 1 ? part + split_offset(pt, p, kc, rows) : pt.Y[p];
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt) {
        const int m = m0 + t0 + mt * 32 + l32;
        if (m >= rows) continue;
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int n = nbase + n0 + nt * 32 + 8 * rg + 4 * lh;
                const f32x4 v = {acc[nt][mt][4 * rg], acc[nt][mt][4 * rg + 1], acc[nt][mt][4 * rg + 2],
                                 acc[nt][mt][4 * rg + 3]};
                *(f32x4*)(Y + (size_t)m * Nloc + n) = v;
            }
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
static int ntile_count(const PartTable& pt) {
    int n = 0;
    for (int p = 0; p < pt.nparts; ++p) n += pt.N[p] / kTN;
    return n;
}

static int ntotal(const PartTable& pt) {
    int n = 0;
    for (int p = 0; p < pt.nparts; ++p) n += pt.N[p];
    return n;
}

static dim3 mmq_grid(int ntm, int ntn) {
    const int ntiles = ntm * ntn;
    const int per = (ntiles + kXcds - 1) / kXcds;
    return dim3(per * kXcds);
}

// K split.  A launch with fewer tiles than the workgroup slots (two per CU
// for the 128-token tiles, three for the 32-token tiles; 512 / 768 on
// MI355X's 256 CUs) leaves CUs idle (one
// token tile of a 9216-row matrix: 72 tiles), so it
// is split over K into up to kMaxKSplit slices of whole K units (stage pairs
// for the DMA-staged kernels, stages for the raw tier) when the caller's
// workspace holds the slices' partial outputs [slice][part][rows][N[part]];
// one more launch sums them in a fixed order.  The choice depends only on the
// shape and the workspace size, so equal calls take equal paths (eager or
// captured in a graph) and give equal bits.
constexpr int kMaxKSplit = 8;

// `cus` below: the CU count of the device the launch runs on (MI355X: 256),
// which sets the workgroup slots every split and tile-height choice counts.
int mmq_ksplit(int rows, int K, int ntot, bool stage_units, size_t ws_floats, int tm, int cus) {
    const int ntiles = ((rows + tm - 1) / tm) * (ntot / kTN);
    if (ntiles <= 0) return 1;
    const int units = stage_units ? (K >> 7) : (K >> 8);
    const int slots = (tm == 32 ? 3 : 2) * cus;  // workgroups resident at once (3 or 2 per CU)
    int ks = std::min(kMaxKSplit, std::max(1, slots / ntiles));
    while (ks > 1 && ((size_t)ks * rows * ntot > ws_floats || units < ks)) --ks;
    // the fewest slices with the same longest slice (fewer partial outputs)
    const int per = (units + ks - 1) / ks;
    return (units + per - 1) / per;
}

// Token-tile height (128 or 32) of the DMA-staged kernels for a launch: the
// one with the smaller estimated work on the busiest CU, ceil(workgroups /
// CUs) x tile height x the longest K slice, the 32-token tile's work
// weighted by e32 (its cost per output relative to the 128-token tile on a
// full GPU, measured at 4096 rows: W144 1.115, Q6_K 1.06, raw Q5_K 1.33 --
// its in-kernel unpack of the weight tile is shared by a quarter of the
// tokens).  Short calls take
// the 32-token tile (the 128-token tile costs the same at any row count up
// to 128); at a few hundred to a few thousand rows it depends on how evenly
// the tiles fill the workgroup slots.
TailSplit mmq_tail_split(int ntiles, int units, size_t ws_floats, int tm, float e, int cus);
constexpr float kTailMinSaving = 192.f;  // see mmq_tail_split
// the fixed cost of a split launch (its summing launch and partial-tile
// traffic, about 8 us) in the tile-height estimate's units
constexpr float kSplitCost = 384.f;

// tail: the kernel takes the leftover-tile split (both Q5_K tiers), so the
// busiest CU's count is the split one
int mmq_tile_rows(int rows, int K, int ntot, bool stage_units, size_t ws_floats, float e32, bool tail, int cus) {
    float best = 0.f;
    int pick = 128;
    for (const int tm : {128, 32}) {
        const int ks = mmq_ksplit(rows, K, ntot, stage_units, ws_floats, tm, cus);
        const long long ctas = (long long)((rows + tm - 1) / tm) * (ntot / kTN) * ks;
        const int units = stage_units ? K >> 7 : K >> 8;
        const int per = (units + ks - 1) / ks;
        float load = (float)((ctas + cus - 1) / cus);
        bool split = ks > 1;
        if (tail && ks == 1) {
            const TailSplit ts = mmq_tail_split((int)ctas, units, ws_floats, tm, tm == 32 ? e32 : 1.f, cus);
            if (ts.k > 1) {
                load = (float)(ctas / cus) + (float)((ts.nleft * ts.k + cus - 1) / cus) / (float)ts.k;
                split = true;
            }
        }
        // a split launch also pays its summing launch and partial-tile traffic
        const float est = load * tm * per * (tm == 32 ? e32 : 1.f) + (split ? kSplitCost : 0.f);
        if (tm == 128 || est < best) {
            best = est;
            pick = tm;
        }
    }
    return pick;
}

// y_p = sum over the K slices of the workspace (fixed order), 4 floats per
// thread over all parts of one launch: element i (in float4 units) of the
// slice belongs to part p when off4[p] <= i < off4[p + 1]
struct SumParts {
    float* Y[kMaxParts];
    size_t off4[kMaxParts + 1];
};
__global__ void __launch_bounds__(256) k_sum_splits(const float* __restrict__ ws, int ks, SumParts sp) {
    const size_t n4 = sp.off4[kMaxParts];
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    f32x4 v = ((const f32x4*)ws)[i];
    for (int k = 1; k < ks; ++k) v = v + ((const f32x4*)ws)[(size_t)k * n4 + i];
    int p = 0;
#pragma unroll
    for (int q = 1; q < kMaxParts; ++q)
        if (i >= sp.off4[q]) p = q;
    ((f32x4*)sp.Y[p])[i - sp.off4[p]] = v;
}

static hipError_t sum_splits(const PartTable& pt, int ks, int rows, const float* ws, hipStream_t st) {
    SumParts sp;
    size_t off = 0;
    for (int p = 0; p < kMaxParts; ++p) {
        sp.off4[p] = off;
        sp.Y[p] = p < pt.nparts ? pt.Y[p] : nullptr;
        if (p < pt.nparts) off += (size_t)rows * pt.N[p] / 4;
    }
    sp.off4[kMaxParts] = off;
    launch_kernel(k_sum_splits, dim3((unsigned)((off + 255) / 256)), dim3(256), 0, st, ws, ks, sp);
    return hipGetLastError();
}

// The leftover-tile split for `ntiles` tiles of `tm` tokens whose K has
// `units` slice units: the k (2..4) that minimises the busiest CU's work,
// floor(ntiles / CUs) + ceil(nleft * k / CUs) / k tiles, if that beats the
// unsplit ceil(ntiles / CUs) by at least half a tile and the slices fit the
// workspace; else k = 1.  Measured (9216 x 3072 W144, eager launches, µs,
// unsplit -> split): 2048 rows (k = 2, 0.5 tile) 181.5 -> 168.5; smaller
// gains did not pay for the shorter slices and the summing launch (2560 rows,
// k = 3 for 0.33 tile: 216 -> 218), nor did more than 4 slices (2304 rows,
// k = 8: 220 -> 227).
// It must also save at least kTailMinSaving tile-token-units (tm x K units x
// e, e = the tile height's relative cost per output) on the busiest CU, about
// half of what the summing launch and the partial tiles cost.
constexpr int kMaxTailSplit = 4;
TailSplit mmq_tail_split(int ntiles, int units, size_t ws_floats, int tm, float e, int cus) {
    TailSplit ts;
    const int q = ntiles / cus, nleft = ntiles % cus;
    // with one whole tile per CU each runs alone on its CU and the leftover
    // slices lose (512 x 9216 W144, 128-token tiles: 62 -> 67 us)
    if (q < 2 || nleft == 0) return ts;
    float best = (float)(q + 1);
    int bk = 1;
    for (int k = 2; k <= std::min(kMaxTailSplit, units); ++k) {
        if ((size_t)nleft * k * kTN * tm > ws_floats) break;
        const float load = (float)q + (float)((nleft * k + cus - 1) / cus) / (float)k;
        if (load < best - 1e-6f) {
            best = load;
            bk = k;
        }
    }
    if (bk == 1 || best > (float)(q + 1) - 0.5f) return ts;
    if (((float)(q + 1) - best) * (float)tm * (float)units * e < kTailMinSaving) return ts;
    ts.k = bk;
    ts.nleft = nleft;
    ts.nfull = ntiles - nleft;
    ts.gridfull = (ts.nfull + kXcds - 1) / kXcds * kXcds;
    return ts;
}

// Workspace floats the leftover-tile split of either Q5_K tier can use for
// this shape (the larger of the two tile heights), at most kTailMaxFloats (32 MiB).
constexpr size_t kTailMaxFloats = (size_t)8 << 20;
size_t mmq_tail_ws_floats(int rows, int K, int ntot, int cus) {
    size_t need = 0;
    for (const int tm : {128, 32}) {
        const int ntiles = ((rows + tm - 1) / tm) * (ntot / kTN);
        if (mmq_ksplit(rows, K, ntot, false, (size_t)-1, tm, cus) > 1) continue;
        for (const int units : {K >> 8, K >> 7}) {  // W144 (stage pairs), raw tier (stages)
            const TailSplit ts = mmq_tail_split(ntiles, units, kTailMaxFloats, tm, tm == 32 ? 1.33f : 1.f, cus);
            if (ts.k > 1) need = std::max(need, (size_t)ts.nleft * ts.k * kTN * tm);
        }
    }
    return need;
}

// Up to this many rows the 32-token W144 tile forms the min term's xdh
// operand itself instead of a k_fill_xdh launch filling it first (9216 x
// 3072: 16 / 32 rows 0.7-1.4 / 0.6-0.8 us faster per call, 48-95 rows
// level; at 512 rows, with 16x the tiles each re-forming the operand, 9 us
// slower).
constexpr int kXdhInlineRows = 64;

template <int TM, bool XI>
static hipError_t launch_w144_tm(const PartTable& pt, int ntm, int ntn, int ks, const TailSplit& ts, int rows,
                                 int K, const int8_t* xq, const float* xd, const int32_t* xsum,
                                 uint16_t* xdh, hipStream_t st, float* ws) {
    if (!XI) {
        const hipError_t e = launch_fill_xdh(xd, xsum, rows * (K / 32), xdh, st);
        if (e != hipSuccess) return e;
    }
    if (ts.k > 1) {
        launch_kernel(k_mmq_w144<TM, XI>, dim3(ts.gridfull + ts.nleft * ts.k), dim3(256), 0, st, pt, ntm, ntn, rows, K,
                      xq, xd, xsum, xdh, 1, ws, ts);
        const size_t n4 = (size_t)ts.nleft * TM * (kTN / 4);
        launch_kernel(k_sum_tail<TM>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, (const float*)ws, pt,
                      ntm, rows, ts);
        return hipGetLastError();
    }
    const dim3 grid(mmq_grid(ntm, ntn).x, ks);
    launch_kernel(k_mmq_w144<TM, XI>, grid, dim3(256), 0, st, pt, ntm, ntn, rows, K, xq, xd, xsum, xdh, ks, ws, ts);
    if (ks > 1) return sum_splits(pt, ks, rows, ws, st);
    return hipGetLastError();
}

hipError_t launch_mmq_q5k_144(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                              const int32_t* xsum, uint16_t* xdh, hipStream_t st, int cus, float* ws,
                              size_t ws_floats) {
    const int tm = mmq_tile_rows(rows, K, ntotal(pt), false, ws ? ws_floats : 0, 1.115f, true, cus);
    const int ntm = (rows + tm - 1) / tm;
    const int ntn = ntile_count(pt);
    if (ntm == 0 || ntn == 0) return hipSuccess;
    const int ks = mmq_ksplit(rows, K, ntotal(pt), false, ws ? ws_floats : 0, tm, cus);
    const TailSplit ts = ks > 1 ? TailSplit{}
                                : mmq_tail_split(ntm * ntn, K >> 8, ws ? ws_floats : 0, tm, tm == 32 ? 1.115f : 1.f, cus);
    if (tm == 32 && rows <= kXdhInlineRows)
        return launch_w144_tm<32, true>(pt, ntm, ntn, ks, ts, rows, K, xq, xd, xsum, xdh, st, ws);
    if (tm == 32) return launch_w144_tm<32, false>(pt, ntm, ntn, ks, ts, rows, K, xq, xd, xsum, xdh, st, ws);
    return launch_w144_tm<128, false>(pt, ntm, ntn, ks, ts, rows, K, xq, xd, xsum, xdh, st, ws);
}

template <int TM>
static hipError_t launch_raw_tm(const PartTable& pt, int ntm, int ntn, int ks, const TailSplit& ts, int rows, int K,
                                const int8_t* xq, const float* xd, const int32_t* xsum, hipStream_t st, float* ws) {
    if (ts.k > 1) {
        launch_kernel(k_mmq_q5k_raw<TM>, dim3(ts.gridfull + ts.nleft * ts.k), dim3(256), 0, st, pt, ntm, ntn, rows,
                      K, xq, xd, xsum, 1, ws, ts);
        const size_t n4 = (size_t)ts.nleft * TM * (kTN / 4);
        launch_kernel(k_sum_tail<TM>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, (const float*)ws, pt,
                      ntm, rows, ts);
        return hipGetLastError();
    }
    const dim3 grid(mmq_grid(ntm, ntn).x, ks);
    launch_kernel(k_mmq_q5k_raw<TM>, grid, dim3(256), 0, st, pt, ntm, ntn, rows, K, xq, xd, xsum, ks, ws, ts);
    if (ks > 1) return sum_splits(pt, ks, rows, ws, st);
    return hipGetLastError();
}

hipError_t launch_mmq_q5k_raw(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                              const int32_t* xsum, hipStream_t st, int cus, float* ws, size_t ws_floats) {
    const int tm = mmq_tile_rows(rows, K, ntotal(pt), true, ws ? ws_floats : 0, 1.33f, true, cus);
    const int ntm = (rows + tm - 1) / tm, ntn = ntile_count(pt);
    if (ntm == 0 || ntn == 0) return hipSuccess;
    const int ks = mmq_ksplit(rows, K, ntotal(pt), true, ws ? ws_floats : 0, tm, cus);
    const TailSplit ts = ks > 1 ? TailSplit{}
                                : mmq_tail_split(ntm * ntn, K >> 7, ws ? ws_floats : 0, tm, tm == 32 ? 1.33f : 1.f, cus);
    if (tm == 32) return launch_raw_tm<32>(pt, ntm, ntn, ks, ts, rows, K, xq, xd, xsum, st, ws);
    return launch_raw_tm<128>(pt, ntm, ntn, ks, ts, rows, K, xq, xd, xsum, st, ws);
}

hipError_t launch_mmq_q6k(PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
                          hipStream_t st, int cus, float* ws, size_t ws_floats) {
    const int tm = mmq_tile_rows(rows, K, ntotal(pt), false, ws ? ws_floats : 0, 1.06f, false, cus);
    const int ntm = (rows + tm - 1) / tm, ntn = ntile_count(pt);
    if (ntm == 0 || ntn == 0) return hipSuccess;
    const int ks = mmq_ksplit(rows, K, ntotal(pt), false, ws ? ws_floats : 0, tm, cus);
    const dim3 grid(mmq_grid(ntm, ntn).x, ks);
    if (tm == 32)
        launch_kernel(k_mmq_q6k_dma<32>, grid, dim3(256), 0, st, pt, ntm, ntn, rows, K, xq, xd, ks, ws);
    else
        launch_kernel(k_mmq_q6k_dma<128>, grid, dim3(256), 0, st, pt, ntm, ntn, rows, K, xq, xd, ks, ws);
    if (ks > 1) return sum_splits(pt, ks, rows, ws, st);
    return hipGetLastError();
}

}  // namespace bq
