// bq_gemv.hip -- k-quant x q8 decode GEMV / multi-row (1..8 rows) kernels for gfx950.
//
// Reference semantics (engine/src/bruce.cu):
//   Q5_K  y[n] = sum_g xd[g] * (ds[n,g]*dot[n,g] - dm[n,g]*xsum[g])
//         k_gemv_q5k :384-440, k_gemv_q5k_fused :5815-5887, k_gemm_tc_verify_q5k :5889-6076
//   Q6_K  y[n] = sum_{16-groups} xd[g32] * (d*sc16) * sum (q-32)*xq
//         k_gemm_q6k :4282-4362 (raw 210 B), k_gemv_q6k_dp :4452-4513 (160 B repack)
//
// MI355X design (not the reference's warp mapping):
//   * The weight matrix is a flat stream of 16-byte chunks.  A wave owns a tile
//     of T consecutive weight rows of one part and walks its "lane tasks"
//     (row, block, chunk) in address order, 64 per step, so every load
//     instruction of a wave covers a dense ~1.4 KiB span of HBM.
//   * Q5_K lane task = one 16-byte chunk of qs (two 16-value halves of a
//     sub-block pair) + the matching 16 bytes of qh + the 16-byte block header
//     (d, dmin, scales).  Three 128-bit loads, 32 values, 8 v_dot4_i32_i8.
//   * A row has K/32 lane tasks; T rows per tile with T*K/32 % 64 == 0 keep
//     every lane busy (K = 3072 -> T = 2, three full steps).
//   * Activations (int8 codes, fp32 scales, sums) of all MR rows are staged in
//     LDS once per workgroup; every weight byte is read once for all MR rows.
//   * Per-row partial sums are reduced across the wave with xor shuffles.
#include "bq_device.hpp"
#include "bq_internal.hpp"

#include <type_traits>

namespace bq {

// rows per wave tile: every row has K/32 lane tasks, so T*K/32 % 64 == 0 keeps
// all 64 lanes busy on every step (K % 2048 -> 1, K % 1024 -> 2, else 4)
static int tile_rows(int K) {
    if (K % 2048 == 0) return 1;
    if (K % 1024 == 0) return 2;
    return 4;
}

BQ_DEV int find_part(const PartTable& pt, int tile) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxParts; ++i)
        if (i < pt.nparts && tile >= pt.tile0[i]) p = i;
    return p;
}

// ---------------------------------------------------------------------------
// Weight-format policies.  A lane task covers 32 values of one weight row:
//   Task  -- the raw bytes a lane loads for it (registers)
//   load  -- issue the task's global loads
//   dot   -- its contribution to activation row m (LDS-staged activations)
// ---------------------------------------------------------------------------
struct ActLds {            // activations of MR rows staged in LDS
    const int8_t* x;       // [MR][K] int8 codes
    const float* xd;       // [MR][K/32]
    const float* aux;      // Q5_K: float(xsum) [MR][K/32]; Q6_K raw: 32*sum16 as int [MR][K/16]
};

struct FmtQ5K {
    static constexpr int kAuxPerRow32 = 1;   // float(xsum) per 32-group
    struct Task { u32x4 hdr, qh, qs; };
    // r = index of the task inside its row: super-block r >> 3, qs chunk r & 7
    static BQ_DEV void load(Task& t, const uint8_t* W, int row, int r, int K) {
        const uint8_t* blk = W + ((size_t)row * (K >> 8) + (r >> 3)) * kQ5Bytes;
        const int c = r & 7;
        t.hdr = ld16(blk);
        t.qh = ld16(blk + 16 + 16 * (c & 1));
        t.qs = ld16(blk + 48 + 16 * c);
    }
    // Precomputed per-task operands, shared by all activation rows.
    struct Prep { uint32_t u0[4], u1[4]; float ds0, ds1, dm0, dm1; int xo, g0; };
    static BQ_DEV void prep(Prep& q, const Task& t, int r) {
        const int sb = r >> 3, c = r & 7;
        const int j0 = (c >> 1) * 2, j1 = j0 + 1, half = c & 1;
        uint32_t sc0, m0, sc1, m1;
        q5k_scale_min(t.hdr.y, t.hdr.z, t.hdr.w, j0, sc0, m0);
        q5k_scale_min(t.hdr.y, t.hdr.z, t.hdr.w, j1, sc1, m1);
        const float d = h2f(t.hdr.x & 0xFFFF), dmin = h2f(t.hdr.x >> 16);
        q.ds0 = d * (float)sc0;
        q.ds1 = d * (float)sc1;
        // the min term of a sub-block is added once, by the lane holding its first half
        q.dm0 = half ? 0.f : dmin * (float)m0;
        q.dm1 = half ? 0.f : dmin * (float)m1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q.u0[i] = (t.qs[i] & 0x0F0F0F0Fu) | (((t.qh[i] >> j0) & 0x01010101u) << 4);
            q.u1[i] = ((t.qs[i] >> 4) & 0x0F0F0F0Fu) | (((t.qh[i] >> j1) & 0x01010101u) << 4);
        }
        q.g0 = sb * 8 + j0;
        q.xo = sb * 256 + 32 * j0 + 16 * half;
    }
    static BQ_DEV float dot(const Prep& q, const ActLds& a, int m, int K) {
        const int nb = K >> 5;
        const u32x4 x0 = *(const u32x4*)(a.x + m * K + q.xo);
        const u32x4 x1 = *(const u32x4*)(a.x + m * K + q.xo + 32);
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = dot4((int)q.u0[i], (int)x0[i], s0);
            s1 = dot4((int)q.u1[i], (int)x1[i], s1);
        }
        const float* xd = a.xd + m * nb + q.g0;
        const float* xs = a.aux + m * nb + q.g0;
        return xd[0] * (q.ds0 * (float)s0 - q.dm0 * xs[0]) + xd[1] * (q.ds1 * (float)s1 - q.dm1 * xs[1]);
    }
};

struct FmtQ6KRaw {
    // task r: super-block r >> 3, ql chunk c = r & 7 holding values
    // 128h + 32*ulo + l0 .. +15 (low nibbles) and quarter ulo + 2 (high nibbles)
    struct Task { u32x4 ql, qh, sc; uint32_t d; };
    static BQ_DEV void load(Task& t, const uint8_t* W, int row, int r, int K) {
        const uint8_t* blk = W + ((size_t)row * (K >> 8) + (r >> 3)) * kQ6Bytes;
        const int c = r & 7, h = c >> 2, l0 = 16 * (c & 1);
        t.ql = ld16_a2(blk + 16 * c);
        t.qh = ld16_a2(blk + 128 + 32 * h + l0);
        t.sc = ld16_a2(blk + 192);
        t.d = *(const uint16_t*)(blk + 208);
    }
    struct Prep { uint32_t qa[4], qb[4]; float sA, sB; int kA; };
    static BQ_DEV void prep(Prep& q, const Task& t, int r) {
        const int sb = r >> 3, c = r & 7, h = c >> 2, ulo = (c >> 1) & 1, l0 = 16 * (c & 1);
        const int gA = 8 * h + 2 * ulo + (c & 1);  // 16-value group in the block; B = gA + 4
        const float d = h2f(t.d);
        const int bA = (int)(int8_t)(t.sc[gA >> 2] >> (8 * (gA & 3)));
        const int bB = (int)(int8_t)(t.sc[(gA + 4) >> 2] >> (8 * (gA & 3)));
        q.sA = d * (float)bA;
        q.sB = d * (float)bB;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q.qa[i] = (t.ql[i] & 0x0F0F0F0Fu) | (((t.qh[i] >> (2 * ulo)) & 0x03030303u) << 4);
            q.qb[i] = ((t.ql[i] >> 4) & 0x0F0F0F0Fu) | (((t.qh[i] >> (2 * ulo + 4)) & 0x03030303u) << 4);
        }
        q.kA = sb * 256 + 128 * h + 32 * ulo + l0;
    }
    // codes are q in 0..63: dot(q - 32, x) = dot(q, x) - 32 * sum16(x)
    static BQ_DEV float dot(const Prep& q, const ActLds& a, int m, int K) {
        const int nb = K >> 5, n16 = K >> 4;
        const u32x4 x0 = *(const u32x4*)(a.x + m * K + q.kA);
        const u32x4 x1 = *(const u32x4*)(a.x + m * K + q.kA + 64);
        const int* s16 = (const int*)a.aux + m * n16 + (q.kA >> 4);
        int s0 = -s16[0], s1 = -s16[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = dot4((int)q.qa[i], (int)x0[i], s0);
            s1 = dot4((int)q.qb[i], (int)x1[i], s1);
        }
        const float* xd = a.xd + m * nb + (q.kA >> 5);
        return xd[0] * q.sA * (float)s0 + xd[2] * q.sB * (float)s1;
    }
};

struct FmtQ6KRep {
    // task r: stage r >> 2, 32 values at 32*(r & 3) (two 16-value scale groups)
    struct Task { u32x4 wa, wb; float2 sc; };
    static BQ_DEV void load(Task& t, const uint8_t* W, int row, int r, int K) {
        const uint8_t* st = W + ((size_t)row * (K >> 7) + (r >> 2)) * kW160;
        const int c4 = r & 3;
        t.wa = ld16(st + 32 * c4);
        t.wb = ld16(st + 32 * c4 + 16);
        t.sc = *(const float2*)(st + 128 + 8 * c4);
    }
    struct Prep { u32x4 wa, wb; float2 sc; int k; };
    static BQ_DEV void prep(Prep& q, const Task& t, int r) {
        q.wa = t.wa;
        q.wb = t.wb;
        q.sc = t.sc;
        q.k = (r >> 2) * 128 + 32 * (r & 3);
    }
    static BQ_DEV float dot(const Prep& q, const ActLds& a, int m, int K) {
        const u32x4 x0 = *(const u32x4*)(a.x + m * K + q.k);
        const u32x4 x1 = *(const u32x4*)(a.x + m * K + q.k + 16);
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = dot4((int)q.wa[i], (int)x0[i], s0);
            s1 = dot4((int)q.wb[i], (int)x1[i], s1);
        }
        return a.xd[m * (K >> 5) + (q.k >> 5)] * (q.sc.x * (float)s0 + q.sc.y * (float)s1);
    }
};

// LDS bytes for MR staged activation rows
template <class F>
constexpr size_t act_lds_bytes(int rows, int K);

template <> constexpr size_t act_lds_bytes<FmtQ5K>(int rows, int K) {
    return (size_t)rows * K + (size_t)rows * (K / 32) * 8;
}
template <> constexpr size_t act_lds_bytes<FmtQ6KRaw>(int rows, int K) {
    return (size_t)rows * K + (size_t)rows * (K / 32) * 4 + (size_t)rows * (K / 16) * 4;
}
template <> constexpr size_t act_lds_bytes<FmtQ6KRep>(int rows, int K) {
    return (size_t)rows * K + (size_t)rows * (K / 32) * 4;
}

// ---------------------------------------------------------------------------
// The GEMV kernel: WAVES waves per workgroup, one tile of T weight rows per
// wave, MR activation rows, S steps (64 tasks each) of loads kept in flight.
//   1. every wave issues the loads of its first S steps,
//   2. the workgroup stages the activations in LDS while those are in flight,
//   3. steps are computed S at a time, the next S steps' loads issued first.
// ---------------------------------------------------------------------------
template <class F, int T, int MR, int S, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
k_gemv(PartTable pt, int K, const int8_t* __restrict__ xq, const float* __restrict__ xd,
       const int32_t* __restrict__ xsum) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const bool valid = tile < pt.ntiles;
    const int p = valid ? find_part(pt, tile) : 0;
    const uint8_t* __restrict__ W = (const uint8_t*)pt.W[p];
    const int Nloc = pt.N[p];
    const int row0 = valid ? (tile - pt.tile0[p]) * T : 0;
    const int tpr = K >> 5;                 // tasks per weight row
    const int total = T * tpr;
    const int nchunks = (total + 64 * S - 1) / (64 * S);

    // task f -> (tile row t, task in row r); rows past N are skipped
    auto locate = [&](int f, int& t, int& r) -> bool {
        t = 0;
        r = f;
#pragma unroll
        for (int i = 1; i < T; ++i)
            if (r >= tpr) { r -= tpr; ++t; }
        return f < total && row0 + t < Nloc;
    };
    typename F::Task cur[S];
    auto load_chunk = [&](int ch, typename F::Task (&buf)[S]) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            int t, r;
            if (locate((ch * S + s) * 64 + lane, t, r)) F::load(buf[s], W, row0 + t, r, K);
        }
    };
    if (valid) load_chunk(0, cur);

    // ---- stage activations
    const int nb = K >> 5;
    ActLds a;
    a.x = (const int8_t*)smem;
    a.xd = (const float*)(smem + MR * K);
    a.aux = a.xd + MR * nb;
    for (int i = threadIdx.x; i < MR * K / 16; i += 64 * WAVES) {
        const u32x4 v = ((const u32x4*)xq)[i];
        ((u32x4*)smem)[i] = v;
        if constexpr (std::is_same<F, FmtQ6KRaw>::value) {
            int s = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) s = dot4((int)v[k], 0x01010101, s);
            ((int*)a.aux)[i] = 32 * s;
        }
    }
    for (int i = threadIdx.x; i < MR * nb; i += 64 * WAVES) {
        ((float*)a.xd)[i] = xd[i];
        if constexpr (std::is_same<F, FmtQ5K>::value) ((float*)a.aux)[i] = (float)xsum[i];
    }
    __syncthreads();
    if (!valid) return;

    float acc[T][MR];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[t][m] = 0.f;

    for (int ch = 0; ch < nchunks; ++ch) {
        typename F::Task nxt[S];
        if (ch + 1 < nchunks) load_chunk(ch + 1, nxt);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            int t, r;
            if (!locate((ch * S + s) * 64 + lane, t, r)) continue;
            typename F::Prep q;
            F::prep(q, cur[s], r);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float v = F::dot(q, a, m, K);
#pragma unroll
                for (int i = 0; i < T; ++i) acc[i][m] += (t == i) ? v : 0.f;
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) cur[s] = nxt[s];
    }

    float* __restrict__ Y = pt.Y[p];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float v = wave_sum(acc[t][m]);
            if (lane == 0 && row0 + t < Nloc) Y[(size_t)m * Nloc + row0 + t] = v;
        }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
static void build_tiles(PartTable& pt, int T) {
    int acc = 0;
    for (int p = 0; p < pt.nparts; ++p) {
        pt.tile0[p] = acc;
        acc += (pt.N[p] + T - 1) / T;
    }
    for (int p = pt.nparts; p < kMaxParts; ++p) pt.tile0[p] = acc;
    pt.ntiles = acc;
}

// steps in flight per wave: 3 for one or two rows (load-latency bound),
// 2 for more rows (VALU heavier, registers scarcer)
template <int MR> constexpr int steps_for() { return MR <= 2 ? 3 : 2; }

template <class F, int T, int MR, int WAVES>
static hipError_t launch_fmt(const PartTable& pt, int K, const int8_t* xq, const float* xd,
                             const int32_t* xsum, size_t lds, hipStream_t st) {
    const dim3 grid((pt.ntiles + WAVES - 1) / WAVES), block(64 * WAVES);
    hipLaunchKernelGGL((k_gemv<F, T, MR, steps_for<MR>(), WAVES>), grid, block, lds, st, pt, K, xq, xd, xsum);
    return hipGetLastError();
}

template <class F, int MR>
static hipError_t dispatch_t(int T, const PartTable& pt, int K, const int8_t* xq, const float* xd,
                             const int32_t* xsum, hipStream_t st) {
    const size_t lds = act_lds_bytes<F>(MR, K);
    const bool big = lds > 32 * 1024;  // one LDS copy shared by 16 waves
#define BQ_LT(TT) return big ? launch_fmt<F, TT, MR, 16>(pt, K, xq, xd, xsum, lds, st) \
                             : launch_fmt<F, TT, MR, 4>(pt, K, xq, xd, xsum, lds, st)
    switch (T) {
        case 1: BQ_LT(1);
        case 2: BQ_LT(2);
        default: BQ_LT(4);
    }
#undef BQ_LT
}

template <class F>
static hipError_t dispatch_rows(int rows, int T, const PartTable& pt, int K, const int8_t* xq,
                                const float* xd, const int32_t* xsum, hipStream_t st) {
    switch (rows) {
        case 1: return dispatch_t<F, 1>(T, pt, K, xq, xd, xsum, st);
        case 2: return dispatch_t<F, 2>(T, pt, K, xq, xd, xsum, st);
        case 3: return dispatch_t<F, 3>(T, pt, K, xq, xd, xsum, st);
        case 4: return dispatch_t<F, 4>(T, pt, K, xq, xd, xsum, st);
        case 5: return dispatch_t<F, 5>(T, pt, K, xq, xd, xsum, st);
        case 6: return dispatch_t<F, 6>(T, pt, K, xq, xd, xsum, st);
        case 7: return dispatch_t<F, 7>(T, pt, K, xq, xd, xsum, st);
        case 8: return dispatch_t<F, 8>(T, pt, K, xq, xd, xsum, st);
        default: return hipErrorInvalidValue;
    }
}

size_t gemv_lds_bytes(GemvKind kind, int rows, int K) {
    switch (kind) {
        case GemvKind::Q5K: return act_lds_bytes<FmtQ5K>(rows, K);
        case GemvKind::Q6KRaw: return act_lds_bytes<FmtQ6KRaw>(rows, K);
        default: return act_lds_bytes<FmtQ6KRep>(rows, K);
    }
}

// rows 1..8 activation rows starting at xq/xd/xsum (already offset)
hipError_t launch_gemv(GemvKind kind, PartTable pt, int rows, int K, const int8_t* xq,
                       const float* xd, const int32_t* xsum, hipStream_t st) {
    const int T = tile_rows(K);
    build_tiles(pt, T);
    if (pt.ntiles == 0) return hipSuccess;
    switch (kind) {
        case GemvKind::Q5K: return dispatch_rows<FmtQ5K>(rows, T, pt, K, xq, xd, xsum, st);
        case GemvKind::Q6KRaw: return dispatch_rows<FmtQ6KRaw>(rows, T, pt, K, xq, xd, xsum, st);
        default: return dispatch_rows<FmtQ6KRep>(rows, T, pt, K, xq, xd, xsum, st);
    }
}

}  // namespace bq
