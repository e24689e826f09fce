// bq_api.hip -- the C ABI of libbq (include/bq.h): argument checks, dispatch.
//
// Mirrors the reference's host launchers in engine/src/bruce.cu (launch_gemv
// :5624, launch_verify_fused :7141, launch_q6_verify_fused :7231,
// launch_gemm_q6k_dp :7285, try_launch_mmq :7366, launch_gemm_b_fused :7421,
// launch_gemm_b :7428, q5k_prepack_launch :4832, q6k_repack_host :4783) with
// three deliberate differences: buffers are passed explicitly instead of read
// from a global model, nothing calls exit() (errors are return codes), and
// unsupported shapes return BQ_UNSUPPORTED before anything is enqueued.
#include <string.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <mutex>

#include "../../include/bq.h"
#include "bq_internal.hpp"

using namespace bq;

namespace {

// Properties of each device the library runs on, read on the first call
// made with that device current: the per-block LDS limit (GEMV row chunks)
// and the CU count (the prefill GEMMs' split choices, the logits head's grid).
struct DevInfo {
    size_t lds_per_block = 65536;
    int cus = 256;
    int status = BQ_OK;
    std::atomic<bool> ready{false};
};

constexpr int kMaxDevices = 64;
std::mutex g_dev_mu;
DevInfo g_devs[kMaxDevices];
thread_local const DevInfo* t_dev = nullptr;  // the current device's entry (set by ensure_init)

int from_hip(hipError_t e) { return e == hipSuccess ? BQ_OK : -(int)e; }
int scratch_ptr(void** out);  // bq_gemm_b_fused_noalloc's scratch (below)

// Every entry point that touches a device calls this first: it looks up (on
// first use, queries) the current device's properties and points t_dev at them.
int ensure_init() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -(int)hipErrorNoDevice;
    if (dev < 0 || dev >= kMaxDevices) return BQ_UNSUPPORTED;
    DevInfo& d = g_devs[dev];
    if (!d.ready.load(std::memory_order_acquire)) {
        std::lock_guard<std::mutex> lk(g_dev_mu);
        if (!d.ready.load(std::memory_order_relaxed)) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
                d.status = -(int)hipErrorNoDevice;
            } else {
                d.lds_per_block = prop.sharedMemPerBlock;
                d.cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
            }
            d.ready.store(true, std::memory_order_release);
        }
    }
    t_dev = &d;
    return d.status;
}

// try_launch_mmq's row threshold (bruce.cu:7369: rows >= 96)
constexpr int kMmqMinRows = 96;

bool weight_ok(const bq_weight* w) { return w && w->K > 0 && w->N > 0 && (w->K % 256) == 0; }

// Every kernel reads weights, activations and fp32 rows with 16-byte loads
// (direct-to-LDS copies included), so each buffer must start 16-byte aligned;
// a misaligned pointer is rejected here instead of reaching the device.
bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
bool weight_al16(const bq_weight* w) { return al16(w->raw) && al16(w->rep) && al16(w->rep_min); }

// Run a multi-row GEMV in row chunks that fit the per-block LDS limit.
int gemv_rows(GemvKind kind, PartTable pt, int rows, int K, const int8_t* xq, const float* xd,
              const int32_t* xsum, hipStream_t st) {
    if (K > kGemvMaxK) return BQ_UNSUPPORTED;
    if (!al16(xq) || !al16(xd) || !al16(xsum)) return BQ_EINVAL;
    for (int p = 0; p < pt.nparts; ++p)
        if (!al16(pt.W[p])) return BQ_EINVAL;
    int r0 = 0;
    while (r0 < rows) {
        int c = std::min(rows - r0, (int)BQ_MAX_ROWS);
        while (c > 1 && gemv_lds_bytes(kind, c, K) > t_dev->lds_per_block) --c;
        if (gemv_lds_bytes(kind, c, K) > t_dev->lds_per_block) return BQ_UNSUPPORTED;
        PartTable q = pt;
        for (int p = 0; p < pt.nparts; ++p) q.Y[p] = pt.Y[p] + (size_t)r0 * pt.N[p];
        const int nb = K / 32;
        hipError_t e = launch_gemv(kind, q, c, K, xq + (size_t)r0 * K, xd + (size_t)r0 * nb,
                                   xsum ? xsum + (size_t)r0 * nb : nullptr, st);
        if (e != hipSuccess) return from_hip(e);
        r0 += c;
    }
    return BQ_OK;
}

PartTable one_part(float* y, const void* W, int N) {
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    pt.W[0] = W;
    pt.Y[0] = y;
    pt.N[0] = N;
    pt.nparts = 1;
    return pt;
}

}  // namespace

namespace bq {
LaunchTiming& next_launch_timing() {
    static thread_local LaunchTiming t;
    return t;
}

ScaledCopy& next_scaled_copy() {
    static thread_local ScaledCopy c;
    return c;
}

int device_cus() { return t_dev ? t_dev->cus : 256; }

int gemv_gate_den_fused(float* y, const void* w_raw, int K, int N, const float* a, const float* den, void* st) {
    if (int r = ensure_init()) return r;
    if (!y || !w_raw || !a || !den || K <= 0 || N <= 0 || K % 256 != 0) return BQ_EINVAL;
    if (!al16(w_raw) || !al16(a) || !al16(den)) return BQ_EINVAL;
    if (!gemv_producer_supported(K)) return BQ_UNSUPPORTED;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    pt.W[0] = w_raw;
    pt.Y[0] = y;
    pt.N[0] = N;
    pt.nparts = 1;
    return from_hip(launch_gemv_producer(GemvKind::Q5K, pt, K, kOpGateDen, nullptr, a, den, nullptr, nullptr, nullptr,
                                         nullptr, nullptr, (hipStream_t)st));
}
}  // namespace bq

extern "C" {

int bq_time_next_launch(void* start_event, void* stop_event) {
    if (!start_event || !stop_event) return BQ_EINVAL;
    next_launch_timing().start = (hipEvent_t)start_event;
    next_launch_timing().stop = (hipEvent_t)stop_event;
    return BQ_OK;
}

int bq_init(void) {
    if (int s = ensure_init()) return s;
    void* p = nullptr;
    return scratch_ptr(&p);  // the current device's allocation-free scratch
}

const char* bq_version(void) { return "bq 0.1 gfx950"; }

const char* bq_strerror(int code) {
    if (code == BQ_OK) return "ok";
    if (code == BQ_UNSUPPORTED) return "unsupported shape or type (nothing enqueued)";
    if (code == BQ_EINVAL) return "invalid argument";
    if (code == BQ_ETOOBIG) return "input larger than the allocation-free entry point's static scratch";
    if (code < 0) return hipGetErrorString((hipError_t)(-code));
    return "unknown bq error";
}

int bq_quantize_q8(const float* x, int rows, int K, int8_t* xq, float* xd, int32_t* xsum,
                   uint16_t* xdh, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (rows < 0 || K <= 0 || (K % 32) != 0) return BQ_EINVAL;
    if (rows == 0) return BQ_OK;
    if (!x || !xq || !xd || !xsum) return BQ_EINVAL;
    if (!al16(x) || !al16(xq)) return BQ_EINVAL;
    return from_hip(launch_quant_q8(x, rows, K, xq, xd, xsum, xdh, (hipStream_t)st));
}

int bq_fill_xdh(const float* xd, const int32_t* xsum, int n, uint16_t* xdh, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (n < 0) return BQ_EINVAL;
    if (n == 0) return BQ_OK;
    if (!xd || !xsum || !xdh) return BQ_EINVAL;
    return from_hip(launch_fill_xdh(xd, xsum, n, xdh, (hipStream_t)st));
}

int bq_gemm_q6k_dp(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                   int xoff, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!weight_ok(w) || !y || !xq || !xd || xoff < 0) return BQ_EINVAL;
    if (w->ggml_type != BQ_TYPE_Q6_K || !w->rep) return BQ_UNSUPPORTED;
    if (rows < 1 || rows > BQ_MAX_ROWS) return BQ_UNSUPPORTED;
    const int K = w->K;
    return gemv_rows(GemvKind::Q6KRep, one_part(y, w->rep, w->N), rows, K, xq + (size_t)xoff * K,
                     xd + (size_t)xoff * (K / 32), nullptr, (hipStream_t)st);
}

int bq_gemm_q6k_raw(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                    int xoff, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!weight_ok(w) || !y || !xq || !xd || xoff < 0) return BQ_EINVAL;
    if (w->ggml_type != BQ_TYPE_Q6_K || !w->raw) return BQ_UNSUPPORTED;
    if (rows < 1 || rows > BQ_MAX_ROWS) return BQ_UNSUPPORTED;
    const int K = w->K;
    return gemv_rows(GemvKind::Q6KRaw, one_part(y, w->raw, w->N), rows, K, xq + (size_t)xoff * K,
                     xd + (size_t)xoff * (K / 32), nullptr, (hipStream_t)st);
}

int bq_gemv(float* y, const bq_weight* w, const int8_t* xq, const float* xd, const int32_t* xsum,
            bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!weight_ok(w) || !y || !xq || !xd) return BQ_EINVAL;
    if (w->ggml_type == BQ_TYPE_Q6_K) {
        if (w->rep) return bq_gemm_q6k_dp(y, w, 1, xq, xd, 0, st);
        return bq_gemm_q6k_raw(y, w, 1, xq, xd, 0, st);
    }
    if (w->ggml_type != BQ_TYPE_Q5_K || !w->raw) return BQ_UNSUPPORTED;
    if (!xsum) return BQ_EINVAL;
    return gemv_rows(GemvKind::Q5K, one_part(y, w->raw, w->N), 1, w->K, xq, xd, xsum, (hipStream_t)st);
}

int bq_verify_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                    const int8_t* xq, const float* xd, const int32_t* xsum, int xoff,
                    bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (rows < 1 || rows > BQ_MAX_ROWS || nparts < 1 || nparts > BQ_MAX_PARTS) return BQ_UNSUPPORTED;
    if (!ys || !ws || !xq || !xd || !xsum || xoff < 0 || !ws[0]) return BQ_EINVAL;
    const int K = ws[0]->K;
    if (K <= 0 || (K % 256) != 0) return BQ_UNSUPPORTED;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    for (int p = 0; p < nparts; ++p) {
        const bq_weight* w = ws[p];
        if (!w || !w->raw || !ys[p] || w->ggml_type != BQ_TYPE_Q5_K) return BQ_UNSUPPORTED;
        if (w->K != K || w->N <= 0 || (w->N % 16) != 0) return BQ_UNSUPPORTED;
        pt.W[p] = w->raw;
        pt.Y[p] = ys[p];
        pt.N[p] = w->N;
    }
    pt.nparts = nparts;
    return gemv_rows(GemvKind::Q5K, pt, rows, K, xq + (size_t)xoff * K, xd + (size_t)xoff * (K / 32),
                     xsum + (size_t)xoff * (K / 32), (hipStream_t)st);
}

int bq_q6_verify_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                       const int8_t* xq, const float* xd, int xoff, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (rows < 2 || rows > BQ_MAX_ROWS || nparts < 1 || nparts > BQ_MAX_PARTS) return BQ_UNSUPPORTED;
    if (!ys || !ws || !xq || !xd || xoff < 0 || !ws[0]) return BQ_EINVAL;
    const int K = ws[0]->K;
    if (K <= 0 || (K % 256) != 0) return BQ_UNSUPPORTED;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    for (int p = 0; p < nparts; ++p) {
        const bq_weight* w = ws[p];
        if (!w || !w->rep || !ys[p] || w->ggml_type != BQ_TYPE_Q6_K) return BQ_UNSUPPORTED;
        if (w->K != K || w->N <= 0 || (w->N % 16) != 0) return BQ_UNSUPPORTED;
        pt.W[p] = w->rep;
        pt.Y[p] = ys[p];
        pt.N[p] = w->N;
    }
    pt.nparts = nparts;
    return gemv_rows(GemvKind::Q6KRep, pt, rows, K, xq + (size_t)xoff * K, xd + (size_t)xoff * (K / 32),
                     nullptr, (hipStream_t)st);
}

int bq_gemv_q8_fused(float* const* ys, const bq_weight* const* ws, int nparts, const float* x,
                     int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (nparts < 1 || nparts > BQ_MAX_PARTS) return BQ_UNSUPPORTED;
    if (!ys || !ws || !ws[0] || !x) return BQ_EINVAL;
    if ((xq != nullptr) != (xd != nullptr) || (xq != nullptr) != (xsum != nullptr)) return BQ_EINVAL;
    const int K = ws[0]->K;
    const uint32_t type = ws[0]->ggml_type;
    const bool q6rep = type == BQ_TYPE_Q6_K && ws[0]->rep;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    for (int p = 0; p < nparts; ++p) {
        const bq_weight* w = ws[p];
        if (!weight_ok(w) || !ys[p]) return BQ_EINVAL;
        if (w->K != K || w->ggml_type != type) return BQ_UNSUPPORTED;
        if (type == BQ_TYPE_Q5_K) {
            if (!w->raw) return BQ_UNSUPPORTED;
            pt.W[p] = w->raw;
        } else if (type == BQ_TYPE_Q6_K) {
            if ((w->rep != nullptr) != q6rep || (!q6rep && !w->raw)) return BQ_UNSUPPORTED;
            pt.W[p] = q6rep ? w->rep : w->raw;
        } else {
            return BQ_UNSUPPORTED;
        }
        pt.Y[p] = ys[p];
        pt.N[p] = w->N;
    }
    pt.nparts = nparts;
    for (int p = 0; p < nparts; ++p)
        if (!al16(pt.W[p])) return BQ_EINVAL;
    if (!al16(x) || !al16(xq) || !al16(xd) || !al16(xsum)) return BQ_EINVAL;
    const GemvKind kind = type == BQ_TYPE_Q5_K ? GemvKind::Q5K : (q6rep ? GemvKind::Q6KRep : GemvKind::Q6KRaw);
    hipStream_t s = (hipStream_t)st;
    if (!gemv_fused_supported(K)) return BQ_UNSUPPORTED;
    return from_hip(launch_gemv_fused_q8(kind, pt, K, x, xq, xd, xsum, s));
}

int bq_gemv_norm_fused(float* const* ys, const bq_weight* const* ws, int nparts, int op, float* out,
                       const float* a, const float* b, const float* c, const float* d, int8_t* xq,
                       float* xd, int32_t* xsum, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (nparts < 1 || nparts > BQ_MAX_PARTS) return BQ_UNSUPPORTED;
    if (!ys || !ws || !ws[0] || !a || op < BQ_OP_NORM || op > BQ_OP_SILU) return BQ_EINVAL;
    if ((xq != nullptr) != (xd != nullptr) || (xq != nullptr) != (xsum != nullptr)) return BQ_EINVAL;
    // inputs of the op
    if (op != BQ_OP_NORM && !b) return BQ_EINVAL;
    if (op >= BQ_OP_RESID && op != BQ_OP_GATE && !c) return BQ_EINVAL;  // gate: c NULL = b already scaled
    if (op == BQ_OP_SILU && !d) return BQ_EINVAL;
    if (out && (out == a || out == b)) return BQ_EINVAL;  // read by every workgroup
    const int K = ws[0]->K;
    const uint32_t type = ws[0]->ggml_type;
    const bool q6rep = type == BQ_TYPE_Q6_K && ws[0]->rep;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    for (int p = 0; p < nparts; ++p) {
        const bq_weight* w = ws[p];
        if (!weight_ok(w) || !ys[p]) return BQ_EINVAL;
        if (w->K != K || w->ggml_type != type) return BQ_UNSUPPORTED;
        if (type == BQ_TYPE_Q5_K) {
            if (!w->raw) return BQ_UNSUPPORTED;
            pt.W[p] = w->raw;
        } else if (type == BQ_TYPE_Q6_K) {
            if ((w->rep != nullptr) != q6rep || (!q6rep && !w->raw)) return BQ_UNSUPPORTED;
            pt.W[p] = q6rep ? w->rep : w->raw;
        } else {
            return BQ_UNSUPPORTED;
        }
        pt.Y[p] = ys[p];
        pt.N[p] = w->N;
    }
    pt.nparts = nparts;
    if (!gemv_producer_supported(K)) return BQ_UNSUPPORTED;
    const float* in[4] = {a, b, c, d};
    for (const float* q : in)
        if ((uintptr_t)q % 16) return BQ_EINVAL;
    if ((uintptr_t)out % 16 || (uintptr_t)xq % 16 || !al16(xd) || !al16(xsum)) return BQ_EINVAL;
    for (int p = 0; p < nparts; ++p)
        if (!al16(pt.W[p])) return BQ_EINVAL;
    const GemvKind kind = type == BQ_TYPE_Q5_K ? GemvKind::Q5K : (q6rep ? GemvKind::Q6KRep : GemvKind::Q6KRaw);
    return from_hip(launch_gemv_producer(kind, pt, K, op, out, a, op != BQ_OP_NORM ? b : nullptr,
                                         op >= BQ_OP_RESID ? c : nullptr, op == BQ_OP_SILU ? d : nullptr, xq, xd,
                                         xsum, (hipStream_t)st));
}

int bq_gate_up_silu(float* h, const bq_weight* wg, const bq_weight* wu, const float* sg, const float* su,
                    const int8_t* xq, const float* xd, const int32_t* xsum, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!h || !sg || !su || !xq || !xd || !weight_ok(wg) || !weight_ok(wu)) return BQ_EINVAL;
    const int K = wg->K, N = wg->N;
    const uint32_t type = wg->ggml_type;
    if (wu->K != K || wu->N != N || wu->ggml_type != type) return BQ_UNSUPPORTED;
    if (K % 256 != 0 || N % 16 != 0) return BQ_UNSUPPORTED;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    GemvKind kind;
    if (type == BQ_TYPE_Q5_K) {
        if (!wg->raw || !wu->raw) return BQ_UNSUPPORTED;
        if (!xsum) return BQ_EINVAL;
        kind = GemvKind::Q5K;
        pt.W[0] = wg->raw;
        pt.W[1] = wu->raw;
    } else if (type == BQ_TYPE_Q6_K) {
        const bool rep = wg->rep != nullptr;
        if ((wu->rep != nullptr) != rep || (!rep && (!wg->raw || !wu->raw))) return BQ_UNSUPPORTED;
        kind = rep ? GemvKind::Q6KRep : GemvKind::Q6KRaw;
        pt.W[0] = rep ? wg->rep : wg->raw;
        pt.W[1] = rep ? wu->rep : wu->raw;
    } else {
        return BQ_UNSUPPORTED;
    }
    if (!al16(pt.W[0]) || !al16(pt.W[1]) || !al16(xq) || !al16(xd) || !al16(xsum)) return BQ_EINVAL;
    pt.N[0] = pt.N[1] = N;
    pt.Y[0] = pt.Y[1] = h;  // not written: the epilogue writes h
    pt.nparts = 2;
    return from_hip(launch_gemv_silu_pair(kind, pt, K, xq, xd, xsum, sg, su, h, (hipStream_t)st));
}

namespace {

// The MMQ launch behind bq_try_mmq and the bq_gemm_b dispatchers.  min_w144 /
// min_raw: the smallest row count taken by the prepacked / raw tier (below
// it BQ_UNSUPPORTED, nothing enqueued).  work / work_bytes: the caller's K-split
// workspace (NULL / 0: no split).
int try_mmq_impl(float* const* ys, const bq_weight* const* ws, int nparts, int rows, const int8_t* xq,
                 const float* xd, const int32_t* xsum, uint16_t* xdh, void* work, size_t work_bytes,
                 bq_stream_t st, int min_w144, int min_raw) {
    if (nparts < 1 || nparts > BQ_MAX_PARTS || rows < std::min(min_w144, min_raw)) return BQ_UNSUPPORTED;
    if (!ys || !ws || !ws[0] || !xq || !xd || !xsum) return BQ_EINVAL;
    if (!al16(work) || !al16(xq) || !al16(xd) || !al16(xsum) || !al16(xdh)) return BQ_EINVAL;
    const int K = ws[0]->K;
    PartTable pt;
    memset(&pt, 0, sizeof(pt));
    bool prepacked = true;
    for (int p = 0; p < nparts; ++p) {
        const bq_weight* w = ws[p];
        if (!w || !w->raw || !ys[p] || w->ggml_type != BQ_TYPE_Q5_K) return BQ_UNSUPPORTED;
        if (w->K != K || w->N <= 0 || (w->N % 128) != 0) return BQ_UNSUPPORTED;
        if (!al16(ys[p]) || !weight_al16(w)) return BQ_EINVAL;  // the tiles store 16-byte vectors
        if (!w->rep || !w->rep_min || (K % 512) != 0) prepacked = false;
        pt.Y[p] = ys[p];
        pt.N[p] = w->N;
    }
    if (K <= 0 || (K % 256) != 0) return BQ_UNSUPPORTED;
    if (prepacked && !xdh) prepacked = false;
    if (rows < (prepacked ? min_w144 : min_raw)) return BQ_UNSUPPORTED;
    pt.nparts = nparts;
    hipStream_t s = (hipStream_t)st;
    float* wf = (float*)work;
    const size_t wn = work ? work_bytes / sizeof(float) : 0;
    if (prepacked) {
        for (int p = 0; p < nparts; ++p) {
            pt.W[p] = ws[p]->rep;
            pt.aux[p] = ws[p]->rep_min;
        }
        return from_hip(launch_mmq_q5k_144(pt, rows, K, xq, xd, xsum, xdh, s, t_dev->cus, wf, wn));
    }
    for (int p = 0; p < nparts; ++p) pt.W[p] = ws[p]->raw;
    return from_hip(launch_mmq_q5k_raw(pt, rows, K, xq, xd, xsum, s, t_dev->cus, wf, wn));
}

// bq_gemm_b / bq_gemm_b_fused: the 8-row GEMV chunks stream the weights once
// per chunk (9216 x 3072: 9 rows 14.5 us, 20 rows 25.6 us, 32 rows 33 us);
// the MMQ kernels' 32-token tile takes 13-14 us at 9 rows and 16-17 us at 32
// (prepacked and raw), so both tiers take it above 8 rows.  (The reference
// sends rows 9..95 to its 64x64 MMA tile.)
constexpr int kGemmBMmqMin = 9;
}  // namespace

size_t bq_gemm_workspace_bytes_cus(int rows, int K, int n_total, int cus) {
    if (rows <= 0 || K <= 0 || n_total <= 0 || cus <= 0) return 0;
    // The largest split any tier or tile height takes for this shape: the
    // caller sizes one workspace per shape before it knows which tier a call
    // takes (the raw tier, which splits at 128-value stages, can take more
    // slices than the W144 and Q6_K kernels, which split at 256).
    const int ks = std::max(mmq_ksplit(rows, K, n_total, true, (size_t)-1, 128, cus),
                            mmq_ksplit(rows, K, n_total, true, (size_t)-1, 32, cus));
    const size_t split = ks > 1 ? (size_t)ks * rows * n_total * sizeof(float) : 0;
    return std::max(split, mmq_tail_ws_floats(rows, K, n_total, cus) * sizeof(float));
}

size_t bq_gemm_workspace_bytes(int rows, int K, int n_total) {
    // sized for the current device (0 when there is none: no split is taken
    // without a workspace, so a call still runs, unsplit)
    if (ensure_init() != BQ_OK) return 0;
    return bq_gemm_workspace_bytes_cus(rows, K, n_total, t_dev->cus);
}

int bq_try_mmq(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
               const int8_t* xq, const float* xd, const int32_t* xsum, uint16_t* xdh,
               void* work, size_t work_bytes, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    return try_mmq_impl(ys, ws, nparts, rows, xq, xd, xsum, xdh, work, work_bytes, st, kMmqMinRows, kMmqMinRows);
}

int bq_gemm_q6k_mma(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
                    void* work, size_t work_bytes, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!weight_ok(w) || !y || !xq || !xd || rows < 1) return BQ_EINVAL;
    if (!al16(y) || !al16(xq) || !al16(xd) || !al16(work) || !weight_al16(w)) return BQ_EINVAL;
    if (w->ggml_type != BQ_TYPE_Q6_K || !w->rep || (w->N % 128) != 0) return BQ_UNSUPPORTED;
    return from_hip(launch_mmq_q6k(one_part(y, w->rep, w->N), rows, w->K, xq, xd, (hipStream_t)st, t_dev->cus, (float*)work,
                                   work ? work_bytes / sizeof(float) : 0));
}

int bq_gemm_b(float* y, const bq_weight* w, int rows, const int8_t* xq, const float* xd,
              const int32_t* xsum, uint16_t* xdh, void* work, size_t work_bytes, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!weight_ok(w) || !y || !xq || !xd || rows < 0) return BQ_EINVAL;
    if (rows == 0) return BQ_OK;
    const bool q5 = w->ggml_type == BQ_TYPE_Q5_K, q6 = w->ggml_type == BQ_TYPE_Q6_K;
    if (!q5 && !q6) return BQ_UNSUPPORTED;
    if (q5 && !xsum) return BQ_EINVAL;
    if (rows > BQ_MAX_ROWS) {
        if (q5) {
            float* ys[1] = {y};
            const bq_weight* wsp[1] = {w};
            const int r = try_mmq_impl(ys, wsp, 1, rows, xq, xd, xsum, xdh, work, work_bytes, st, kGemmBMmqMin,
                                       kGemmBMmqMin);
            if (r != BQ_UNSUPPORTED) return r;
        } else if (w->rep && (w->N % 128) == 0) {
            return bq_gemm_q6k_mma(y, w, rows, xq, xd, work, work_bytes, st);
        }
    }
    // 1..8-row kernels, in 8-row chunks
    const int K = w->K, nb = K / 32;
    for (int r0 = 0; r0 < rows; r0 += BQ_MAX_ROWS) {
        const int c = std::min(rows - r0, (int)BQ_MAX_ROWS);
        float* yc = y + (size_t)r0 * w->N;
        int r;
        if (q6) {
            r = w->rep ? bq_gemm_q6k_dp(yc, w, c, xq, xd, r0, st) : bq_gemm_q6k_raw(yc, w, c, xq, xd, r0, st);
        } else {
            PartTable pt = one_part(yc, w->raw, w->N);
            r = gemv_rows(GemvKind::Q5K, pt, c, K, xq + (size_t)r0 * K, xd + (size_t)r0 * nb,
                          xsum + (size_t)r0 * nb, (hipStream_t)st);
        }
        if (r != BQ_OK) return r;
    }
    return BQ_OK;
}

namespace {
// Allocation-free scratch of bq_gemm_b_fused_noalloc: one file-scope device
// array, so each GPU the library runs on holds its own copy until the process
// ends.  [0, kScratchXdh): the W144 tier's xdh rows; the rest: the K-split
// workspace.  Host code never passes `scratch` itself to a kernel (in host
// code the name is a stand-in, not a device address): the address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kScratchBytes = 16u << 20;
constexpr size_t kScratchXdh = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// the current device's scratch address (looked up on its first use)
int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return from_hip(e);
    if (dev < 0 || dev >= kMaxDevices) return BQ_UNSUPPORTED;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return from_hip(e);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return BQ_OK;
}
}  // namespace

int bq_gemm_b_fused(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                    const int8_t* xq, const float* xd, const int32_t* xsum, uint16_t* xdh,
                    void* work, size_t work_bytes, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!ys || !ws || nparts < 1 || nparts > BQ_MAX_PARTS) return BQ_EINVAL;
    if (rows > BQ_MAX_ROWS) {
        const int r = try_mmq_impl(ys, ws, nparts, rows, xq, xd, xsum, xdh, work, work_bytes, st,
                                   kGemmBMmqMin, kGemmBMmqMin);
        if (r != BQ_UNSUPPORTED) return r;
    }
    for (int p = 0; p < nparts; ++p) {
        const int r = bq_gemm_b(ys[p], ws[p], rows, xq, xd, xsum, xdh, work, work_bytes, st);
        if (r != BQ_OK) return r;
    }
    return BQ_OK;
}

size_t bq_noalloc_scratch_bytes(void) { return kScratchBytes; }

int bq_gemm_b_fused_noalloc(float* const* ys, const bq_weight* const* ws, int nparts, int rows,
                            const int8_t* xq, const float* xd, const int32_t* xsum, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!ys || !ws || !ws[0] || nparts < 1 || nparts > BQ_MAX_PARTS || rows < 0) return BQ_EINVAL;
    if (rows == 0) return BQ_OK;
    const int K = ws[0]->K;
    if (K <= 0 || (K % 32) != 0) return BQ_EINVAL;
    // Only the prepacked (W144) tier reads xdh: every part Q5_K with its
    // repack, K % 512 == 0, N % 128 == 0 and more than 8 rows.  Such a call
    // needs xdh [rows][K/32] fp16 to fit its region; any other call passes no
    // xdh and takes the whole scratch as its K-split workspace.
    bool w144 = rows > BQ_MAX_ROWS && (K % 512) == 0;
    for (int p = 0; p < nparts && w144; ++p) {
        const bq_weight* w = ws[p];
        w144 = w && w->ggml_type == BQ_TYPE_Q5_K && w->rep && w->rep_min && (w->N % 128) == 0;
    }
    if (w144 && (size_t)rows * (size_t)(K / 32) * 2 > kScratchXdh) return BQ_ETOOBIG;
    void* base = nullptr;
    if (int r = scratch_ptr(&base)) return r;
    if (!w144) return bq_gemm_b_fused(ys, ws, nparts, rows, xq, xd, xsum, nullptr, base, kScratchBytes, st);
    uint16_t* xdh = (uint16_t*)base;
    void* work = (uint8_t*)base + kScratchXdh;
    return bq_gemm_b_fused(ys, ws, nparts, rows, xq, xd, xsum, xdh, work, kScratchBytes - kScratchXdh, st);
}

size_t bq_repack_q5k_bytes(int K, int N) { return (size_t)(K / 128) * N * 144; }
size_t bq_repack_q5k_min_bytes(int K, int N) { return (size_t)N * (K / 32) * 2; }
size_t bq_repack_q6k_bytes(int K, int N) { return (size_t)N * (K / 128) * 160; }

int bq_repack_q5k(const void* raw, int K, int N, void* w144, uint16_t* dm, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!raw || !w144 || !dm || K <= 0 || N <= 0 || (K % 256) != 0) return BQ_EINVAL;
    return from_hip(launch_repack_q5k(raw, K, N, w144, dm, (hipStream_t)st));
}

int bq_repack_q6k(const void* raw, int K, int N, void* w160, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!raw || !w160 || K <= 0 || N <= 0 || (K % 256) != 0) return BQ_EINVAL;
    return from_hip(launch_repack_q6k(raw, K, N, w160, (hipStream_t)st));
}

// Host repack (q6k_repack_host, bruce.cu:4783-4811).  Plain C++, no device.
int bq_repack_q6k_host(const void* rawv, int K, int N, void* dstv) {
    if (!rawv || !dstv || K <= 0 || N <= 0 || (K % 256) != 0) return BQ_EINVAL;
    const uint8_t* raw = (const uint8_t*)rawv;
    uint8_t* dst = (uint8_t*)dstv;
    const int nsb = K / 256, nst = K / 128;
    for (int n = 0; n < N; ++n)
        for (int s = 0; s < nst; ++s) {
            const uint8_t* b = raw + ((size_t)n * nsb + s / 2) * 210;
            const int hh = s & 1;
            uint8_t* o = dst + ((size_t)n * nst + s) * 160;
            const uint16_t hb = (uint16_t)(b[208] | (b[209] << 8));
            // binary16 -> binary32 with denormals (exponent 0 -> m * 2^-24)
            const uint32_t e = (hb >> 10) & 0x1F, m = hb & 0x3FF;
            float d;
            if (e == 0) {
                d = (float)m * 5.9604644775390625e-8f;
                if (hb & 0x8000) d = -d;
            } else {
                const uint32_t bits = ((uint32_t)(hb & 0x8000) << 16) |
                                      (e == 31 ? (0x7F800000u | (m << 13)) : (((e + 112u) << 23) | (m << 13)));
                memcpy(&d, &bits, 4);
            }
            for (int k = 0; k < 128; ++k) {
                const int u = k >> 5, l = k & 31;
                const uint8_t q = b[64 * hh + 32 * (u & 1) + l];
                const int lo = (u < 2) ? (q & 0xF) : (q >> 4);
                const int hi = (b[128 + 32 * hh + l] >> (2 * u)) & 3;
                o[k] = (uint8_t)(int8_t)((lo | (hi << 4)) - 32);
            }
            for (int g = 0; g < 8; ++g) {
                const float v = d * (float)(int8_t)b[192 + 8 * hh + g];
                memcpy(o + 128 + 4 * g, &v, 4);
            }
        }
    return BQ_OK;
}

// ---- q8 producers (norm + quantize) -----------------------------------------

namespace {
int norm_q8(int op, float* out, const float* a, const float* b, const float* c, const float* d, int rows,
            int n, int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (rows < 0 || n <= 0 || (n % 32) != 0) return BQ_EINVAL;
    if (rows == 0) return BQ_OK;
    if (!a || !xq || !xd || !xsum) return BQ_EINVAL;
    if (!al16(out) || !al16(a) || !al16(b) || !al16(c) || !al16(d) || !al16(xq)) return BQ_EINVAL;
    if (n > kNormMaxN) return BQ_UNSUPPORTED;
    return from_hip(launch_norm_q8(op, out, a, b, c, d, rows, n, xq, xd, xsum, (hipStream_t)st));
}
}  // namespace

int bq_norm_q8(float* dst, const float* src, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
               bq_stream_t st) {
    return norm_q8(0, dst, src, nullptr, nullptr, nullptr, rows, n, xq, xd, xsum, st);
}

int bq_add_norm_q8(float* x, const float* h, int rows, int n, int8_t* xq, float* xd, int32_t* xsum,
                   bq_stream_t st) {
    if (!x || !h) return BQ_EINVAL;
    return norm_q8(1, x, x, h, nullptr, nullptr, rows, n, xq, xd, xsum, st);
}

int bq_resid_q8(float* x, const float* upd, const float* alpha, int rows, int n, int8_t* xq, float* xd,
                int32_t* xsum, bq_stream_t st) {
    if (!x || !upd || !alpha) return BQ_EINVAL;
    return norm_q8(2, x, x, upd, alpha, nullptr, rows, n, xq, xd, xsum, st);
}

int bq_gate_norm_q8(float* dst, const float* aout, const float* gate, const float* sg, int rows, int n,
                    int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st) {
    if (!gate || !sg) return BQ_EINVAL;
    return norm_q8(3, dst, aout, gate, sg, nullptr, rows, n, xq, xd, xsum, st);
}

int bq_silu_mul_norm_q8(float* dst, const float* g, const float* u, const float* sg, const float* su, int rows,
                        int n, int8_t* xq, float* xd, int32_t* xsum, bq_stream_t st) {
    if (!u || !sg || !su) return BQ_EINVAL;
    return norm_q8(4, dst, g, u, sg, su, rows, n, xq, xd, xsum, st);
}

// ---- Q8_0 logits head ------------------------------------------------------

size_t bq_q8s_bytes(int K, int N) { return (size_t)N * (K / 256) * 272; }

int bq_quantize_q8s(const uint16_t* bf16, int K, int N, void* dst, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (K <= 0 || N < 0 || (K % 256) != 0) return BQ_EINVAL;
    if (N == 0) return BQ_OK;
    if (!bf16 || !dst || ((uintptr_t)bf16 & 15) || ((uintptr_t)dst & 15)) return BQ_EINVAL;
    return from_hip(launch_quant_q8s(bf16, K, N, (uint8_t*)dst, (hipStream_t)st));
}

namespace {
// binary32 -> binary16, round to nearest even (the reference's __float2half)
uint16_t host_f2h_rn(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520: inf
    uint32_t mant, shift, q;
    if (ax < 0x38800000u) {  // half denormal or zero: units of 2^-24
        if (ax < 0x33000000u) return (uint16_t)sign;
        mant = (ax & 0x7FFFFFu) | 0x800000u;
        shift = 126u - (ax >> 23);
        q = mant >> shift;
    } else {
        mant = ax;
        shift = 13u;
        q = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    }
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}
}  // namespace

// q8k_quant_host (bruce.cu:4843-4867): the same bytes as bq_quantize_q8s,
// including groups with 0 < amax < 127 * 2^-128 (id = inf), where the device
// kernels follow __float2int_rn: zeros -> 0, other values -> +-127.
int bq_quantize_q8s_host(const uint16_t* bf16, int K, int N, void* dstv) {
    if (K <= 0 || N < 0 || (K % 256) != 0) return BQ_EINVAL;
    if (N == 0) return BQ_OK;
    if (!bf16 || !dstv) return BQ_EINVAL;
    uint8_t* dst = (uint8_t*)dstv;
    const int nsb = K / 256;
    for (int r = 0; r < N; ++r)
        for (int s = 0; s < nsb; ++s) {
            uint8_t* blk = dst + ((size_t)r * nsb + s) * 272;
            for (int g = 0; g < 8; ++g) {
                const uint16_t* p = bf16 + (size_t)r * K + (size_t)s * 256 + (size_t)g * 32;
                float v[32], amax = 0.f;
                for (int i = 0; i < 32; ++i) {
                    const uint32_t bits = (uint32_t)p[i] << 16;
                    memcpy(&v[i], &bits, 4);
                    amax = std::max(amax, std::fabs(v[i]));
                }
                const float d = amax * (1.f / 127.f);
                const float id = d > 0.f ? 1.f / d : 0.f;
                const uint16_t h = host_f2h_rn(d);
                memcpy(blk + 2 * g, &h, 2);
                for (int i = 0; i < 32; ++i) {
                    // __float2int_rn semantics (PTX cvt.rni): NaN (0 * inf, when id
                    // overflows to inf) -> 0, +-inf saturates; then the clamp
                    const float t = v[i] * id;
                    const float c = t != t ? 0.f : std::min(127.f, std::max(-127.f, t));
                    blk[16 + 32 * g + i] = (uint8_t)(int8_t)std::lrint(c);
                }
            }
        }
    return BQ_OK;
}

int bq_gemv_q8s(float* y, const void* w, const int8_t* xq, const float* xd, int K, int N, int rows,
                const float* rs, bq_stream_t st) {
    if (int s = ensure_init()) return s;
    if (!y || !w || !xq || !xd || K <= 0 || N <= 0 || (K % 256) != 0) return BQ_EINVAL;
    if (!al16(w) || !al16(xq) || !al16(xd)) return BQ_EINVAL;
    if (rows < 1 || rows > BQ_MAX_ROWS || K > kQ8SMaxK) return BQ_UNSUPPORTED;
    return from_hip(launch_gemv_q8s(w, K, N, rows, xq, xd, rs, y, (hipStream_t)st, t_dev->cus));
}

}  // extern "C"
