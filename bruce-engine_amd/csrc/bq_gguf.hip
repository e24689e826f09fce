// bq_gguf.hip -- GGUF v3 reader and streaming weight loader feeding the
// repacks.  Host code only; the device work is
// hipMemcpyAsync plus the repack / conversion kernels of this library.
//
// Format (what engine/src/gguf.h:146-312 parses): little-endian
//   u32 magic "GGUF" | u32 version (3) | u64 n_tensors | u64 n_kv
//   n_kv x { string key, u32 type, value }        string = u64 length + bytes
//     value types 0..12: u8 i8 u16 i16 u32 i32 f32 bool string array u64 i64 f64
//     array = u32 element type, u64 count, elements
//   n_tensors x { string name, u32 ndim (<= 4), u64 ne[ndim], u32 ggml type, u64 offset }
//   data section at the first multiple of general.alignment (default 32);
//   tensor offsets are relative to it.
// Tensor byte sizes follow ggml's block sizes (gguf.h:40-75); only the types
// the reference can size are accepted (unknown types fail, as there).
//
// The metadata is read through the same pread path as the weights, with the
// prefix buffer grown until it holds the whole header (the reference reads a
// 32 MiB prefix and doubles it on "unexpected eof", gguf.h:163-176).
// Weights are streamed, not memory-mapped: pread into one of two pinned
// staging slots, hipMemcpyAsync to the caller's device buffer, so reading the
// next chunk overlaps the copy of the previous one (bruce.cu:4869-5131 streams
// through LS_SLOT-sized slots the same way).  The staging slots are allocated
// at the first load and freed by bq_gguf_close: loading is a set-up step, not
// a hot-path call.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/bq.h"
#include "bq_internal.hpp"

namespace {

size_t type_size(uint32_t t) {
    switch (t) {
        case 0: return 4;    // F32
        case 1: return 2;    // F16
        case 30: return 2;   // BF16
        case 2: return 18;   // Q4_0 (32 values)
        case 3: return 20;   // Q4_1
        case 6: return 22;   // Q5_0
        case 7: return 24;   // Q5_1
        case 8: return 34;   // Q8_0
        case 9: return 36;   // Q8_1
        case 10: return 84;  // Q2_K (256 values)
        case 11: return 110; // Q3_K
        case 12: return 144; // Q4_K
        case 13: return 176; // Q5_K
        case 14: return 210; // Q6_K
        case 20: return 18;  // IQ4_NL
        case 39: return 17;  // MXFP4
        default: return 0;
    }
}
int block_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: return 1;
        case 2: case 3: case 6: case 7: case 8: case 9: case 20: case 39: return 32;
        case 10: case 11: case 12: case 13: case 14: return 256;
        default: return 1;
    }
}

struct Value {
    uint32_t type = 0, arr_type = 0;
    double num = 0;
    std::string s;
    uint64_t arr_n = 0;
};

struct Tensor {
    std::string name, suffix;
    uint32_t type = 0, ndim = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
    int block = -1;
};

enum class Err { Ok, Eof, Bad };

struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    Err err = Err::Ok;
    template <typename T>
    T rd() {
        T v{};
        if (err != Err::Ok) return v;
        if ((size_t)(end - p) < sizeof(T)) { err = Err::Eof; return v; }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = rd<uint64_t>();
        if (err != Err::Ok) return {};
        if ((uint64_t)(end - p) < n) { err = Err::Eof; return {}; }
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if (err != Err::Ok) return;
        if ((uint64_t)(end - p) < n) { err = Err::Eof; return; }
        p += n;
    }
};

}  // namespace

struct bq_gguf {
    int fd = -1;
    uint64_t file_size = 0, data_offset = 0, n_kv = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, Value> kv;
    std::unordered_map<std::string, int64_t> by_name;
    // streaming slots (pinned), allocated at the first load
    void* slot[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    size_t slot_bytes = 0;

    bool read_at(void* dst, size_t n, uint64_t off) const {
        uint8_t* p = (uint8_t*)dst;
        while (n) {
            const ssize_t got = pread(fd, p, n, (off_t)off);
            if (got < 0) {
                if (errno == EINTR) continue;
                return false;
            }
            if (got == 0) return false;
            p += got;
            n -= (size_t)got;
            off += (uint64_t)got;
        }
        return true;
    }
    // The same with the range split over up to kReadThreads threads (pread is
    // position-independent): one thread copies page-cached data at ~20 GB/s,
    // below what the pinned host-to-device copy of the chunk takes (330 MB
    // streamed load: 1 / 2 / 4 / 8 threads 22 / 32 / 39 / 41 GB/s).  At most
    // half the hardware threads are used.
    static constexpr int kReadThreads = 8;
    bool read_at_parallel(void* dst, size_t n, uint64_t off) const {
        constexpr size_t kMinPiece = 4u << 20;
        const int hw = std::max(1, (int)std::thread::hardware_concurrency() / 2);
        const int nt = (int)std::min<size_t>(std::min(kReadThreads, hw), std::max<size_t>(1, n / kMinPiece));
        if (nt == 1) return read_at(dst, n, off);
        const size_t piece = (n / nt + 4095) & ~(size_t)4095;
        bool ok[kReadThreads] = {};
        std::thread th[kReadThreads - 1];
        int started = 0;
        for (int k = 1; k < nt; ++k) {
            const size_t b = std::min(n, piece * k), e = std::min(n, piece * (k + 1));
            try {
                th[k - 1] = std::thread([this, &ok, k, dst, b, e, off] {
                    ok[k] = read_at((uint8_t*)dst + b, e - b, off + b);
                });
                started = k;
            } catch (...) {  // no thread: read that piece here
                ok[k] = read_at((uint8_t*)dst + b, e - b, off + b);
                started = k;
            }
        }
        ok[0] = read_at(dst, std::min(n, piece), off);
        for (int k = 1; k <= started; ++k)
            if (th[k - 1].joinable()) th[k - 1].join();
        for (int k = 0; k < nt; ++k)
            if (!ok[k]) return false;
        return true;
    }

    // Parse the header from a prefix of the file; Err::Eof asks for a longer prefix.
    Err parse(const std::vector<uint8_t>& meta) {
        Cursor c{meta.data(), meta.data() + meta.size()};
        tensors.clear();
        kv.clear();
        by_name.clear();
        const uint32_t magic = c.rd<uint32_t>();
        const uint32_t version = c.rd<uint32_t>();
        const uint64_t nt = c.rd<uint64_t>();
        n_kv = c.rd<uint64_t>();
        if (c.err != Err::Ok) return c.err;
        if (magic != 0x46554747u || version != 3) return Err::Bad;
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string key = c.str();
            Value v;
            v.type = c.rd<uint32_t>();
            switch (v.type) {
                case 0: v.num = c.rd<uint8_t>(); break;
                case 1: v.num = c.rd<int8_t>(); break;
                case 2: v.num = c.rd<uint16_t>(); break;
                case 3: v.num = c.rd<int16_t>(); break;
                case 4: v.num = c.rd<uint32_t>(); break;
                case 5: v.num = c.rd<int32_t>(); break;
                case 6: v.num = c.rd<float>(); break;
                case 7: v.num = c.rd<uint8_t>() ? 1 : 0; break;
                case 8: v.s = c.str(); break;
                case 10: v.num = (double)c.rd<uint64_t>(); break;
                case 11: v.num = (double)c.rd<int64_t>(); break;
                case 12: v.num = c.rd<double>(); break;
                case 9: {
                    v.arr_type = c.rd<uint32_t>();
                    v.arr_n = c.rd<uint64_t>();
                    static const uint8_t esz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
                    if (c.err != Err::Ok) return c.err;
                    if (v.arr_type == 8) {
                        for (uint64_t k = 0; k < v.arr_n && c.err == Err::Ok; ++k) c.str();
                    } else if (v.arr_type < 13 && esz[v.arr_type]) {
                        if (v.arr_n > (uint64_t)(c.end - c.p) / esz[v.arr_type]) return Err::Eof;
                        c.skip(v.arr_n * esz[v.arr_type]);
                    } else {
                        return Err::Bad;
                    }
                    break;
                }
                default: return c.err != Err::Ok ? c.err : Err::Bad;
            }
            if (c.err != Err::Ok) return c.err;
            kv[key] = std::move(v);
        }
        uint64_t align = 32;
        auto it = kv.find("general.alignment");
        if (it != kv.end() && it->second.num >= 1) align = (uint64_t)it->second.num;
        tensors.reserve((size_t)std::min<uint64_t>(nt, 1u << 20));
        for (uint64_t i = 0; i < nt; ++i) {
            Tensor t;
            t.name = c.str();
            t.ndim = c.rd<uint32_t>();
            if (c.err != Err::Ok) return c.err;
            if (t.ndim > 4) return Err::Bad;
            for (uint32_t d = 0; d < t.ndim; ++d) t.ne[d] = c.rd<uint64_t>();
            t.type = c.rd<uint32_t>();
            t.offset = c.rd<uint64_t>();
            if (c.err != Err::Ok) return c.err;
            const size_t ts = type_size(t.type);
            if (!ts) return Err::Bad;
            uint64_t n = 1;
            for (uint32_t d = 0; d < t.ndim; ++d) n *= t.ne[d];
            t.nbytes = n / (uint64_t)block_size(t.type) * ts;
            if (t.name.rfind("blk.", 0) == 0) {
                const size_t dot = t.name.find('.', 4);
                if (dot != std::string::npos) {
                    t.block = atoi(t.name.substr(4, dot - 4).c_str());
                    t.suffix = t.name.substr(dot + 1);
                }
            }
            by_name[t.name] = (int64_t)tensors.size();
            tensors.push_back(std::move(t));
        }
        const uint64_t pos = (uint64_t)(c.p - meta.data());
        data_offset = (pos + align - 1) / align * align;
        return Err::Ok;
    }

    void free_slots() {
        for (int s = 0; s < 2; ++s) {
            if (done[s]) (void)hipEventDestroy(done[s]);
            if (slot[s]) (void)hipHostFree(slot[s]);
            done[s] = nullptr;
            slot[s] = nullptr;
        }
        slot_bytes = 0;
    }
};

namespace {
constexpr size_t kSlotBytes = 64u << 20;  // one staging slot

int slots_ready(bq_gguf* g) {
    if (g->slot[0]) return BQ_OK;
    for (int s = 0; s < 2; ++s) {
        if (hipHostMalloc(&g->slot[s], kSlotBytes, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&g->done[s], hipEventDisableTiming) != hipSuccess) {
            g->free_slots();
            return -(int)hipErrorOutOfMemory;
        }
    }
    g->slot_bytes = kSlotBytes;
    return BQ_OK;
}

// Stream `n` bytes at file offset `off` to device memory `dst` on `st`.
int stream_to_device(bq_gguf* g, uint64_t off, size_t n, uint8_t* dst, hipStream_t st) {
    if (int r = slots_ready(g)) return r;
    int s = 0;
    bool used[2] = {false, false};
    for (size_t done = 0; done < n; done += g->slot_bytes, s ^= 1) {
        const size_t len = std::min(g->slot_bytes, n - done);
        if (used[s] && hipEventSynchronize(g->done[s]) != hipSuccess) return -(int)hipErrorUnknown;
        if (!g->read_at_parallel(g->slot[s], len, off + done)) return BQ_EINVAL;
        if (hipMemcpyAsync(dst + done, g->slot[s], len, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipEventRecord(g->done[s], st) != hipSuccess)
            return -(int)hipErrorUnknown;
        used[s] = true;
    }
    // the slots are reused by the next call: wait for the last copies
    for (int k = 0; k < 2; ++k)
        if (used[k] && hipEventSynchronize(g->done[k]) != hipSuccess) return -(int)hipErrorUnknown;
    return BQ_OK;
}
}  // namespace

extern "C" {

int bq_gguf_open(const char* path, bq_gguf** out) {
    if (!path || !out) return BQ_EINVAL;
    *out = nullptr;
    bq_gguf* g = new (std::nothrow) bq_gguf();
    if (!g) return BQ_EINVAL;
    g->fd = ::open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        bq_gguf_close(g);
        return BQ_EINVAL;
    }
    g->file_size = (uint64_t)st.st_size;
    size_t want = (size_t)std::min<uint64_t>(g->file_size, 1u << 20);
    std::vector<uint8_t> meta;
    for (;;) {
        meta.resize(want);
        if (!g->read_at(meta.data(), want, 0)) {
            bq_gguf_close(g);
            return BQ_EINVAL;
        }
        const Err e = g->parse(meta);
        if (e == Err::Ok) break;
        if (e == Err::Bad || want >= g->file_size) {
            bq_gguf_close(g);
            return BQ_EINVAL;
        }
        want = (size_t)std::min<uint64_t>(g->file_size, (uint64_t)want * 2);
    }
    // every tensor must lie inside the file
    for (const Tensor& t : g->tensors)
        if (g->data_offset + t.offset + t.nbytes > g->file_size) {
            bq_gguf_close(g);
            return BQ_EINVAL;
        }
    *out = g;
    return BQ_OK;
}

void bq_gguf_close(bq_gguf* g) {
    if (!g) return;
    g->free_slots();
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

int64_t bq_gguf_n_tensors(const bq_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t bq_gguf_find(const bq_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

int bq_gguf_tensor_info(const bq_gguf* g, int64_t i, bq_gguf_tensor* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return BQ_EINVAL;
    const Tensor& t = g->tensors[(size_t)i];
    out->name = t.name.c_str();
    out->ggml_type = t.type;
    out->ndim = t.ndim;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = g->data_offset + t.offset;
    out->nbytes = t.nbytes;
    out->block = t.block;
    out->suffix = t.suffix.c_str();
    return BQ_OK;
}

int bq_gguf_kv_num(const bq_gguf* g, const char* key, double* out) {
    if (!g || !key || !out) return BQ_EINVAL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type == 8 || it->second.type == 9) return BQ_UNSUPPORTED;
    *out = it->second.num;
    return BQ_OK;
}

int bq_gguf_kv_str(const bq_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return BQ_EINVAL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 8) return BQ_UNSUPPORTED;
    *out = it->second.s.c_str();
    return BQ_OK;
}

int bq_gguf_read(const bq_gguf* g, int64_t i, void* dst, size_t n, uint64_t off) {
    if (!g || !dst || i < 0 || i >= (int64_t)g->tensors.size()) return BQ_EINVAL;
    const Tensor& t = g->tensors[(size_t)i];
    if (off > t.nbytes || n > t.nbytes - off) return BQ_EINVAL;
    return g->read_at(dst, n, g->data_offset + t.offset + off) ? BQ_OK : BQ_EINVAL;
}

int bq_gguf_load(bq_gguf* g, int64_t i, void* raw, void* rep, void* rep_min, bq_weight* w, bq_stream_t st) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return BQ_EINVAL;
    const Tensor& t = g->tensors[(size_t)i];
    if (t.ndim != 2 || t.ne[0] > (1u << 30) || t.ne[1] > (1u << 30)) return BQ_UNSUPPORTED;
    const int K = (int)t.ne[0], N = (int)t.ne[1];
    const bool q5 = t.type == BQ_TYPE_Q5_K, q6 = t.type == BQ_TYPE_Q6_K, bf = t.type == 30;
    if (!q5 && !q6 && !bf) return BQ_UNSUPPORTED;
    if ((K % 256) != 0) return BQ_UNSUPPORTED;
    if (!raw) return BQ_EINVAL;
    if (q5 && (rep != nullptr) != (rep_min != nullptr)) return BQ_EINVAL;
    if (bf && !rep) return BQ_EINVAL;  // a BF16 matrix is only loaded as its Q8S conversion
    if (int s = bq_init()) return s;
    hipStream_t s = (hipStream_t)st;
    if (int r = stream_to_device(g, g->data_offset + t.offset, (size_t)t.nbytes, (uint8_t*)raw, s)) return r;
    int r = BQ_OK;
    if (q5 && rep) r = bq_repack_q5k(raw, K, N, rep, (uint16_t*)rep_min, st);
    else if (q6 && rep) r = bq_repack_q6k(raw, K, N, rep, st);
    else if (bf) r = bq_quantize_q8s((const uint16_t*)raw, K, N, rep, st);
    if (r != BQ_OK) return r;
    if (w) {
        w->raw = bf ? rep : raw;
        w->rep = bf ? nullptr : rep;
        w->rep_min = q5 ? rep_min : nullptr;
        w->ggml_type = bf ? 8u : t.type;  // the converted head is Q8_0-family
        w->K = K;
        w->N = N;
    }
    return BQ_OK;
}

}  // extern "C"
