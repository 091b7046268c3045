// GGUF ingestion: a reader for GGUF v2 / v3 files (memory-mapped, every length and offset
// bounds-checked) and a streaming loader that turns one tensor into a device weight.
//
// The reference crate receives its weights as jero_core::TensorView byte slices of a GGUF
// file and repacks them at load time, in parallel over tile ranges (repack_into_tile_range,
// repack.rs:1579, assembled by RepackedWeight::from_tile_buffers, repack.rs:2386). Here the
// loader streams the tensor's rows through two pinned host buffers: while the DMA engine copies
// chunk k to the device and the device repacks it (jk_weight_repack_tile_range), host threads
// copy chunk k + 1 out of the mapped file. The bytes are handed over unchanged, exactly as a
// TensorView over the file would hand them to the reference.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <system_error>
#include <thread>
#include <vector>

#include "jk_internal.hpp"

using namespace jk;

namespace {

struct TensorRec {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t rel_offset = 0;  // from the start of the data section
    uint64_t nbytes = 0;      // 0 when the type's size is not known here
};

constexpr uint64_t kBytesOverflow = UINT64_MAX;  // type_bytes: the byte count does not fit 64 bits

// Bytes of n elements of ggml type t (the block formats this library reads, plus the dense
// types a model file commonly holds), 0 when unknown or not a whole number of blocks,
// kBytesOverflow when the count does not fit in 64 bits.
uint64_t type_bytes(uint32_t t, uint64_t n) {
    uint64_t unit = 0, count = n, extra = 0;
    switch (t) {
    case 0: unit = 4; break;   // F32
    case 1: unit = 2; break;   // F16
    case 30: unit = 2; break;  // BF16
    default: {
        if (!fmt_known((int)t)) return 0;
        const Fmt f = fmt_of((int)t);
        if (n % (uint64_t)f.be) return 0;
        unit = (uint64_t)f.bb;
        count = n / (uint64_t)f.be;
        extra = trailer_bytes((int)t);
    }
    }
    if (count > (UINT64_MAX - extra) / unit) return kBytesOverflow;
    return count * unit + extra;
}

// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
    const uint8_t *p;
    uint64_t size, pos = 0;
    bool ok = true;
    bool take(void *dst, uint64_t n) {
        if (!ok || n > size - pos) return ok = false;
        memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!ok || n > size - pos) return ok = false;
        pos += n;
        return true;
    }
    uint32_t u32() {
        uint32_t v = 0;
        take(&v, 4);
        return v;
    }
    uint64_t u64() {
        uint64_t v = 0;
        take(&v, 8);
        return v;
    }
    bool str(std::string *out) {
        const uint64_t n = u64();
        if (!ok || n > size - pos) return ok = false;
        if (out) out->assign((const char *)p + pos, n);
        pos += n;
        return true;
    }
};

// Skips (or, for general.alignment, reads) one metadata value of type vt.
bool read_value(Cursor &c, uint32_t vt, int depth, uint64_t *as_u64) {
    static const uint8_t kSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (vt > 12) return c.ok = false;
    if (vt == 8) return c.str(nullptr);
    if (vt == 9) {  // array: element type, count, elements
        if (depth > 4) return c.ok = false;
        const uint32_t et = c.u32();
        const uint64_t n = c.u64();
        if (!c.ok || et > 12) return c.ok = false;
        if (et != 8 && et != 9) {
            if (n > (c.size - c.pos) / kSize[et]) return c.ok = false;
            return c.skip(n * kSize[et]);
        }
        for (uint64_t i = 0; i < n && c.ok; ++i) read_value(c, et, depth + 1, nullptr);
        return c.ok;
    }
    uint64_t v = 0;
    if (!c.take(&v, kSize[vt])) return false;
    if (as_u64) *as_u64 = v;
    return true;
}

}  // namespace

struct jk_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_start = 0, n_kv = 0;
    std::vector<TensorRec> tensors;
    // Streaming buffers, kept from one load to the next (loads of one file are serialized):
    // two pinned host buffers, two device staging buffers on device `device`, their events.
    std::mutex mu;
    size_t buf_bytes = 0;
    int device = -1;
    void *pinned[2] = {nullptr, nullptr}, *staging[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
};

static void release_buffers(jk_gguf *g) {
    for (int b = 0; b < 2; ++b) {
        if (g->ev[b]) (void)hipEventDestroy(g->ev[b]);
        if (g->staging[b]) (void)hipFree(g->staging[b]);
        if (g->pinned[b]) (void)hipHostFree(g->pinned[b]);
        g->ev[b] = nullptr;
        g->staging[b] = g->pinned[b] = nullptr;
    }
    g->buf_bytes = 0;
    g->device = -1;
}

// Makes the streaming buffers hold at least bytes each, on the current device.
static hipError_t ensure_buffers(jk_gguf *g, size_t bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (g->buf_bytes >= bytes && g->device == dev) return hipSuccess;
    release_buffers(g);
    for (int b = 0; b < 2 && e == hipSuccess; ++b) {
        e = hipHostMalloc(&g->pinned[b], bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&g->staging[b], bytes);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&g->ev[b], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        release_buffers(g);
        return e;
    }
    g->buf_bytes = bytes;
    g->device = dev;
    return hipSuccess;
}

static void gguf_release(jk_gguf *g) {
    if (g->buf_bytes) release_buffers(g);
    if (g->map) munmap((void *)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

static jk_status gguf_parse(jk_gguf *g, const char *path) {
    Cursor c{g->map, g->size};
    uint32_t magic = c.u32();
    if (!c.ok || magic != 0x46554747u) return fail(JK_TENSOR_BOUNDS, "%s: not a GGUF file (bad magic)", path);
    g->version = c.u32();
    if (g->version != 2 && g->version != 3)
        return fail(JK_CAPABILITY_MISMATCH, "%s: GGUF version %u is not supported (2 and 3 are)", path, g->version);
    const uint64_t n_tensors = c.u64();
    g->n_kv = c.u64();
    if (!c.ok) return fail(JK_TENSOR_BOUNDS, "%s: truncated GGUF header", path);
    for (uint64_t i = 0; i < g->n_kv; ++i) {
        std::string key;
        c.str(&key);
        const uint32_t vt = c.u32();
        uint64_t v = 0;
        read_value(c, vt, 0, &v);
        if (!c.ok) return fail(JK_TENSOR_BOUNDS, "%s: metadata entry %llu is truncated or malformed", path,
                               (unsigned long long)i);
        if (key == "general.alignment") {
            if (vt != 4 || v == 0 || (v & (v - 1)))
                return fail(JK_TENSOR_BOUNDS, "%s: general.alignment must be a power-of-two uint32", path);
            g->alignment = v;
        }
    }
    if (n_tensors > (g->size - c.pos) / 24)  // every tensor record holds at least 24 bytes
        return fail(JK_TENSOR_BOUNDS, "%s: tensor count %llu exceeds the file", path, (unsigned long long)n_tensors);
    // (records are appended as they are read: the count is only bounded by the file size)
    g->tensors.reserve((size_t)std::min<uint64_t>(n_tensors, 4096));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        g->tensors.emplace_back();
        TensorRec &t = g->tensors.back();
        c.str(&t.name);
        t.n_dims = c.u32();
        if (c.ok && (t.n_dims == 0 || t.n_dims > 4))
            return fail(JK_TENSOR_BOUNDS, "%s: tensor %s has %u dimensions", path, t.name.c_str(), t.n_dims);
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims && c.ok; ++d) {
            t.ne[d] = c.u64();
            if (t.ne[d] == 0 || n > UINT64_MAX / t.ne[d]) c.ok = false;
            else n *= t.ne[d];
        }
        t.type = c.u32();
        t.rel_offset = c.u64();
        if (!c.ok) return fail(JK_TENSOR_BOUNDS, "%s: tensor record %llu is truncated or malformed", path,
                               (unsigned long long)i);
        if (t.rel_offset % g->alignment)
            return fail(JK_TENSOR_BOUNDS, "%s: tensor %s offset %llu is not %llu-aligned", path, t.name.c_str(),
                        (unsigned long long)t.rel_offset, (unsigned long long)g->alignment);
        t.nbytes = type_bytes(t.type, n);
        if (t.nbytes == kBytesOverflow)
            return fail(JK_TENSOR_BOUNDS, "%s: tensor %s byte count overflows 64 bits", path, t.name.c_str());
    }
    g->data_start = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const TensorRec &t : g->tensors) {
        if (g->data_start > g->size || t.rel_offset > g->size - g->data_start ||
            t.nbytes > g->size - g->data_start - t.rel_offset)
            return fail(JK_TENSOR_BOUNDS, "%s: tensor %s data lies outside the file", path, t.name.c_str());
    }
    return JK_OK;
}

// C++ exceptions (an allocation that fails, a thread that cannot start) never cross the C
// ABI: the extern "C" entries below that allocate turn them into an error status.
template <class F>
static jk_status no_throw(const char *what, F &&f) {
    try {
        return f();
    } catch (const std::exception &e) {
        return fail(JK_TENSOR_BOUNDS, "%s: %s", what, e.what());
    } catch (...) {
        return fail(JK_TENSOR_BOUNDS, "%s: unexpected exception", what);
    }
}

static jk_status gguf_open(const char *path, jk_gguf **out);
static jk_status gguf_load_weight(jk_stream s, const jk_gguf *g, size_t i, size_t chunk_bytes, jk_weight **out);

extern "C" {

jk_status jk_gguf_open(const char *path, jk_gguf **out) {
    return no_throw("jk_gguf_open", [&] { return gguf_open(path, out); });
}

jk_status jk_gguf_load_weight(jk_stream s, const jk_gguf *g, size_t i, size_t chunk_bytes, jk_weight **out) {
    return no_throw("jk_gguf_load_weight", [&] { return gguf_load_weight(s, g, i, chunk_bytes, out); });
}

}  // extern "C"

static jk_status gguf_open(const char *path, jk_gguf **out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "gguf: null out-pointer");
    *out = nullptr;
    if (!path) return fail(JK_TENSOR_BOUNDS, "gguf: null path");
    // the handle is released on every way out but success, exceptions included
    struct Guard {
        jk_gguf *g;
        ~Guard() {
            if (g) gguf_release(g);
        }
    } guard{new jk_gguf()};
    jk_gguf *g = guard.g;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0)
        return fail(JK_TENSOR_BOUNDS, "gguf: cannot open %s: %s", path, strerror(errno));
    g->size = (uint64_t)st.st_size;
    if (g->size < 24)
        return fail(JK_TENSOR_BOUNDS, "%s: not a GGUF file (%llu bytes)", path, (unsigned long long)g->size);
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fail(JK_TENSOR_BOUNDS, "gguf: cannot map %s: %s", path, strerror(errno));
    g->map = (const uint8_t *)m;
    JK_TRY(gguf_parse(g, path));
    *out = g;
    guard.g = nullptr;
    return JK_OK;
}

extern "C" {

jk_status jk_gguf_close(jk_gguf *g) {
    if (g) gguf_release(g);
    return JK_OK;
}

jk_status jk_gguf_get_file_info(const jk_gguf *g, jk_gguf_file_info *out) {
    if (!g || !out) return fail(JK_TENSOR_BOUNDS, "gguf: null argument");
    out->version = g->version;
    out->n_tensors = g->tensors.size();
    out->n_kv = g->n_kv;
    out->alignment = g->alignment;
    out->data_offset = g->data_start;
    out->file_bytes = g->size;
    return JK_OK;
}

jk_status jk_gguf_tensor_info(const jk_gguf *g, size_t i, jk_gguf_tensor *out) {
    if (!g || !out) return fail(JK_TENSOR_BOUNDS, "gguf: null argument");
    if (i >= g->tensors.size())
        return fail(JK_TENSOR_BOUNDS, "gguf: tensor index %zu >= %zu tensors", i, g->tensors.size());
    const TensorRec &t = g->tensors[i];
    out->name = t.name.c_str();
    out->ggml_type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = g->data_start + t.rel_offset;
    out->nbytes = t.nbytes;
    out->data = t.nbytes ? g->map + g->data_start + t.rel_offset : nullptr;
    return JK_OK;
}

jk_status jk_gguf_find(const jk_gguf *g, const char *name, size_t *index) {
    if (!g || !name || !index) return fail(JK_TENSOR_BOUNDS, "gguf: null argument");
    for (size_t i = 0; i < g->tensors.size(); ++i)
        if (g->tensors[i].name == name) {
            *index = i;
            return JK_OK;
        }
    return fail(JK_TENSOR_BOUNDS, "gguf: no tensor named %s", name);
}

}  // extern "C"

static jk_status gguf_load_weight(jk_stream s, const jk_gguf *g, size_t i, size_t chunk_bytes, jk_weight **out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "gguf: null weight out-pointer");
    *out = nullptr;
    if (!g) return fail(JK_TENSOR_BOUNDS, "gguf: null file");
    if (i >= g->tensors.size())
        return fail(JK_TENSOR_BOUNDS, "gguf: tensor index %zu >= %zu tensors", i, g->tensors.size());
    const TensorRec &t = g->tensors[i];
    if (!fmt_known((int)t.type))
        return fail(JK_CAPABILITY_MISMATCH, "%s: ggml type %u is not a block format of this library", t.name.c_str(),
                    t.type);
    if (t.n_dims != 2) return fail(JK_TENSOR_BOUNDS, "%s: a weight matrix has 2 dimensions, not %u", t.name.c_str(),
                                   t.n_dims);
    // TensorView over the mapped bytes: shape [ne0, ne1] = [cols, rows].
    const size_t shape[2] = {(size_t)t.ne[0], (size_t)t.ne[1]};
    jk_tensor_view v = {t.name.c_str(), (int32_t)t.type, shape, 2, g->map + g->data_start + t.rel_offset,
                        (size_t)t.nbytes, g->data_start + t.rel_offset};
    jk_weight_layout L;
    JK_TRY(jk_weight_layout_for(&v, shape[1], shape[0], &L));
    jk_weight *w = nullptr;
    JK_TRY(jk_weight_create(s, &L, &w));
    w->name = t.name;
    w->offset = v.offset;
    if (chunk_bytes == 0) chunk_bytes = (size_t)32 << 20;
    const size_t tile_bytes = 8 * L.row_bytes;
    const size_t tiles_per_chunk = std::max<size_t>(1, chunk_bytes / tile_bytes);
    const size_t buf_bytes = std::min(tiles_per_chunk * tile_bytes, L.rows * L.row_bytes);
    hipStream_t st = (hipStream_t)s;
    jk_gguf *gm = const_cast<jk_gguf *>(g);  // the streaming buffers are the handle's cache
    std::lock_guard<std::mutex> lock(gm->mu);
    jk_status rs = JK_OK;
    hipError_t e = ensure_buffers(gm, buf_bytes);
    void *const *pinned = gm->pinned, *const *staging = gm->staging;
    hipEvent_t *ev = gm->ev;
    const unsigned nthreads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    try {
        th.reserve(nthreads);  // (no reallocation below; without it every part is copied here)
    } catch (const std::bad_alloc &) {
    }
    const uint8_t *src = (const uint8_t *)v.bytes;
    for (size_t t0 = 0, k = 0; e == hipSuccess && rs == JK_OK && t0 < L.n_tiles; t0 += tiles_per_chunk, ++k) {
        const size_t t1 = std::min(L.n_tiles, t0 + tiles_per_chunk);
        const size_t r0 = t0 * 8, r1 = std::min(L.rows, t1 * 8);
        const size_t bytes = (r1 - r0) * L.row_bytes;
        const int b = (int)(k & 1);
        if (k >= 2) e = hipEventSynchronize(ev[b]);  // the DMA of chunk k - 2 has read this buffer
        if (e != hipSuccess) break;
        // host threads copy the chunk out of the mapping (page faults and all) in parallel; a
        // thread that cannot be started leaves its part (and the later ones) to this thread
        const size_t part = (bytes + nthreads - 1) / nthreads;
        auto copy_part = [&](unsigned p) {
            const size_t o = p * part, n = std::min(part, bytes - o);
            memcpy((uint8_t *)pinned[b] + o, src + r0 * L.row_bytes + o, n);
        };
        th.clear();
        unsigned started = 0;
        try {
            for (; started < th.capacity() && started < nthreads && started * part < bytes; ++started)
                th.emplace_back(copy_part, started);
        } catch (const std::system_error &) {
        }
        for (unsigned p = started; p < nthreads && p * part < bytes; ++p) copy_part(p);
        for (auto &x : th) x.join();
        e = hipMemcpyAsync(staging[b], pinned[b], bytes, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) rs = jk_weight_repack_tile_range(s, w, staging[b], bytes, t0, t1);
        if (e == hipSuccess && rs == JK_OK) e = hipEventRecord(ev[b], st);
    }
    // Complete before the buffers are reused or the handle is returned.
    const hipError_t se = hipStreamSynchronize(st);
    if (e == hipSuccess) e = se;
    if (rs == JK_OK && e != hipSuccess) rs = hip_fail(e, "jk_gguf_load_weight");
    if (rs == JK_OK) rs = jk_weight_seal(w);
    if (rs != JK_OK) {
        jk_weight_free(w);
        return rs;
    }
    *out = w;
    return JK_OK;
}

