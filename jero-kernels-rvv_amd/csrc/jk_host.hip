// jk_host.hip -- host tier: synchronous host-memory mirrors of the reference signatures.
//
// Each call validates exactly as the reference entry it mirrors, copies its activation in,
// runs the device-tier kernel on the calling thread's stream, copies the result back and
// synchronizes that stream.
//
// Weights can be kept resident (opt in). By default every call uploads its weight, as the
// reference reads the slice's bytes on every call. After jk_host_cache_set_limit(bytes > 0), a
// weight named by a TensorView (host bytes) is uploaded once and cached, keyed by the view's byte
// range, format and matrix shape plus a fingerprint of sampled bytes; later calls with the same
// view reuse the device copy without any upload or allocation. The cache then assumes what the
// reference's callers give it, immutable weight slices (a model's tensors, typically a
// memory-mapped file): bytes behind a cached view must not change while it is cached, unless
// jk_host_cache_invalidate is called for them (the fingerprint catches a buffer that is freed and
// refilled with a different tensor at the same address in all but contrived cases). With
// jk_host_cache_set_verify(1) every cache hit also hashes all of the view's bytes and compares
// them with the hash taken at upload; a mismatch drops the entry and uploads again
// (stale_reuploads counts these), so an in-place edit cannot return results of the old bytes.
// Entries are evicted least-recently-used beyond the byte limit; an entry in use by a call is
// never freed under it.
//
// Per-call device memory (activations, outputs, workspaces) comes from a per-thread scratch
// buffer that only grows; a thread's stream and scratch are kept until jk_host_release_thread.
// With a warm cache and scratch, a call performs no device allocation.
#include <limits.h>
#include <string.h>

#include <list>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "jk_internal.hpp"

namespace jk {

// ------------------------------------------------------------------ statistics
static std::atomic<uint64_t> g_uploads{0}, g_hits{0}, g_evictions{0}, g_device_allocs{0}, g_stale{0};
static std::atomic<bool> g_verify{false};

// ------------------------------------------------------------------ per-thread context
struct HostCtx {
    int device = -1;
    hipStream_t stream = nullptr;
    void *scratch = nullptr;
    size_t cap = 0;
};
static thread_local HostCtx *t_ctx = nullptr;

static jk_status ctx_get(HostCtx **out) {
    int dev = 0;
    JK_HIP(hipGetDevice(&dev));
    if (t_ctx && t_ctx->device != dev) {
        // the thread switched devices: its stream and scratch belong to the old one
        (void)hipStreamSynchronize(t_ctx->stream);
        int cur = dev;
        (void)hipSetDevice(t_ctx->device);
        if (t_ctx->scratch) (void)hipFree(t_ctx->scratch);
        (void)hipStreamDestroy(t_ctx->stream);
        (void)hipSetDevice(cur);
        delete t_ctx;
        t_ctx = nullptr;
    }
    if (!t_ctx) {
        HostCtx *c = new HostCtx();
        c->device = dev;
        const hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            return hip_fail(e, "host tier stream");
        }
        t_ctx = c;
    }
    *out = t_ctx;
    return JK_OK;
}

// Carves consecutive 256-byte aligned sections out of the thread's scratch, growing it first
// when the request does not fit (the only allocation of a warm call path is this growth).
struct Scratch {
    HostCtx *c;
    size_t sizes[6];
    int n = 0;
    void *p[6];
    jk_status take(std::initializer_list<size_t> need) {
        size_t total = 0;
        n = 0;
        for (size_t b : need) {
            sizes[n++] = total;
            total += (b + 255) / 256 * 256;
        }
        if (total > c->cap) {
            JK_HIP(hipStreamSynchronize(c->stream));
            if (c->scratch) JK_HIP(hipFree(c->scratch));
            c->scratch = nullptr;
            c->cap = 0;
            const size_t grow = std::max(total, (size_t)1 << 20);
            JK_HIP(hipMalloc(&c->scratch, grow));
            g_device_allocs.fetch_add(1);
            c->cap = grow;
        }
        for (int i = 0; i < n; ++i) p[i] = static_cast<uint8_t *>(c->scratch) + sizes[i];
        return JK_OK;
    }
};

static jk_status h2d(HostCtx *c, void *dst, const void *src, size_t n) {
    if (n) JK_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
    return JK_OK;
}

// Copies back and waits for the thread's stream.
static jk_status d2h_sync(HostCtx *c, void *dst, const void *src, size_t n) {
    if (n) JK_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
    JK_HIP(hipStreamSynchronize(c->stream));
    return JK_OK;
}

// ------------------------------------------------------------------ resident weights
struct CacheKey {
    int device;
    const void *ptr;
    size_t len;
    int quant;
    size_t rows, cols;
    uint64_t fp;
    bool operator==(const CacheKey &o) const {
        return device == o.device && ptr == o.ptr && len == o.len && quant == o.quant && rows == o.rows &&
               cols == o.cols && fp == o.fp;
    }
};
struct CacheKeyHash {
    size_t operator()(const CacheKey &k) const {
        uint64_t h = (uint64_t)(uintptr_t)k.ptr * 0x9E3779B97F4A7C15ull;
        h ^= (uint64_t)k.len + 0x632BE59BD9B4E019ull + (h << 6) + (h >> 2);
        h ^= (uint64_t)k.rows * 31 + (uint64_t)k.cols * 131 + (uint64_t)k.quant * 7 + (uint64_t)k.device;
        return (size_t)(h ^ k.fp);
    }
};

struct CacheEntry {
    CacheKey key;
    jk_weight *w = nullptr;
    size_t bytes = 0;
    uint64_t full = 0;  // hash of every byte of the view at upload (verify mode)
    int users = 0;
    bool evicted = false;
};

struct WeightCache {
    std::mutex mu;
    size_t limit = 0;  // residency is opt in
    size_t bytes = 0;
    std::list<std::shared_ptr<CacheEntry>> lru;  // front: most recently used
    std::unordered_map<CacheKey, std::list<std::shared_ptr<CacheEntry>>::iterator, CacheKeyHash> map;
};
// Never destroyed: entries may be released by threads during process teardown.
static WeightCache &cache() {
    static WeightCache *c = new WeightCache();
    return *c;
}

// FNV-1a over every byte of views up to 64 KiB; beyond that over the first and last 1 KiB and
// 256 evenly spaced 64-byte windows (about 18 KiB, a few microseconds).
static uint64_t fingerprint(const uint8_t *p, size_t n) {
    uint64_t h = 0xCBF29CE484222325ull;
    auto mix = [&](size_t off, size_t len) {
        for (size_t i = 0; i < len && off + i < n; ++i) h = (h ^ p[off + i]) * 0x100000001B3ull;
    };
    if (n <= ((size_t)64 << 10)) {
        mix(0, n);
    } else {
        mix(0, 1024);
        mix(n - 1024, 1024);
        for (size_t k = 1; k < 256; ++k) mix(n / 256 * k, 64);
    }
    return h ^ n;
}

// A 64-bit hash of every byte of the view (verify mode): 8-byte words mixed by multiply-xor, a few
// GB/s on one core.
static uint64_t full_hash(const uint8_t *p, size_t n) {
    uint64_t h = 0x9E3779B97F4A7C15ull ^ n;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t v;
        memcpy(&v, p + i, 8);
        h = (h ^ v) * 0xFF51AFD7ED558CCDull;
        h ^= h >> 29;
    }
    for (; i < n; ++i) h = (h ^ p[i]) * 0x100000001B3ull;
    return h ^ (h >> 32);
}

// Frees entries (least recent first) until the cache fits its limit; entries in use are
// unlinked and freed by their last user. Caller holds the lock.
static void evict_locked(WeightCache &c, std::vector<jk_weight *> &to_free) {
    auto it = c.lru.end();
    while (c.bytes > c.limit && it != c.lru.begin()) {
        --it;
        std::shared_ptr<CacheEntry> e = *it;
        c.map.erase(e->key);
        c.bytes -= e->bytes;
        e->evicted = true;
        g_evictions.fetch_add(1);
        if (e->users == 0) to_free.push_back(e->w), e->w = nullptr;
        it = c.lru.erase(it);
    }
}

static void free_all(std::vector<jk_weight *> &ws) {
    for (jk_weight *w : ws) (void)jk_weight_free(w);
    ws.clear();
}

// A resident weight for one call: the cached handle (released when the call ends), or, with
// the cache off, a handle of its own freed at the end.
struct ResidentWeight {
    std::shared_ptr<CacheEntry> entry;
    jk_weight *own = nullptr;
    const jk_weight *w = nullptr;
    ~ResidentWeight() {
        if (own) (void)jk_weight_free(own);
        if (entry) {
            jk_weight *drop = nullptr;
            {
                std::lock_guard<std::mutex> lock(cache().mu);
                if (--entry->users == 0 && entry->evicted) drop = entry->w, entry->w = nullptr;
            }
            if (drop) (void)jk_weight_free(drop);
        }
    }
};

// The device copy of view v as a [rows, cols] matrix (validated by the caller).
static jk_status resident(HostCtx *ctx, const jk_tensor_view *v, size_t rows, size_t cols, ResidentWeight *out) {
    WeightCache &c = cache();
    CacheKey key{ctx->device, v->bytes, v->byte_len, v->quant, rows, cols,
                 fingerprint(static_cast<const uint8_t *>(v->bytes), v->byte_len)};
    size_t limit;
    {
        std::lock_guard<std::mutex> lock(c.mu);
        limit = c.limit;
    }
    const bool verify = limit > 0 && g_verify.load();
    const uint64_t full = verify ? full_hash(static_cast<const uint8_t *>(v->bytes), v->byte_len) : 0;
    if (limit > 0) {
        std::vector<jk_weight *> stale;
        {
            std::lock_guard<std::mutex> lock(c.mu);
            auto it = c.map.find(key);
            if (it != c.map.end()) {
                std::shared_ptr<CacheEntry> e = *it->second;
                if (!verify || e->full == full) {
                    c.lru.splice(c.lru.begin(), c.lru, it->second);
                    ++e->users;
                    g_hits.fetch_add(1);
                    out->entry = e;
                    out->w = e->w;
                    return JK_OK;
                }
                // the bytes changed since the upload: drop the entry, upload again below
                c.map.erase(it);
                c.lru.remove(e);
                c.bytes -= e->bytes;
                e->evicted = true;
                g_stale.fetch_add(1);
                if (e->users == 0) stale.push_back(e->w), e->w = nullptr;
            }
        }
        free_all(stale);
    }
    jk_weight *w = nullptr;
    JK_TRY(jk_weight_upload(ctx->stream, v, rows, cols, &w));
    g_uploads.fetch_add(1);
    g_device_allocs.fetch_add(2);  // the handle and its transient staging buffer
    if (limit == 0 || w->device_bytes > limit) {
        out->own = w;
        out->w = w;
        return JK_OK;
    }
    std::vector<jk_weight *> to_free;
    {
        std::lock_guard<std::mutex> lock(c.mu);
        auto it = c.map.find(key);
        if (it != c.map.end()) {  // another thread uploaded the same view meanwhile
            std::shared_ptr<CacheEntry> e = *it->second;
            ++e->users;
            out->entry = e;
            out->w = e->w;
            to_free.push_back(w);
        } else {
            auto e = std::make_shared<CacheEntry>();
            e->key = key;
            e->w = w;
            e->bytes = w->device_bytes;
            e->full = full;
            e->users = 1;
            c.lru.push_front(e);
            c.map[key] = c.lru.begin();
            c.bytes += e->bytes;
            out->entry = e;
            out->w = w;
            evict_locked(c, to_free);
        }
    }
    free_all(to_free);
    return JK_OK;
}

// ------------------------------------------------------------------ shared call bodies
static jk_status host_gemv(int quant, float *out, size_t out_len, const jk_tensor_view *w, const void *x, size_t nx,
                           size_t xblock_bytes, const char *name) {
    const Fmt f = fmt_of(quant);
    size_t rows, cols;
    JK_TRY(validate_matvec(w, quant, out_len, nx * (size_t)f.be, &rows, &cols));
    if (nx != cols / (size_t)f.be)  // check_q8_block_len (quant_q8.rs:1562-1578)
        return fail_tb(Tb{tb_view(w).name, w->offset, nx, cols / (size_t)f.be}, "%s: x_blocks len %zu != expected %zu",
                       name, nx, cols / (size_t)f.be);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "%s: null pointer", name);
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    ResidentWeight rw;
    JK_TRY(resident(ctx, w, rows, cols, &rw));
    Scratch sc{ctx};
    JK_TRY(sc.take({nx * xblock_bytes, rows * sizeof(float)}));
    JK_TRY(h2d(ctx, sc.p[0], x, nx * xblock_bytes));
    JK_TRY(launch_gemv_q8(ctx->stream, rw.w->dev, sc.p[0], (float *)sc.p[1], 0, (int)rows));
    return d2h_sync(ctx, out, sc.p[1], rows * sizeof(float));
}

// validate_q8_block_row_bytes (quant_q8.rs:644-664) then the single-row driver: a 1-row
// matrix, whose only row is a tail row of run_4row_chunked_gemv and so sums like `.sum()`.
static jk_status host_vec_dot_row(int quant, const void *wb, size_t w_len, const void *x, size_t nx, float *out,
                                  size_t xblock_bytes, const char *name) {
    const Fmt f = fmt_of(quant);
    if (nx == 0 || w_len != nx * (size_t)f.bb)
        return fail_tb(Tb{name, 0, w_len, nx * (size_t)f.bb}, "%s: expected %zu weight bytes for %zu blocks, got %zu",
                       name, nx * (size_t)f.bb, nx, w_len);
    if (!wb || !x || !out) return fail(JK_TENSOR_BOUNDS, "%s: null pointer", name);
    size_t shape[2] = {1, nx * (size_t)f.be};
    jk_tensor_view v = {name, quant, shape, 2, wb, w_len, 0};
    return host_gemv(quant, out, 1, &v, x, nx, xblock_bytes, name);
}

static jk_status host_vec_dot_f32(int quant, float *out, size_t out_len, const jk_tensor_view *w, const float *in,
                                  size_t in_len) {
    size_t rows, cols;
    JK_TRY(validate_matvec(w, quant, out_len, in_len, &rows, &cols));
    if (!in || !out) return fail(JK_TENSOR_BOUNDS, "vec_dot: null pointer");
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    ResidentWeight rw;
    JK_TRY(resident(ctx, w, rows, cols, &rw));
    Scratch sc{ctx};
    JK_TRY(sc.take({cols * sizeof(float), rows * sizeof(float)}));
    JK_TRY(h2d(ctx, sc.p[0], in, cols * sizeof(float)));
    JK_TRY(launch_vec_dot_f32(ctx->stream, rw.w->dev, (const float *)sc.p[0], (float *)sc.p[1]));
    return d2h_sync(ctx, out, sc.p[1], rows * sizeof(float));
}

}  // namespace jk

using namespace jk;

extern "C" {

// ------------------------------------------------------------------ cache control
jk_status jk_host_cache_set_limit(size_t bytes) {
    std::vector<jk_weight *> to_free;
    {
        std::lock_guard<std::mutex> lock(cache().mu);
        cache().limit = bytes;
        evict_locked(cache(), to_free);
    }
    free_all(to_free);
    return JK_OK;
}

jk_status jk_host_cache_invalidate(const void *bytes, size_t len) {
    WeightCache &c = cache();
    std::vector<jk_weight *> to_free;
    {
        std::lock_guard<std::mutex> lock(c.mu);
        const uintptr_t lo = (uintptr_t)bytes, hi = lo + len;
        for (auto it = c.lru.begin(); it != c.lru.end();) {
            std::shared_ptr<CacheEntry> e = *it;
            const uintptr_t a = (uintptr_t)e->key.ptr, b = a + e->key.len;
            if (a < hi && lo < b) {  // the ranges overlap
                c.map.erase(e->key);
                c.bytes -= e->bytes;
                e->evicted = true;
                if (e->users == 0) to_free.push_back(e->w), e->w = nullptr;
                it = c.lru.erase(it);
            } else {
                ++it;
            }
        }
    }
    free_all(to_free);
    return JK_OK;
}

jk_status jk_host_cache_clear(void) { return jk_host_cache_invalidate(nullptr, SIZE_MAX); }

jk_status jk_host_cache_set_verify(int on) {
    // entries uploaded before verify mode have no full hash: start over
    g_verify.store(on != 0);
    return jk_host_cache_clear();
}

jk_status jk_host_get_stats(jk_host_stats *out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "host_get_stats: null pointer");
    std::lock_guard<std::mutex> lock(cache().mu);
    out->weight_uploads = g_uploads.load();
    out->cache_hits = g_hits.load();
    out->cache_evictions = g_evictions.load();
    out->device_allocs = g_device_allocs.load();
    out->cached_weights = cache().lru.size();
    out->cached_bytes = cache().bytes;
    out->cache_limit = cache().limit;
    out->stale_reuploads = g_stale.load();
    out->verify = g_verify.load() ? 1 : 0;
    return JK_OK;
}

jk_status jk_host_release_thread(void) {
    if (!t_ctx) return JK_OK;
    HostCtx *c = t_ctx;
    t_ctx = nullptr;
    int cur = 0;
    JK_HIP(hipGetDevice(&cur));
    JK_HIP(hipSetDevice(c->device));
    hipError_t e = hipStreamSynchronize(c->stream);
    if (c->scratch) {
        const hipError_t f = hipFree(c->scratch);
        if (e == hipSuccess) e = f;
    }
    const hipError_t d = hipStreamDestroy(c->stream);
    if (e == hipSuccess) e = d;
    delete c;
    (void)hipSetDevice(cur);
    if (e != hipSuccess) return hip_fail(e, "jk_host_release_thread");
    return JK_OK;
}

// ------------------------------------------------------------------ quantizers
jk_status jk_host_quantize_row_q8_0(const float *x, size_t n, jk_block_q8_0 *out, size_t out_len) {
    if (n == 0 || n % 32)
        return fail_tb(Tb{"quantize_row_q8_0_f32", 0, n * 4, out_len},
                       "quantize_row_q8_0_f32: input length %zu must be a positive multiple of 32", n);
    if (out_len != n / 32)
        return fail_tb(Tb{"quantize_row_q8_0_f32", 0, n * 4, out_len},
                       "quantize_row_q8_0_f32: output block count %zu != expected %zu", out_len, n / 32);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_0: null pointer");
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({n * sizeof(float), out_len * sizeof(jk_block_q8_0)}));
    JK_TRY(h2d(ctx, sc.p[0], x, n * sizeof(float)));
    JK_TRY(launch_quantize_q8_0(ctx->stream, (const float *)sc.p[0], out_len, (jk_block_q8_0 *)sc.p[1]));
    return d2h_sync(ctx, out, sc.p[1], out_len * sizeof(jk_block_q8_0));
}

jk_status jk_host_quantize_row_q8_k(const float *x, size_t n, jk_block_q8k *out, size_t out_len) {
    if (n == 0 || n % 256)
        return fail_tb(Tb{"quantize_row_q8_k", 0, n * 4, out_len},
                       "quantize_row_q8_k: input length %zu must be a positive multiple of 256", n);
    if (out_len != n / 256)
        return fail_tb(Tb{"quantize_row_q8_k", 0, n * 4, out_len},
                       "quantize_row_q8_k: output block count %zu != expected %zu", out_len, n / 256);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: null pointer");
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({n * sizeof(float), out_len * sizeof(jk_block_q8k)}));
    JK_TRY(h2d(ctx, sc.p[0], x, n * sizeof(float)));
    JK_TRY(launch_quantize_q8_k(ctx->stream, (const float *)sc.p[0], out_len, (jk_block_q8k *)sc.p[1]));
    return d2h_sync(ctx, out, sc.p[1], out_len * sizeof(jk_block_q8k));
}

// ------------------------------------------------------------------ single-row dots
jk_status jk_host_vec_dot_q4_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q4_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0), "vec_dot_q4_0_q8_0");
}
jk_status jk_host_vec_dot_q8_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q8_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0), "vec_dot_q8_0_q8_0");
}
jk_status jk_host_vec_dot_q4_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q4_K, w, w_len, x, nx, out, sizeof(jk_block_q8k), "vec_dot_q4_k_q8_k");
}
jk_status jk_host_vec_dot_q6_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q6_K, w, w_len, x, nx, out, sizeof(jk_block_q8k), "vec_dot_q6_k_q8_k");
}
jk_status jk_host_vec_dot_tq2_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_TQ2_0, w, w_len, x, nx, out, sizeof(jk_block_q8k), "vec_dot_tq2_0_q8_k");
}
jk_status jk_host_vec_dot_q5_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q5_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0), "vec_dot_q5_0_q8_0_blocks");
}
jk_status jk_host_vec_dot_q5_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q5_K, w, w_len, x, nx, out, sizeof(jk_block_q8k), "vec_dot_q5_k_q8_k");
}
jk_status jk_host_vec_dot_tq1_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_TQ1_0, w, w_len, x, nx, out, sizeof(jk_block_q8k), "vec_dot_tq1_0_q8_k");
}

// ------------------------------------------------------------------ M=1 GEMV
jk_status jk_host_gemv_q4_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q4_0, out, n, w, x, nx, sizeof(jk_block_q8_0), "gemv_q4_0_q8_0");
}
jk_status jk_host_gemv_q8_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q8_0, out, n, w, x, nx, sizeof(jk_block_q8_0), "gemv_q8_0_q8_0");
}
jk_status jk_host_gemv_q4_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q4_K, out, n, w, x, nx, sizeof(jk_block_q8k), "gemv_q4_k_q8_k");
}
jk_status jk_host_gemv_q6_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q6_K, out, n, w, x, nx, sizeof(jk_block_q8k), "gemv_q6_k_q8_k");
}
jk_status jk_host_gemv_tq2_0_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_TQ2_0, out, n, w, x, nx, sizeof(jk_block_q8k), "gemv_tq2_0_q8_k");
}
jk_status jk_host_gemv_q5_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q5_0, out, n, w, x, nx, sizeof(jk_block_q8_0), "gemv_q5_0_q8_0");
}
jk_status jk_host_gemv_q5_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q5_K, out, n, w, x, nx, sizeof(jk_block_q8k), "gemv_q5_k_q8_k");
}
jk_status jk_host_gemv_tq1_0_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_TQ1_0, out, n, w, x, nx, sizeof(jk_block_q8k), "gemv_tq1_0_q8_k");
}

// ------------------------------------------------------------------ f32-activation matvec
jk_status jk_host_vec_dot_q4_0(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q4_0, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q8_0(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q8_0, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q6_k(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q6_K, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q4_k_m(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q4_K, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_i2_s(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_I2_S, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q5_0(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q5_0, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q5_k(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q5_K, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q4_1(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q4_1, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q5_1(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q5_1, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q2_k(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q2_K, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_q3_k(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_Q3_K, out, n, w, in, in_len);
}
jk_status jk_host_vec_dot_iq4_nl(float *out, size_t n, const jk_tensor_view *w, const float *in, size_t in_len) {
    return host_vec_dot_f32(JK_IQ4_NL, out, n, w, in, in_len);
}

// dequantize_tensor_row (quant.rs:2492-2568) with validate_token_row_geometry (1749-1808): the
// whole tensor is made resident as [nrows, cols] (an embedding table is looked up row by row).
jk_status jk_host_dequantize_tensor_row(const jk_tensor_view *w, size_t row, float *out, size_t out_len) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape)) return fail(JK_TENSOR_BOUNDS, "null tensor view");
    if (!fmt_known(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "dequantize_tensor_row: quant type %d is not supported", (int)w->quant);
    const Tb t = tb_view(w);
    const size_t cols = out_len;
    if (cols == 0) return fail_tb(t, "%s: dequantize_token_row output slice cannot be empty", t.name);
    size_t total = 0;
    if (w->ndim) {
        total = 1;
        for (size_t i = 0; i < w->ndim; i++) total *= w->shape[i];
    }
    if (total == 0 || total % cols)
        return fail_tb(t, "%s: tensor element count %zu is not a positive multiple of row width %zu", t.name, total,
                       cols);
    const size_t nrows = total / cols;
    if (w->ndim == 2 && !((w->shape[0] == cols && w->shape[1] == nrows) || (w->shape[1] == cols && w->shape[0] == nrows)))
        return fail_tb(t, "%s: tensor shape does not match row width %zu and row count %zu", t.name, cols, nrows);
    if (row >= nrows) return fail_tb(t, "%s: row index %zu out of bounds for %zu rows", t.name, row, nrows);
    const Fmt f = fmt_of(w->quant);
    if (cols % (size_t)f.be) return fail_tb(t, "%s: row width %zu is not a multiple of %d", t.name, cols, f.be);
    const size_t row_bytes = cols / (size_t)f.be * (size_t)f.bb, payload = nrows * row_bytes;
    if (w->byte_len < payload + trailer_bytes(w->quant))
        return fail_tb(t, "%s: buffer length %zu < required %zu", t.name, w->byte_len,
                       payload + trailer_bytes(w->quant));
    if (!out) return fail(JK_TENSOR_BOUNDS, "null output");
    if (nrows >= ((size_t)1 << 30) || cols / (size_t)f.be >= ((size_t)1 << 30))
        return fail_tb(t, "%s: [%zu, %zu] exceeds the device index range", t.name, nrows, cols);
    size_t shape[2] = {nrows, cols};
    jk_tensor_view v = {w->name, w->quant, shape, 2, w->bytes, w->byte_len, w->offset};
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    ResidentWeight rw;
    JK_TRY(resident(ctx, &v, nrows, cols, &rw));
    Scratch sc{ctx};
    JK_TRY(sc.take({cols * sizeof(float)}));
    JK_TRY(launch_dequant_rows(ctx->stream, rw.w->dev, (int)row, (int)row + 1, (float *)sc.p[0]));
    return d2h_sync(ctx, out, sc.p[0], cols * sizeof(float));
}

jk_status jk_host_gemm_repacked_f32(float *out, size_t out_len, const jk_weight *w, const float *input, size_t m,
                                   size_t r0, size_t r1) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "gemm_repacked_f32: null weight handle");
    if (!w->ready) return fail(JK_TENSOR_BOUNDS, "gemm_repacked_f32: the weight has not been sealed (jk_weight_seal)");
    const size_t cols = (size_t)w->dev.cols;
    if (m == 0 || !input)
        return fail_tb(Tb{"gemm_repacked_f32", 0, m * cols * 4, 0},
                       "gemm_repacked_f32: input must hold m * cols = %zu * %zu values", m, cols);
    if (r0 > r1 || r1 > (size_t)w->dev.rows)
        return fail_tb(Tb{"gemm_repacked", r0, r1 >= r0 ? r1 - r0 : 0, (size_t)w->dev.rows},
                       "gemm_repacked: invalid row_range %zu..%zu for weight rows %d", r0, r1, w->dev.rows);
    if (out_len != m * (r1 - r0))
        return fail_tb(Tb{"gemm_repacked", 0, out_len * 4, m * (r1 - r0) * 4},
                       "gemm_repacked: output length %zu != m (%zu) * sub_rows (%zu)", out_len, m, r1 - r0);
    if (r0 == r1) return JK_OK;
    if (!out) return fail(JK_TENSOR_BOUNDS, "null output");
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    const size_t act_bytes = jk_act_q8_bytes(m, cols);
    Scratch sc{ctx};
    JK_TRY(sc.take({m * cols * sizeof(float), act_bytes, out_len * sizeof(float)}));
    JK_TRY(h2d(ctx, sc.p[0], input, m * cols * sizeof(float)));
    jk_act_q8 act;
    JK_TRY(jk_act_q8_bind(sc.p[1], act_bytes, m, cols, &act));
    JK_TRY(launch_quantize_act_q8(ctx->stream, (const float *)sc.p[0], act));
    JK_TRY(launch_gemm_repacked(ctx->stream, w->dev, act, (float *)sc.p[2], (int)r0, (int)r1));
    return d2h_sync(ctx, out, sc.p[2], out_len * sizeof(float));
}

// swiglu_f32 (swiglu.rs:62) / relu_squared_gate_f32 (lib.rs:1111) on host slices, with the
// reference's length check (validate_gated_activation_args, swiglu.rs:33-52).
static jk_status host_gated(int act, float *out, size_t out_len, const float *gate, size_t gate_len, const float *up,
                            size_t up_len) {
    if (gate_len == 0 || out_len != gate_len || up_len != gate_len)
        return fail_tb(Tb{act == JK_ACT_SWIGLU ? "swiglu" : "relu_squared_gate", 0, gate_len, out_len},
                       "dimension mismatch: gate=%zu, up=%zu, out=%zu", gate_len, up_len, out_len);
    if (!out || !gate || !up) return fail(JK_TENSOR_BOUNDS, "null pointer");
    const size_t b = gate_len * sizeof(float);
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({b, b, b}));
    JK_TRY(h2d(ctx, sc.p[0], gate, b));
    JK_TRY(h2d(ctx, sc.p[1], up, b));
    JK_TRY(launch_gated(ctx->stream, act, (const float *)sc.p[0], (const float *)sc.p[1], gate_len, (float *)sc.p[2]));
    return d2h_sync(ctx, out, sc.p[2], b);
}

jk_status jk_host_swiglu_f32(float *out, size_t out_len, const float *gate, size_t gate_len, const float *up,
                             size_t up_len) {
    return host_gated(JK_ACT_SWIGLU, out, out_len, gate, gate_len, up, up_len);
}

jk_status jk_host_relu_squared_gate_f32(float *out, size_t out_len, const float *gate, size_t gate_len,
                                        const float *up, size_t up_len) {
    return host_gated(JK_ACT_RELU2, out, out_len, gate, gate_len, up, up_len);
}

// argmax_f32 (lib.rs:662): *index = -1 for None.
jk_status jk_host_argmax_f32(const float *x, size_t n, int64_t *index) {
    if (!index || (n && !x)) return fail(JK_TENSOR_BOUNDS, "argmax: null pointer");
    if (n > (size_t)INT32_MAX) return fail(JK_TENSOR_BOUNDS, "argmax: %zu values exceed the int32 index range", n);
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({n * sizeof(float), argmax_ws_bytes(n), sizeof(int32_t)}));
    JK_TRY(h2d(ctx, sc.p[0], x, n * sizeof(float)));
    JK_TRY(launch_argmax(ctx->stream, (const float *)sc.p[0], n, (int32_t *)sc.p[2], sc.p[1]));
    int32_t idx = -1;
    JK_TRY(d2h_sync(ctx, &idx, sc.p[2], sizeof idx));
    *index = idx;
    return JK_OK;
}

// gemm_i8_vector (ime.rs:563-583) on host slices: c[row][n - n0]. Only A's m x k bytes and B's rows
// n0..n1 cross PCIe.
jk_status jk_host_gemm_i8(const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0,
                          size_t n1, size_t k, int32_t *c, size_t c_len) {
    clear_error();
    JK_TRY(gemm_i8_check(a, a_len, m, b, b_len, n0, n1, k, c, c_len));
    if (m == 0 || n1 == n0) return JK_OK;
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    const size_t na = m * k, nb = (n1 - n0) * k;
    JK_TRY(sc.take({na, nb, c_len * sizeof(int32_t)}));
    JK_TRY(h2d(ctx, sc.p[0], a, na));
    JK_TRY(h2d(ctx, sc.p[1], b + n0 * k, nb));
    JK_TRY(jk_gemm_i8(ctx->stream, (const int8_t *)sc.p[0], na, m, (const int8_t *)sc.p[1], nb, 0, n1 - n0, k,
                      (int32_t *)sc.p[2], c_len));
    return d2h_sync(ctx, c, sc.p[2], c_len * sizeof(int32_t));
}

// dot_i8_vector (ime.rs:548-557) on host slices, over the zip of the two.
jk_status jk_host_dot_i8(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, int32_t *out) {
    clear_error();
    JK_TRY(dot_i8_check(a, a_len, b, b_len, out));
    const size_t k = a_len < b_len ? a_len : b_len;
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({k, k, sizeof(int32_t)}));
    JK_TRY(h2d(ctx, sc.p[0], a, k));
    JK_TRY(h2d(ctx, sc.p[1], b, k));
    JK_TRY(jk_dot_i8(ctx->stream, (const int8_t *)sc.p[0], k, (const int8_t *)sc.p[1], k, (int32_t *)sc.p[2]));
    return d2h_sync(ctx, out, sc.p[2], sizeof(int32_t));
}

// convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790): two 32-byte I2_S blocks and an f16 scale -> one
// 66-byte TQ2_0 block.
jk_status jk_host_convert_i2_s_blocks_to_tq2_0(const uint8_t *blk0, const uint8_t *blk1, uint16_t scale_f16_bits,
                                               uint8_t *out) {
    if (!blk0 || !blk1 || !out) return fail(JK_TENSOR_BOUNDS, "convert_i2_s_blocks_to_tq2_0: null pointer");
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    Scratch sc{ctx};
    JK_TRY(sc.take({64, 66}));
    JK_TRY(h2d(ctx, sc.p[0], blk0, 32));
    JK_TRY(h2d(ctx, static_cast<uint8_t *>(sc.p[0]) + 32, blk1, 32));
    JK_TRY(launch_i2s_to_tq2(ctx->stream, static_cast<const uint8_t *>(sc.p[0]), 1, scale_f16_bits,
                             static_cast<uint8_t *>(sc.p[1])));
    return d2h_sync(ctx, out, sc.p[1], 66);
}

// bitlinear_i8_rvv (ime.rs:882-938) with validate_bitlinear_dimensions (660-763).
jk_status jk_host_bitlinear_i8(float *out, size_t out_len, const jk_tensor_view *w, const int8_t *act, size_t act_len,
                               float act_scale) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape)) return fail(JK_TENSOR_BOUNDS, "null tensor view");
    const Tb t = tb_view(w);
    const int q = w->quant;
    if (!has_bitlinear(q)) return fail_tb(t, "%s: BitLinear: unsupported quant type %d", t.name, q);
    if (w->ndim == 0) return fail_tb(t, "%s: empty tensor shape", t.name);
    const Fmt f = fmt_of(q);
    if (w->ndim == 2) {
        const size_t d0 = w->shape[0], d1 = w->shape[1];
        if (!((out_len == d0 && act_len == d1 && d1 % (size_t)f.be == 0) ||
              (out_len == d1 && act_len == d0 && d0 % (size_t)f.be == 0)))
            return fail_tb(t, "%s: BitLinear: shape [%zu, %zu] does not match out %zu / act %zu", t.name, d0, d1,
                           out_len, act_len);
    } else {
        size_t total = 1;
        for (size_t i = 0; i < w->ndim; i++) total *= w->shape[i];
        if (act_len == 0 || out_len == 0 || act_len % (size_t)f.be || out_len * act_len != total)
            return fail_tb(t, "%s: BitLinear: tensor elements %zu do not match %zu * %zu", t.name, total, out_len,
                           act_len);
    }
    const size_t need = out_len * act_len / (size_t)f.be * (size_t)f.bb + trailer_bytes(q);
    if (w->byte_len < need)
        return fail_tb(t, "%s: BitLinear: buffer length %zu < required %zu", t.name, w->byte_len, need);
    if (!act || !out) return fail(JK_TENSOR_BOUNDS, "BitLinear: null pointer");
    // The matrix is read as [out_len, act_len] row-major blocks; an explicit [rows, cols]
    // view of the same bytes keeps the orientation the validator accepted.
    size_t shape[2] = {out_len, act_len};
    jk_tensor_view v = {w->name, q, shape, 2, w->bytes, w->byte_len, w->offset};
    HostCtx *ctx;
    JK_TRY(ctx_get(&ctx));
    ResidentWeight rw;
    JK_TRY(resident(ctx, &v, out_len, act_len, &rw));
    Scratch sc{ctx};
    JK_TRY(sc.take({act_len, sizeof(float), out_len * sizeof(float)}));
    JK_TRY(h2d(ctx, sc.p[0], act, act_len));
    JK_TRY(h2d(ctx, sc.p[1], &act_scale, sizeof(float)));
    JK_TRY(launch_bitlinear(ctx->stream, rw.w->dev, (const int8_t *)sc.p[0], (const float *)sc.p[1], 1,
                            (float *)sc.p[2]));
    count_vector_dots((uint64_t)out_len * (uint64_t)(act_len / fmt_of(q).be));  // as bitlinear_i8_rvv (ime.rs:919-936)
    return d2h_sync(ctx, out, sc.p[2], out_len * sizeof(float));
}

}  // extern "C"
