// jk_runtime.hip -- device-tier C ABI of libjk: errors, streams, weight handles,
// activation buffers and the argument validation of every entry point.
//
// Validation mirrors the reference validators cited at each entry and always runs
// before any device work is enqueued (fail closed).
#include <limits.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "jk_internal.hpp"

namespace jk {

// The most recent failure on this thread: K3Error's payload (TensorBoundsError's tensor_name,
// offset, byte_len, buffer_len and reason; the reason alone for the other kinds).
struct ErrInfo {
    jk_status status = JK_OK;
    std::string name, reason;
    size_t offset = 0, byte_len = 0, buffer_len = 0;
};
static thread_local ErrInfo g_err;

static jk_status set_error(jk_status st, const char *name, size_t off, size_t bl, size_t buf, const char *fmt,
                           va_list ap) {
    char msg[512];
    vsnprintf(msg, sizeof msg, fmt, ap);
    g_err.status = st;
    g_err.reason = msg;
    g_err.offset = off;
    g_err.byte_len = bl;
    g_err.buffer_len = buf;
    if (name) {
        g_err.name = name;
    } else {
        // messages name their tensor or operation first ("name: reason")
        const char *colon = strstr(msg, ": ");
        g_err.name = colon && !memchr(msg, ' ', (size_t)(colon - msg)) ? std::string(msg, (size_t)(colon - msg)) : "";
    }
    return st;
}

jk_status fail(jk_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    set_error(st, nullptr, 0, 0, 0, fmt, ap);
    va_end(ap);
    return st;
}

jk_status fail_tb(const Tb &t, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    set_error(JK_TENSOR_BOUNDS, t.name ? t.name : "", t.offset, t.byte_len, t.buffer_len, fmt, ap);
    va_end(ap);
    return JK_TENSOR_BOUNDS;
}

Tb tb_view(const jk_tensor_view *w) {
    return Tb{w->name ? w->name : "<tensor>", w->offset, w->byte_len, w->byte_len};
}

jk_status hip_fail(hipError_t e, const char *what) {
    return fail(JK_DEVICE_ERROR, "%s failed: %s", what, hipGetErrorString(e));
}

void clear_error() { g_err = ErrInfo(); }

thread_local LaunchPlan t_plan;

jk_status check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return JK_OK;
}

static const char *quant_name(int q) {
    switch (q) {
    case JK_Q4_0: return "Q4_0";
    case JK_Q4_1: return "Q4_1";
    case JK_Q5_0: return "Q5_0";
    case JK_Q5_1: return "Q5_1";
    case JK_IQ4_NL: return "IQ4_NL";
    case JK_Q2_K: return "Q2_K";
    case JK_Q3_K: return "Q3_K";
    case JK_Q8_0: return "Q8_0";
    case JK_Q4_K: return "Q4_K_M";
    case JK_Q5_K: return "Q5_K";
    case JK_Q6_K: return "Q6_K";
    case JK_TQ1_0: return "TQ1_0";
    case JK_TQ2_0: return "TQ2_0";
    case JK_I2_S: return "I2_S";
    default: return "unsupported";
    }
}

static size_t num_elements(const jk_tensor_view *w) {
    if (w->ndim == 0) return 0;
    size_t n = 1;
    for (size_t i = 0; i < w->ndim; i++) n *= w->shape[i];
    return n;
}

static const char *tname(const jk_tensor_view *w) { return w->name ? w->name : "<tensor>"; }

// Orientation and byte-length rule of validate_quant_matvec_dimensions (quant.rs:1810-1894),
// validate_q4_0/q8_0/q6_k_dimensions (quant.rs:762-892, 1315-1394) and
// validate_q4_k_m_dimensions (lib.rs:1195-1260). A quant mismatch is a TensorBoundsError
// there. The byte-length check is applied to every format (the Q8_0/Q6_K/Q4_K validators
// rely on a slice bound that panics instead).
jk_status validate_matvec(const jk_tensor_view *w, int quant, size_t out_len, size_t in_len,
                          size_t *rows, size_t *cols) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape))
        return fail(JK_TENSOR_BOUNDS, "null tensor view");
    if (w->quant != quant)
        return fail_tb(tb_view(w), "%s: expected %s quant type, got %s", tname(w),
                    quant_name(quant), quant_name(w->quant));
    if (w->ndim == 0) return fail_tb(tb_view(w), "%s: empty tensor shape", tname(w));
    const Fmt f = fmt_of(quant);
    if (w->ndim == 2) {
        size_t d0 = w->shape[0], d1 = w->shape[1];
        if (out_len == d0 && in_len == d1 && d1 % f.be == 0) { *rows = d0; *cols = d1; }
        else if (out_len == d1 && in_len == d0 && d0 % f.be == 0) { *rows = d1; *cols = d0; }
        else
            return fail_tb(tb_view(w),
                        "%s: matrix shape [%zu, %zu] does not match output len %zu and %s-aligned input len %zu",
                        tname(w), d0, d1, out_len, quant_name(quant), in_len);
    } else {
        size_t total = num_elements(w);
        if (in_len == 0 || out_len == 0 || in_len % f.be || out_len * in_len != total)
            return fail_tb(tb_view(w), "%s: tensor elements %zu do not match output len %zu * input len %zu",
                        tname(w), total, out_len, in_len);
        *rows = out_len;
        *cols = in_len;
    }
    if (*rows == 0 || *cols == 0)
        return fail_tb(tb_view(w), "%s: empty matrix [%zu, %zu]", tname(w), *rows, *cols);
    size_t need = (*rows * *cols / f.be) * f.bb + trailer_bytes(quant);
    if (w->byte_len < need)
        return fail_tb(tb_view(w), "%s: %s buffer length %zu < required %zu", tname(w),
                    quant_name(quant), w->byte_len, need);
    return JK_OK;
}

// validate_matrix_view (repack.rs:1208-1281) with validate_matrix_shape (1172-1206).
static jk_status validate_matrix_view(const jk_tensor_view *w, size_t rows, size_t cols) {
    if (rows == 0 || cols == 0)
        return fail_tb(tb_view(w), "%s: repack dimensions must be non-zero, got [%zu, %zu]", tname(w), rows, cols);
    const Fmt f = fmt_of(w->quant);
    if (cols % f.be)
        return fail_tb(tb_view(w), "%s: cols %zu not a multiple of block size %d", tname(w), cols, f.be);
    if (w->ndim == 1) {
        if (rows * cols != w->shape[0])
            return fail_tb(tb_view(w), "%s: 1D shape %zu != rows * cols %zu", tname(w), w->shape[0], rows * cols);
    } else if (w->ndim == 2) {
        size_t d0 = w->shape[0], d1 = w->shape[1];
        if (!((d0 == rows && d1 == cols) || (d0 == cols && d1 == rows)))
            return fail_tb(tb_view(w), "%s: shape [%zu, %zu] does not match [%zu, %zu]", tname(w), d0, d1, rows, cols);
    } else {
        return fail_tb(tb_view(w), "%s: expected 1D or 2D weight tensor, got %zuD", tname(w), w->ndim);
    }
    size_t need = rows * (cols / f.be) * f.bb + trailer_bytes(w->quant);
    if (w->byte_len < need)
        return fail_tb(tb_view(w), "%s: buffer length %zu < required %zu", tname(w), w->byte_len, need);
    return JK_OK;
}

static float read_trailer_scale(const uint8_t *t, size_t len) {
    if (len < 4) return 0.0f;
    float v;
    memcpy(&v, t, 4);
    return std::isfinite(v) ? v : 0.0f;  // read_i2_s_trailer_scale, quant.rs:360-366
}

// Device weight limits: row and block indices are 32-bit inside the kernels.
static const size_t kMaxRows = (size_t)1 << 30;

// Compute entry points accept only a complete (sealed) handle.
static jk_status weight_usable(const jk_weight *w, const char *what) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "%s: null weight handle", what);
    if (!w->ready) return fail(JK_TENSOR_BOUNDS, "%s: the weight has not been sealed (jk_weight_seal)", what);
    return JK_OK;
}

// Validation of a GEMV whose argmax is fused into its store phase (gemv_* followed by
// argmax_f32, quant_q8.rs:1586-3273 and lib.rs:662): the job over all rows of w, with the
// argmax slots still to be filled in by the caller.
jk_status gemv_argmax_job(const char *what, const jk_weight *w, const void *x_q8, const float *x_f32, size_t x_len,
                          float *y, int32_t *index, GemvJob *out) {
    JK_TRY(weight_usable(w, what));
    if (!has_q8_gemv(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "%s: %s has no quant_q8 GEMV", what, quant_name(w->quant));
    if ((x_q8 == nullptr) == (x_f32 == nullptr))
        return fail(JK_TENSOR_BOUNDS, "%s: exactly one of x_q8 and x_f32 must be set", what);
    if (x_q8 ? x_len != (size_t)w->dev.nb : x_len != (size_t)w->dev.cols)
        return fail(JK_TENSOR_BOUNDS, "%s: activation length %zu does not match the weight", what, x_len);
    if ((uintptr_t)x_q8 % 4 || (uintptr_t)x_f32 % 16)
        return fail(JK_TENSOR_BOUNDS, "%s: x_q8 must be 4-byte and x_f32 16-byte aligned", what);
    if (x_f32 && (size_t)w->dev.cols > gemv_f32_max_cols(w->dev.quant))
        return fail(JK_CAPABILITY_MISMATCH, "%s: f32 activations need K <= %zu, got %d", what,
                    gemv_f32_max_cols(w->dev.quant), w->dev.cols);
    if (!index) return fail(JK_TENSOR_BOUNDS, "%s: null pointer", what);
    memset(out, 0, sizeof *out);
    out->w = w->dev;
    out->xq = x_q8;
    out->xf = x_f32;
    out->y = y;
    out->am_index = index;
    out->r0 = 0;
    out->r1 = w->dev.rows;
    return JK_OK;
}

}  // namespace jk

using namespace jk;

extern "C" {

const char *jk_last_error(void) { return g_err.reason.c_str(); }

jk_status jk_last_error_info(jk_error_info *out) {
    if (!out) return JK_TENSOR_BOUNDS;
    out->status = g_err.status;
    out->tensor_name = g_err.name.c_str();
    out->offset = g_err.offset;
    out->byte_len = g_err.byte_len;
    out->buffer_len = g_err.buffer_len;
    out->reason = g_err.reason.c_str();
    return JK_OK;
}
int jk_abi_version(void) { return JK_ABI_VERSION; }

jk_status jk_init(int device) {
    JK_HIP(hipSetDevice(device));
    return noalloc_setup();
}

jk_status jk_stream_create(jk_stream *out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "null stream out-pointer");
    hipStream_t s;
    JK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = (jk_stream)s;
    return JK_OK;
}

jk_status jk_stream_destroy(jk_stream s) {
    if (s) JK_HIP(hipStreamDestroy((hipStream_t)s));
    return JK_OK;
}

jk_status jk_stream_sync(jk_stream s) {
    JK_HIP(hipStreamSynchronize((hipStream_t)s));
    return JK_OK;
}

jk_status jk_device_alloc(size_t bytes, void **out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "null out-pointer");
    *out = nullptr;
    if (bytes == 0) return JK_OK;
    JK_HIP(hipMalloc(out, bytes));
    return JK_OK;
}

jk_status jk_device_free(void *p) {
    if (p) JK_HIP(hipFree(p));
    return JK_OK;
}

jk_status jk_copy_to_device(jk_stream s, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return JK_OK;
    JK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s));
    return JK_OK;
}

jk_status jk_copy_to_host(jk_stream s, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return JK_OK;
    JK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s));
    return JK_OK;
}

// ------------------------------------------------------------------ weights
// Byte sizes of the device layout of a [rows, cols] weight in GGUF format quant.
struct PlaneSizes {
    size_t nb, payload, plane_bytes, dbytes, dpad, hbytes;
};
static PlaneSizes plane_sizes(int quant, size_t rows, size_t cols) {
    const Fmt f = fmt_of(quant);             // GGUF block geometry
    const Fmt fd = fmt_of(dev_quant(quant));  // device layout
    PlaneSizes p;
    p.nb = cols / f.be;
    p.payload = rows * p.nb * f.bb;
    p.plane_bytes = rows * p.nb * (size_t)fd.chunks * 16;
    p.dbytes = fd.d_off >= 0 ? rows * p.nb * 2 : 0;
    p.dpad = (p.dbytes + 255) / 256 * 256;  // keeps the word plane 256-byte aligned
    p.hbytes = fd.h_off >= 0 ? rows * p.nb * (size_t)fd.h_len : 0;
    return p;
}

// Checks a view and explicit dimensions as BlockScaledTileLayout::for_tensor does
// (repack.rs:1308-1333, validate_matrix_view 1208-1281), plus the kernels' index range.
static jk_status check_view_dims(const jk_tensor_view *w, size_t rows, size_t cols) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape)) return fail(JK_TENSOR_BOUNDS, "null tensor view");
    if (!fmt_known(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "%s: quant type %d is not supported by libjk", tname(w), (int)w->quant);
    JK_TRY(validate_matrix_view(w, rows, cols));
    const size_t be = (size_t)fmt_of(w->quant).be;
    if (rows >= kMaxRows || cols / be >= kMaxRows || rows * (cols / be) >= ((size_t)1 << 28))
        return fail(JK_TENSOR_BOUNDS, "%s: matrix [%zu, %zu] exceeds the device index range", tname(w), rows, cols);
    return JK_OK;
}

// A handle with its device allocation and plane pointers; the planes' contents are undefined.
static jk_status alloc_handle(int quant, size_t rows, size_t cols, float tensor_scale, jk_weight **out) {
    const PlaneSizes p = plane_sizes(quant, rows, cols);
    jk_weight *h = new jk_weight();
    hipError_t e = hipGetDevice(&h->device);
    if (e == hipSuccess) e = hipMalloc(&h->alloc, p.plane_bytes + p.dpad + p.hbytes + 256);
    if (e != hipSuccess) {
        delete h;
        return hip_fail(e, "weight allocation");
    }
    h->dev.planes = (const uint8_t *)h->alloc;
    h->dev.dplane = p.dbytes ? (const uint16_t *)((uint8_t *)h->alloc + p.plane_bytes) : nullptr;
    h->dev.hplane = p.hbytes ? (const uint32_t *)((uint8_t *)h->alloc + p.plane_bytes + p.dpad) : nullptr;
    h->dev.quant = dev_quant(quant);
    h->quant = quant;
    h->dev.rows = (int)rows;
    h->dev.cols = (int)cols;
    h->dev.nb = (int)p.nb;
    h->dev.tensor_scale = tensor_scale;
    h->device_bytes = p.plane_bytes + p.dbytes + p.hbytes;
    h->gguf_bytes = p.payload + trailer_bytes(quant);
    h->row_bytes = p.nb * (size_t)fmt_of(quant).bb;
    h->tile_done.assign((rows + 7) / 8, 0);
    *out = h;
    return JK_OK;
}

static void free_handle(jk_weight *h) {
    if (h->alloc) (void)hipFree(h->alloc);
    delete h;
}

// Copies rows [r0, r1) of a host GGUF payload to a transient device buffer and repacks them
// into h; returns once the stream has consumed the host bytes and the buffer.
static jk_status upload_rows(hipStream_t st, jk_weight *h, const uint8_t *rows_bytes, size_t r0, size_t r1,
                             const char *what) {
    const size_t bytes = (r1 - r0) * h->row_bytes;
    uint8_t *staging = nullptr;
    hipError_t e = hipMalloc(&staging, bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(staging, rows_bytes, bytes, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) {
        if (staging) (void)hipFree(staging);
        return hip_fail(e, what);
    }
    const jk_status rs = launch_repack(st, h->dev, h->quant, staging, (int)r0, (int)r1);
    // The staging buffer may only be released once the repack kernel has consumed it.
    const hipError_t se = hipStreamSynchronize(st);
    (void)hipFree(staging);
    if (rs != JK_OK) return rs;
    if (se != hipSuccess) return hip_fail(se, what);
    return JK_OK;
}

// Tile bookkeeping of a handle being assembled: refuses a sealed handle or a bad range.
static jk_status tile_range_check(jk_weight *w, size_t tb, size_t te, const char *what) {
    if (w->ready) return fail(JK_TENSOR_BOUNDS, "%s: the weight is sealed and immutable", what);
    const size_t n_tiles = w->tile_done.size();
    if (tb > te || te > n_tiles)
        return fail(JK_TENSOR_BOUNDS, "%s: tile_range %zu..%zu exceeds n_tiles (%zu)", what, tb, te, n_tiles);
    return JK_OK;
}

static void mark_tiles(jk_weight *w, size_t tb, size_t te) {
    std::lock_guard<std::mutex> lock(w->mu);
    for (size_t t = tb; t < te; ++t) w->tile_done[t] = 1;
}

jk_status jk_weight_upload(jk_stream s, const jk_tensor_view *w, size_t rows, size_t cols,
                           jk_weight **out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "null weight out-pointer");
    *out = nullptr;
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape))
        return fail(JK_TENSOR_BOUNDS, "null tensor view");
    // BlockScaledTileLayout::for_tensor (repack.rs:1308-1333): dense and unsupported
    // formats are a CapabilityMismatch.
    if (!fmt_known(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "%s: quant type %d is not supported by libjk", tname(w), (int)w->quant);
    if (rows == 0 && cols == 0) {
        // RepackedWeight::repack orientation inference (repack.rs:2255-2285).
        if (w->ndim != 2)
            return fail(JK_TENSOR_BOUNDS, "%s: RepackedWeight::repack requires a 2D tensor, got %zuD", tname(w), w->ndim);
        size_t d0 = w->shape[0], d1 = w->shape[1], be = (size_t)fmt_of(w->quant).be;
        if (d0 % be == 0 && d1 % be != 0) { rows = d1; cols = d0; }
        else if (d1 % be == 0 && d0 % be != 0) { rows = d0; cols = d1; }
        else { rows = d1; cols = d0; }
    }
    JK_TRY(check_view_dims(w, rows, cols));
    const size_t payload = plane_sizes(w->quant, rows, cols).payload;
    const float scale = w->quant == JK_I2_S
                            ? read_trailer_scale((const uint8_t *)w->bytes + payload, w->byte_len - payload)
                            : 0.0f;
    jk_weight *h = nullptr;
    JK_TRY(alloc_handle(w->quant, rows, cols, scale, &h));
    h->name = tname(w);
    h->offset = w->offset;
    const jk_status st = upload_rows((hipStream_t)s, h, (const uint8_t *)w->bytes, 0, rows, "jk_weight_upload");
    if (st != JK_OK) {
        free_handle(h);
        return st;
    }
    mark_tiles(h, 0, h->tile_done.size());
    h->ready = true;
    *out = h;
    return JK_OK;
}

jk_status jk_weight_layout_for(const jk_tensor_view *w, size_t rows, size_t cols, jk_weight_layout *out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "null layout out-pointer");
    JK_TRY(check_view_dims(w, rows, cols));
    const int q = w->quant;
    const PlaneSizes p = plane_sizes(q, rows, cols);
    memset(out, 0, sizeof *out);
    out->quant = q;
    out->rows = rows;
    out->cols = cols;
    out->row_bytes = p.nb * (size_t)fmt_of(q).bb;
    out->k_padded = (cols + 31) / 32 * 32;  // ACT_Q8_GROUP_ELEMENTS
    out->n_tiles = (rows + 7) / 8;          // tile_count (ime.rs:70), TILE_N = 8
    out->k_chunks = out->k_padded / 16;     // TILE_K = 16
    out->chunks_per_scale = (q == JK_Q6_K || q == JK_Q3_K || q == JK_Q2_K) ? 1 : 2;
    out->scale_groups = out->k_chunks / out->chunks_per_scale;
    out->has_mins = q == JK_Q4_K || q == JK_Q5_K || q == JK_Q4_1 || q == JK_Q5_1 || q == JK_Q2_K;
    out->total_tiles = out->n_tiles * out->k_chunks;
    out->total_scales = out->n_tiles * out->scale_groups * 8;
    out->total_mins = out->has_mins ? out->total_scales : 0;
    out->device_bytes = p.plane_bytes + p.dbytes + p.hbytes;
    out->gguf_bytes = p.payload + trailer_bytes(q);
    out->tensor_scale =
        q == JK_I2_S ? read_trailer_scale((const uint8_t *)w->bytes + p.payload, w->byte_len - p.payload) : 0.0f;
    return JK_OK;
}

jk_status jk_weight_create(jk_stream s, const jk_weight_layout *L, jk_weight **out) {
    if (!out) return fail(JK_TENSOR_BOUNDS, "null weight out-pointer");
    *out = nullptr;
    if (!L) return fail(JK_TENSOR_BOUNDS, "jk_weight_create: null layout");
    if (!fmt_known(L->quant))
        return fail(JK_CAPABILITY_MISMATCH, "jk_weight_create: quant type %d is not supported by libjk", (int)L->quant);
    const size_t be = (size_t)fmt_of(L->quant).be;
    if (L->rows == 0 || L->cols == 0 || L->cols % be || L->rows >= kMaxRows || L->cols / be >= kMaxRows ||
        L->rows * (L->cols / be) >= ((size_t)1 << 28))
        return fail(JK_TENSOR_BOUNDS, "jk_weight_create: invalid dimensions [%zu, %zu]", L->rows, L->cols);
    const PlaneSizes p = plane_sizes(L->quant, L->rows, L->cols);
    if (L->n_tiles != (L->rows + 7) / 8 || L->row_bytes != p.nb * (size_t)fmt_of(L->quant).bb ||
        L->device_bytes != p.plane_bytes + p.dbytes + p.hbytes)
        return fail(JK_TENSOR_BOUNDS, "jk_weight_create: the layout does not describe a [%zu, %zu] %s weight", L->rows,
                    L->cols, quant_name(L->quant));
    jk_weight *h = nullptr;
    JK_TRY(alloc_handle(L->quant, L->rows, L->cols, L->quant == JK_I2_S ? L->tensor_scale : 0.0f, &h));
    const size_t total = p.plane_bytes + p.dpad + p.hbytes + 256;
    hipError_t e = hipMemsetAsync(h->alloc, 0, total, (hipStream_t)s);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)s);
    if (e != hipSuccess) {
        free_handle(h);
        return hip_fail(e, "jk_weight_create");
    }
    *out = h;
    return JK_OK;
}

jk_status jk_weight_upload_tile_range(jk_stream s, jk_weight *w, const jk_tensor_view *v, size_t tb, size_t te) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "repack_into_tile_range: null weight handle");
    const size_t rows = (size_t)w->dev.rows, cols = (size_t)w->dev.cols;
    JK_TRY(check_view_dims(v, rows, cols));
    if (v->quant != w->quant)
        return fail(JK_TENSOR_BOUNDS, "%s: view format %s does not match the weight's %s", tname(v),
                    quant_name(v->quant), quant_name(w->quant));
    if (w->quant == JK_I2_S) {
        const size_t payload = rows * w->row_bytes;
        const float sc = read_trailer_scale((const uint8_t *)v->bytes + payload, v->byte_len - payload);
        if (memcmp(&sc, &w->dev.tensor_scale, 4))
            return fail(JK_TENSOR_BOUNDS, "%s: I2_S trailer scale differs from the layout's", tname(v));
    }
    JK_TRY(tile_range_check(w, tb, te, "repack_into_tile_range"));
    if (tb == te) return JK_OK;
    const size_t r0 = tb * 8, r1 = std::min(rows, te * 8);
    JK_TRY(upload_rows((hipStream_t)s, w, (const uint8_t *)v->bytes + r0 * w->row_bytes, r0, r1,
                       "repack_into_tile_range"));
    mark_tiles(w, tb, te);
    return JK_OK;
}

jk_status jk_weight_repack_tile_range(jk_stream s, jk_weight *w, const void *gguf, size_t gguf_len, size_t tb,
                                      size_t te) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "repack_tile_range: null weight handle");
    JK_TRY(tile_range_check(w, tb, te, "repack_tile_range"));
    const size_t r0 = tb * 8, r1 = std::min((size_t)w->dev.rows, te * 8);
    const size_t need = tb == te ? 0 : (r1 - r0) * w->row_bytes;
    if (gguf_len != need)
        return fail(JK_TENSOR_BOUNDS, "repack_tile_range: %zu bytes != %zu for tiles %zu..%zu", gguf_len, need, tb, te);
    if (tb == te) return JK_OK;
    if (!gguf) return fail(JK_TENSOR_BOUNDS, "repack_tile_range: null GGUF bytes");
    JK_TRY(launch_repack((hipStream_t)s, w->dev, w->quant, (const uint8_t *)gguf, (int)r0, (int)r1));
    mark_tiles(w, tb, te);
    return JK_OK;
}

jk_status jk_weight_seal(jk_weight *w) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "from_tile_buffers: null weight handle");
    std::lock_guard<std::mutex> lock(w->mu);
    size_t missing = 0, first = 0;
    for (size_t t = 0; t < w->tile_done.size(); ++t)
        if (!w->tile_done[t] && missing++ == 0) first = t;
    if (missing)
        return fail(JK_TENSOR_BOUNDS, "from_tile_buffers: %zu of %zu tiles never written (first: tile %zu)", missing,
                    w->tile_done.size(), first);
    w->ready = true;
    return JK_OK;
}


jk_status jk_weight_free(jk_weight *w) {
    if (!w) return JK_OK;
    hipError_t e = w->alloc ? hipFree(w->alloc) : hipSuccess;
    delete w;
    if (e != hipSuccess) return hip_fail(e, "jk_weight_free");
    return JK_OK;
}

jk_status jk_weight_get_info(const jk_weight *w, jk_weight_info *out) {
    if (!w || !out) return fail(JK_TENSOR_BOUNDS, "null weight handle");
    out->quant = w->quant;
    out->rows = (size_t)w->dev.rows;
    out->cols = (size_t)w->dev.cols;
    out->device_bytes = w->device_bytes;
    out->gguf_bytes = w->gguf_bytes;
    return JK_OK;
}

jk_status jk_weight_dequantize_rows(jk_stream s, const jk_weight *w, size_t r0, size_t r1, float *out,
                                    size_t out_len) {
    JK_TRY(weight_usable(w, "dequantize_rows"));
    if (r0 >= r1 || r1 > (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "row range %zu..%zu out of bounds for %d rows", r0, r1, w->dev.rows);
    if (out_len != (r1 - r0) * (size_t)w->dev.cols)
        return fail(JK_TENSOR_BOUNDS, "output length %zu != %zu rows * %d cols", out_len, r1 - r0, w->dev.cols);
    if (!out) return fail(JK_TENSOR_BOUNDS, "null output");
    return launch_dequant_rows((hipStream_t)s, w->dev, (int)r0, (int)r1, out);
}

// ------------------------------------------------------ activation quantization
jk_status jk_quantize_row_q8_0(jk_stream s, const float *x, size_t n, jk_block_q8_0 *out, size_t out_blocks) {
    // validate_activation_quant_slice (quant_q8.rs:111-149)
    if (n == 0 || n % 32)
        return fail_tb(Tb{"quantize_row_q8_0_f32", 0, n * 4, out_blocks},
                       "quantize_row_q8_0_f32: input length %zu must be a positive multiple of 32", n);
    if (out_blocks != n / 32)
        return fail_tb(Tb{"quantize_row_q8_0_f32", 0, n * 4, out_blocks},
                       "quantize_row_q8_0_f32: output block count %zu != expected %zu", out_blocks, n / 32);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_0: null pointer");
    return launch_quantize_q8_0((hipStream_t)s, x, n / 32, out);
}

jk_status jk_quantize_row_q8_k(jk_stream s, const float *x, size_t n, jk_block_q8k *out, size_t out_blocks) {
    if (n == 0 || n % 256)
        return fail_tb(Tb{"quantize_row_q8_k", 0, n * 4, out_blocks},
                       "quantize_row_q8_k: input length %zu must be a positive multiple of 256", n);
    if (out_blocks != n / 256)
        return fail_tb(Tb{"quantize_row_q8_k", 0, n * 4, out_blocks},
                       "quantize_row_q8_k: output block count %zu != expected %zu", out_blocks, n / 256);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: null pointer");
    return launch_quantize_q8_k((hipStream_t)s, x, n / 256, out);
}

size_t jk_act_q8_bytes(size_t m, size_t k) {
    size_t kp = (k + 31) / 32 * 32, kb = kp / 32, kc = kp / 16, sb = (k + 255) / 256;
    // float arrays first (4-byte aligned), then the i8 values, padded to 256 bytes
    return 4 * m * (kb + kb + kc + sb) + m * kp + 256;
}

jk_status jk_act_q8_bind(void *storage, size_t storage_len, size_t m, size_t k, jk_act_q8 *o) {
    if (!o) return fail(JK_TENSOR_BOUNDS, "null jk_act_q8");
    if (m == 0 || k == 0)
        return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: m and k must be non-zero, got [%zu, %zu]", m, k);
    if (m >= kMaxRows || k >= kMaxRows) return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: [%zu, %zu] too large", m, k);
    if (!storage || storage_len < jk_act_q8_bytes(m, k))
        return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: storage %zu < required %zu", storage_len, jk_act_q8_bytes(m, k));
    if ((uintptr_t)storage % 16)
        return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: storage must be 16-byte aligned");
    o->m = m;
    o->k = k;
    o->k_padded = (k + 31) / 32 * 32;
    o->k_blocks32 = o->k_padded / 32;
    o->k_chunks = o->k_padded / 16;
    o->sb256 = (k + 255) / 256;
    float *f = (float *)storage;
    o->scales = f; f += m * o->k_blocks32;
    o->sums = f; f += m * o->k_blocks32;
    o->sums16 = f; f += m * o->k_chunks;
    o->super256 = f; f += m * o->sb256;
    uintptr_t q = ((uintptr_t)f + 255) & ~(uintptr_t)255;
    o->qs = (int8_t *)q;
    return JK_OK;
}

jk_status jk_quantize_act_q8(jk_stream s, const float *x, size_t m, size_t k, const jk_act_q8 *act) {
    // QuantizedActQ8::quantize_into (repack.rs:542-568)
    if (!act) return fail(JK_TENSOR_BOUNDS, "null jk_act_q8");
    if (m == 0 || k == 0)
        return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: m and k must be non-zero, got [%zu, %zu]", m, k);
    if (act->m != m || act->k != k)
        return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: buffer bound for [%zu, %zu], got [%zu, %zu]", act->m, act->k, m, k);
    if (!x) return fail(JK_TENSOR_BOUNDS, "QuantizedActQ8: null input");
    return launch_quantize_act_q8((hipStream_t)s, x, *act);
}

jk_status jk_subln_quantize_absmax_i8(jk_stream s, const float *x, const float *norm_w, size_t m, size_t k,
                                      float eps, int8_t *q, float *scales) {
    // lib.rs:1048-1061: empty input is a TensorBoundsError
    if (m == 0 || k == 0) return fail(JK_TENSOR_BOUNDS, "subln: dimension mismatch: m=%zu, k=%zu", m, k);
    if (!x || !norm_w || !q || !scales) return fail(JK_TENSOR_BOUNDS, "subln: null pointer");
    if (k >= kMaxRows || m >= kMaxRows) return fail(JK_TENSOR_BOUNDS, "subln: [%zu, %zu] too large", m, k);
    return launch_absmax_i8((hipStream_t)s, x, norm_w, m, k, eps, q, scales);
}

jk_status jk_quantize_absmax_i8(jk_stream s, const float *x, size_t m, size_t k, int8_t *q, float *scales) {
    if (m == 0 || k == 0) return fail(JK_TENSOR_BOUNDS, "absmax: dimension mismatch: m=%zu, k=%zu", m, k);
    if (!x || !q || !scales) return fail(JK_TENSOR_BOUNDS, "absmax: null pointer");
    if (k >= kMaxRows || m >= kMaxRows) return fail(JK_TENSOR_BOUNDS, "absmax: [%zu, %zu] too large", m, k);
    return launch_absmax_i8((hipStream_t)s, x, nullptr, m, k, 0.0f, q, scales);
}

// --------------------------------------------------------------- quant_q8 GEMV
static jk_status gemv_check(const jk_weight *w, int quant, const void *x, size_t nx, const float *y,
                            size_t r0, size_t r1, const char *name) {
    JK_TRY(weight_usable(w, name));
    if (quant && w->quant != quant)
        return fail(JK_TENSOR_BOUNDS, "%s: expected %s quant type, got %s", name, quant_name(quant),
                    quant_name(w->quant));
    if (!has_q8_gemv(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "%s: %s has no quant_q8 GEMV", name, quant_name(w->quant));
    // check_q8_block_len (quant_q8.rs:1562-1578)
    if (nx != (size_t)w->dev.nb)
        return fail_tb(Tb{w->name.c_str(), w->offset, nx, (size_t)w->dev.nb}, "%s: x_blocks len %zu != expected %d",
                       name, nx, w->dev.nb);
    if (r0 > r1 || r1 > (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "%s: row range %zu..%zu out of bounds for %d rows", name, r0, r1, w->dev.rows);
    if (!x || (!y && r1 > r0)) return fail(JK_TENSOR_BOUNDS, "%s: null pointer", name);
    return JK_OK;
}

static jk_status gemv_full(jk_stream s, const jk_weight *w, int quant, const void *x, size_t nx, float *y,
                           size_t y_len, const char *name) {
    JK_TRY(gemv_check(w, quant, x, nx, y, 0, w ? (size_t)w->dev.rows : 0, name));
    if (y_len != (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "%s: output len %zu != rows %d", name, y_len, w->dev.rows);
    return launch_gemv_q8((hipStream_t)s, w->dev, x, y, 0, w->dev.rows);
}

jk_status jk_gemv_q4_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q4_0, x, nx, y, n, "gemv_q4_0_q8_0");
}
jk_status jk_gemv_q8_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q8_0, x, nx, y, n, "gemv_q8_0_q8_0");
}
jk_status jk_gemv_q4_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q4_K, x, nx, y, n, "gemv_q4_k_q8_k");
}
jk_status jk_gemv_q6_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q6_K, x, nx, y, n, "gemv_q6_k_q8_k");
}
jk_status jk_gemv_tq2_0_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_TQ2_0, x, nx, y, n, "gemv_tq2_0_q8_k");
}
jk_status jk_gemv_q5_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q5_0, x, nx, y, n, "gemv_q5_0_q8_0");
}
jk_status jk_gemv_q5_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_Q5_K, x, nx, y, n, "gemv_q5_k_q8_k");
}
jk_status jk_gemv_tq1_0_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx, float *y, size_t n) {
    return gemv_full(s, w, JK_TQ1_0, x, nx, y, n, "gemv_tq1_0_q8_k");
}

jk_status jk_gemv_q8_rows(jk_stream s, const jk_weight *w, const void *x, size_t nx, float *y, size_t r0, size_t r1) {
    JK_TRY(gemv_check(w, 0, x, nx, y, r0, r1, "gemv_q8_rows"));
    if (r0 == r1) return JK_OK;
    return launch_gemv_q8((hipStream_t)s, w->dev, x, y, (int)r0, (int)r1);
}

// Validation shared by the grouped / fused GEMV entries (no reference counterpart for the
// grouping itself; each job follows gemv_* validation, check_q8_block_len quant_q8.rs:1562).
static jk_status gemv_job_check(const jk_gemv_job *j, size_t i, GemvJob *out) {
    const jk_weight *w = j->w;
    if (!w) return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: job %zu: null weight handle", i);
    JK_TRY(weight_usable(w, "gemv_q8_batch"));
    const int q = w->quant;
    if (!has_q8_gemv(q))
        return fail(JK_CAPABILITY_MISMATCH, "gemv_q8_batch: job %zu: %s has no quant_q8 GEMV", i, quant_name(q));
    if ((j->x_q8 == nullptr) == (j->x_f32 == nullptr))
        return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: job %zu: exactly one of x_q8 and x_f32 must be set", i);
    if ((uintptr_t)j->x_q8 % 4 || (uintptr_t)j->x_f32 % 16)
        return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: job %zu: x_q8 must be 4-byte and x_f32 16-byte aligned", i);
    if (j->row_begin > j->row_end || j->row_end > (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: job %zu: row range %zu..%zu out of bounds for %d rows", i,
                    j->row_begin, j->row_end, w->dev.rows);
    if (!j->y && j->row_end > j->row_begin) return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: job %zu: null output", i);
    if (j->x_f32 && (size_t)w->dev.cols > gemv_f32_max_cols(w->dev.quant))
        return fail(JK_CAPABILITY_MISMATCH, "gemv_q8_batch: job %zu: f32 activations need K <= %zu, got %d", i,
                    gemv_f32_max_cols(w->dev.quant), w->dev.cols);
    memset(out, 0, sizeof *out);
    out->w = w->dev;
    out->xq = j->x_q8;
    out->xf = j->x_f32;
    out->y = j->y;
    out->r0 = (int)j->row_begin;
    out->r1 = (int)j->row_end;
    return JK_OK;
}

jk_status jk_gemv_q8_batch(jk_stream s, const jk_gemv_job *jobs, size_t njobs) {
    if (njobs == 0) return JK_OK;
    if (!jobs) return fail(JK_TENSOR_BOUNDS, "gemv_q8_batch: null job array");
    // validate everything before launching anything (fail closed)
    for (size_t i = 0; i < njobs; ++i) {
        GemvJob tmp;
        JK_TRY(gemv_job_check(&jobs[i], i, &tmp));
    }
    // launch runs of consecutive non-empty jobs that share a weight format
    GemvJob run[kMaxGemvJobs];
    int n = 0, quant = 0;
    for (size_t i = 0; i < njobs; ++i) {
        GemvJob gj;
        JK_TRY(gemv_job_check(&jobs[i], i, &gj));
        if (gj.r1 == gj.r0) continue;
        if (n == kMaxGemvJobs || (n > 0 && gj.w.quant != quant)) {
            JK_TRY(launch_gemv_group((hipStream_t)s, run, n));
            n = 0;
        }
        quant = gj.w.quant;
        run[n++] = gj;
    }
    return launch_gemv_group((hipStream_t)s, run, n);
}

jk_status jk_gemv_q8_f32(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y, size_t y_len) {
    JK_TRY(weight_usable(w, "gemv_q8_f32"));
    if (n != (size_t)w->dev.cols)
        return fail(JK_TENSOR_BOUNDS, "gemv_q8_f32: input len %zu != cols %d", n, w->dev.cols);
    if (y_len != (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "gemv_q8_f32: output len %zu != rows %d", y_len, w->dev.rows);
    if (!x) return fail(JK_TENSOR_BOUNDS, "gemv_q8_f32: null input");
    jk_gemv_job j = {w, nullptr, x, y, 0, (size_t)w->dev.rows};
    return jk_gemv_q8_batch(s, &j, 1);
}

// --------------------------------------------------------------- epilogues
// validate_gated_activation_args (swiglu.rs:33-52; lib.rs:1112-1125 likewise)
static jk_status gated_check(const char *name, const float *gate, const float *up, size_t n, const void *out) {
    if (n == 0) return fail(JK_TENSOR_BOUNDS, "%s: dimension mismatch: gate=0", name);
    if (!gate || !up || !out) return fail(JK_TENSOR_BOUNDS, "%s: null pointer", name);
    return JK_OK;
}

jk_status jk_swiglu_f32(jk_stream s, const float *gate, const float *up, size_t n, float *out) {
    JK_TRY(gated_check("swiglu", gate, up, n, out));
    return launch_gated((hipStream_t)s, JK_ACT_SWIGLU, gate, up, n, out);
}

jk_status jk_relu_squared_gate_f32(jk_stream s, const float *gate, const float *up, size_t n, float *out) {
    JK_TRY(gated_check("relu_squared", gate, up, n, out));
    return launch_gated((hipStream_t)s, JK_ACT_RELU2, gate, up, n, out);
}

jk_status jk_quantize_row_q8_k_gated(jk_stream s, int act, const float *gate, const float *up, size_t n,
                                     jk_block_q8k *out, size_t out_blocks) {
    if (act != JK_ACT_SWIGLU && act != JK_ACT_RELU2)
        return fail(JK_CAPABILITY_MISMATCH, "quantize_row_q8_k_gated: unknown activation %d", act);
    JK_TRY(gated_check("quantize_row_q8_k_gated", gate, up, n, out));
    if (n % 256)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: input length %zu must be a positive multiple of 256", n);
    if (out_blocks != n / 256)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: output block count %zu != expected %zu", out_blocks, n / 256);
    return launch_quantize_q8_k_gated((hipStream_t)s, act, gate, up, n / 256, out);
}

jk_status jk_quantize_act_q8_gated(jk_stream s, int act, const float *gate, const float *up, size_t m, size_t k,
                                   const jk_act_q8 *a) {
    if (act != JK_ACT_SWIGLU && act != JK_ACT_RELU2)
        return fail(JK_CAPABILITY_MISMATCH, "quantize_act_q8_gated: unknown activation %d", act);
    if (!a || a->m != m || a->k != k || m == 0 || k == 0)
        return fail(JK_TENSOR_BOUNDS, "quantize_act_q8_gated: activation buffer does not hold [%zu, %zu]", m, k);
    if (!gate || !up) return fail(JK_TENSOR_BOUNDS, "quantize_act_q8_gated: null input");
    return launch_quantize_act_q8_gated((hipStream_t)s, act, gate, up, *a);
}

size_t jk_argmax_workspace_bytes(size_t n) { return argmax_ws_bytes(n); }

static jk_status argmax_ws_check(const char *what, const void *ws, size_t ws_bytes, size_t n) {
    if (!ws) return fail(JK_TENSOR_BOUNDS, "%s: null workspace", what);
    if ((uintptr_t)ws % 8) return fail(JK_TENSOR_BOUNDS, "%s: workspace must be 8-byte aligned", what);
    if (ws_bytes < argmax_ws_bytes(n))
        return fail(JK_TENSOR_BOUNDS, "%s: workspace of %zu bytes < %zu needed for %zu values", what, ws_bytes,
                    argmax_ws_bytes(n), n);
    return JK_OK;
}

jk_status jk_argmax_f32(jk_stream s, const float *x, size_t n, int32_t *index, void *ws, size_t ws_bytes) {
    if (!index || (n && !x)) return fail(JK_TENSOR_BOUNDS, "argmax: null pointer");
    if (n > (size_t)INT32_MAX) return fail(JK_TENSOR_BOUNDS, "argmax: %zu values exceed the int32 index range", n);
    JK_TRY(argmax_ws_check("argmax", ws, ws_bytes, n));
    return launch_argmax((hipStream_t)s, x, n, index, ws);
}

jk_status jk_gemv_q8_argmax(jk_stream s, const jk_weight *w, const void *x_q8, const float *x_f32, size_t x_len,
                            float *y, int32_t *index, void *ws, size_t ws_bytes) {
    GemvJob j;
    JK_TRY(gemv_argmax_job("gemv_q8_argmax", w, x_q8, x_f32, x_len, y, index, &j));
    JK_TRY(argmax_ws_check("gemv_q8_argmax", ws, ws_bytes, (size_t)w->dev.rows));
    j.am_slots = static_cast<unsigned long long *>(ws);
    return launch_gemv_group((hipStream_t)s, &j, 1);
}

// ------------------------------------------------ I2_S -> TQ2_0 conversion
// convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790) over a run of block pairs.
jk_status jk_convert_i2_s_to_tq2_0(jk_stream s, const void *i2s, size_t i2s_blocks, uint16_t scale_f16_bits,
                                   void *tq2, size_t tq2_blocks) {
    if (i2s_blocks != 2 * tq2_blocks)
        return fail(JK_TENSOR_BOUNDS, "convert_i2_s_blocks_to_tq2_0: %zu I2_S blocks != 2 x %zu TQ2_0 blocks",
                    i2s_blocks, tq2_blocks);
    if (tq2_blocks == 0) return JK_OK;
    if (!i2s || !tq2) return fail(JK_TENSOR_BOUNDS, "convert_i2_s_blocks_to_tq2_0: null pointer");
    if (tq2_blocks > ((size_t)1 << 31) / 17)
        return fail(JK_TENSOR_BOUNDS, "convert_i2_s_blocks_to_tq2_0: %zu blocks exceed one launch", tq2_blocks);
    return launch_i2s_to_tq2((hipStream_t)s, static_cast<const uint8_t *>(i2s), tq2_blocks, scale_f16_bits,
                             static_cast<uint8_t *>(tq2));
}

// -------------------------------------------------------------- vec_dot (f32)
static jk_status vec_dot_check(const jk_weight *w, const float *x, size_t n, const float *y, size_t y_len) {
    JK_TRY(weight_usable(w, "vec_dot"));
    int q = w->quant;
    if (!has_vec_dot_f32(q))
        return fail(JK_CAPABILITY_MISMATCH, "vec_dot: %s has no f32-activation matvec", quant_name(q));
    if (n != (size_t)w->dev.cols || y_len != (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "vec_dot: matrix [%d, %d] does not match output len %zu and input len %zu",
                    w->dev.rows, w->dev.cols, y_len, n);
    if (!x || !y) return fail(JK_TENSOR_BOUNDS, "vec_dot: null pointer");
    return JK_OK;
}

jk_status jk_vec_dot_f32(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y, size_t y_len) {
    JK_TRY(vec_dot_check(w, x, n, y, y_len));
    return launch_vec_dot_f32((hipStream_t)s, w->dev, x, y);
}

jk_status jk_vec_dot_f32_tol(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y, size_t y_len) {
    JK_TRY(vec_dot_check(w, x, n, y, y_len));
    return launch_vec_dot_f32_tol((hipStream_t)s, w->dev, x, y);
}

// ------------------------------------------------------------ repacked GEMM
// execute_gemm_repacked_rows (repack.rs:2725-2778) validation, shared by both GEMM modes. *run
// is false for an empty row range or token count (nothing to launch).
static jk_status gemm_check(const jk_weight *w, const jk_act_q8 *act, const float *y, size_t y_len, size_t r0,
                            size_t r1, bool *run) {
    *run = false;
    if (!w || !act) return fail(JK_TENSOR_BOUNDS, "gemm_repacked: null argument");
    JK_TRY(weight_usable(w, "gemm_repacked"));
    // the reference reports the output bytes and the repacked storage (aligned_bytes) as byte_len /
    // buffer_len; the storage here is the device layout
    if (act->k != (size_t)w->dev.cols)
        return fail_tb(Tb{"gemm_repacked", 0, y_len * 4, w->device_bytes},
                       "gemm_repacked: activation K (%zu) != weight cols (%d)", act->k, w->dev.cols);
    if (r0 > r1 || r1 > (size_t)w->dev.rows)
        return fail_tb(Tb{"gemm_repacked", r0, r1 >= r0 ? r1 - r0 : 0, (size_t)w->dev.rows},
                       "gemm_repacked: invalid row_range %zu..%zu for weight rows %d", r0, r1, w->dev.rows);
    if (y_len != act->m * (r1 - r0))
        return fail_tb(Tb{"gemm_repacked", 0, y_len * 4, act->m * (r1 - r0) * 4},
                       "gemm_repacked: output length %zu != m (%zu) * sub_rows (%zu)", y_len, act->m, r1 - r0);
    if (r1 == r0 || act->m == 0) return JK_OK;
    if (!y) return fail(JK_TENSOR_BOUNDS, "gemm_repacked: null output");
    if (act->m > ((size_t)1 << 24))
        return fail(JK_TENSOR_BOUNDS, "gemm_repacked: %zu tokens exceed the 2^24 per call this device path tiles",
                    act->m);
    *run = true;
    return JK_OK;
}

jk_status jk_gemm_repacked(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y, size_t y_len,
                           size_t r0, size_t r1) {
    bool run;
    JK_TRY(gemm_check(w, act, y, y_len, r0, r1, &run));
    if (!run) return JK_OK;
    return launch_gemm_repacked((hipStream_t)s, w->dev, *act, y, (int)r0, (int)r1);
}

jk_status jk_gemm_repacked_tol(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y, size_t y_len,
                               size_t r0, size_t r1) {
    bool run;
    JK_TRY(gemm_check(w, act, y, y_len, r0, r1, &run));
    if (!run) return JK_OK;
    return launch_gemm_repacked_tol((hipStream_t)s, w->dev, *act, y, (int)r0, (int)r1);
}
jk_status jk_gemv_repacked(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y, size_t y_len,
                           size_t r0, size_t r1) {
    if (act && act->m != 1)
        return fail_tb(Tb{"gemv_repacked", 0, y_len * 4, w ? w->device_bytes : 0},
                       "gemv_repacked: gemv_repacked requires act.m() == 1, got %zu", act->m);
    return jk_gemm_repacked(s, w, act, y, y_len, r0, r1);
}

// Which kernel a jk_gemm_repacked (tolerance = 0) or jk_gemm_repacked_tol (1) call with these
// arguments launches: the launcher runs with its launch recorded instead of made.
jk_status jk_gemm_plan(const jk_weight *w, const jk_act_q8 *act, size_t r0, size_t r1, int tolerance,
                       const char **kernel) {
    if (!kernel) return fail(JK_TENSOR_BOUNDS, "gemm_plan: null kernel");
    *kernel = nullptr;
    bool run;
    float dummy;
    JK_TRY(gemm_check(w, act, &dummy, act ? act->m * (r1 - r0) : 0, r0, r1, &run));
    if (!run) return JK_OK;
    t_plan = LaunchPlan{true, nullptr};
    const jk_status st = tolerance ? launch_gemm_repacked_tol(nullptr, w->dev, *act, &dummy, (int)r0, (int)r1)
                                   : launch_gemm_repacked(nullptr, w->dev, *act, &dummy, (int)r0, (int)r1);
    *kernel = t_plan.kernel;
    t_plan = LaunchPlan{};
    return st;
}

// ---------------------------------------------------------------- BitLinear
// validate_bitlinear_dimensions (ime.rs:660-684): other formats are a TensorBoundsError
static jk_status bitlinear_check(const jk_weight *w, const int8_t *act, const float *act_scales, size_t m, size_t k,
                                 const float *y, size_t y_len) {
    JK_TRY(weight_usable(w, "bitlinear"));
    const int q = w->quant;
    const Tb wt{w->name.c_str(), w->offset, w->gguf_bytes, w->gguf_bytes};
    if (!has_bitlinear(q)) return fail_tb(wt, "%s: bitlinear: unsupported quant type %s", wt.name, quant_name(q));
    if (m == 0 || k != (size_t)w->dev.cols || y_len != m * (size_t)w->dev.rows)
        return fail_tb(wt, "%s: bitlinear: weights [%d, %d] do not match m=%zu k=%zu out=%zu", wt.name, w->dev.rows,
                       w->dev.cols, m, k, y_len);
    if (m >= kMaxRows) return fail(JK_TENSOR_BOUNDS, "bitlinear: m=%zu too large", m);
    if (!act || !act_scales || !y) return fail(JK_TENSOR_BOUNDS, "bitlinear: null pointer");
    return JK_OK;
}

// bitlinear_i8_rvv adds one dot_i8_vector call per weight block and token to the crate's vector-dot
// counter (ime.rs:919-936); the batched kernels count the same
static void count_bitlinear_dots(const jk_weight *w, size_t m) {
    count_vector_dots((uint64_t)m * (uint64_t)w->dev.rows * (uint64_t)(w->dev.cols / fmt_of(w->quant).be));
}

jk_status jk_bitlinear_i8(jk_stream s, const jk_weight *w, const int8_t *act, const float *act_scales, size_t m,
                          size_t k, float *y, size_t y_len) {
    JK_TRY(bitlinear_check(w, act, act_scales, m, k, y, y_len));
    // batches of tokens run as an int8-MFMA GEMM (same per-block arithmetic and block order)
    if (m >= (size_t)kBitlinearMfmaMinTokens)
        JK_TRY(launch_bitlinear_mfma((hipStream_t)s, w->dev, act, act_scales, (int)m, y));
    else
        JK_TRY(launch_bitlinear((hipStream_t)s, w->dev, act, act_scales, (int)m, y));
    count_bitlinear_dots(w, m);
    return JK_OK;
}

jk_status jk_bitlinear_i8_tol(jk_stream s, const jk_weight *w, const int8_t *act, const float *act_scales, size_t m,
                              size_t k, float *y, size_t y_len) {
    JK_TRY(bitlinear_check(w, act, act_scales, m, k, y, y_len));
    if (m >= (size_t)kBitlinearMfmaMinTokens)
        JK_TRY(launch_bitlinear_mfma_tol((hipStream_t)s, w->dev, act, act_scales, (int)m, y));
    else
        JK_TRY(launch_bitlinear((hipStream_t)s, w->dev, act, act_scales, (int)m, y));  // bit-exact rows
    count_bitlinear_dots(w, m);
    return JK_OK;
}

// Which kernel a jk_bitlinear_i8 (tolerance 0) or jk_bitlinear_i8_tol (1) call of m tokens on w
// launches, for activation rows at `act` (their alignment can choose the kernel).
jk_status jk_bitlinear_plan(const jk_weight *w, const int8_t *act, size_t m, int tolerance, const char **kernel) {
    if (!kernel) return fail(JK_TENSOR_BOUNDS, "bitlinear_plan: null kernel");
    *kernel = nullptr;
    JK_TRY(weight_usable(w, "bitlinear"));
    if (!has_bitlinear(w->quant)) return fail(JK_CAPABILITY_MISMATCH, "bitlinear_plan: unsupported quant %d", w->quant);
    if (m == 0 || m >= kMaxRows || !act) return fail(JK_TENSOR_BOUNDS, "bitlinear_plan: m=%zu", m);
    float dummy;
    t_plan = LaunchPlan{true, nullptr};
    jk_status st;
    if (m < (size_t)kBitlinearMfmaMinTokens) st = launch_bitlinear(nullptr, w->dev, act, &dummy, (int)m, &dummy);
    else if (tolerance) st = launch_bitlinear_mfma_tol(nullptr, w->dev, act, &dummy, (int)m, &dummy);
    else st = launch_bitlinear_mfma(nullptr, w->dev, act, &dummy, (int)m, &dummy);
    *kernel = t_plan.kernel;
    t_plan = LaunchPlan{};
    return st;
}

}  // extern "C"
