// jk_host.hip -- host tier: synchronous host-memory mirrors of the reference signatures.
//
// Each call validates exactly as the reference entry it mirrors, then stages its
// operands on the current device, runs the device-tier kernel, copies the result back
// and synchronizes. Engines that keep weights resident use the device tier instead.
#include <limits.h>
#include <string.h>

#include <vector>

#include "jk_internal.hpp"

namespace jk {

// RAII device buffer for the host tier.
struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    jk_status alloc(size_t n) {
        if (n == 0) n = 16;
        JK_HIP(hipMalloc(&p, n));
        return JK_OK;
    }
};

struct WeightGuard {
    jk_weight *w = nullptr;
    ~WeightGuard() {
        if (w) (void)jk_weight_free(w);
    }
};

static jk_status h2d(void *dst, const void *src, size_t n) {
    if (n) JK_HIP(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    return JK_OK;
}

static jk_status d2h(void *dst, const void *src, size_t n) {
    if (n) JK_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return JK_OK;
}

static jk_status host_gemv(int quant, float *out, size_t out_len, const jk_tensor_view *w, const void *x, size_t nx,
                           size_t xblock_bytes) {
    const Fmt f = fmt_of(quant);
    size_t rows, cols;
    JK_TRY(validate_matvec(w, quant, out_len, nx * (size_t)f.be, &rows, &cols));
    if (nx != cols / (size_t)f.be)  // check_q8_block_len (quant_q8.rs:1562-1578)
        return fail(JK_TENSOR_BOUNDS, "x_blocks len %zu != expected %zu", nx, cols / (size_t)f.be);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "null pointer");
    WeightGuard wg;
    JK_TRY(jk_weight_upload(nullptr, w, rows, cols, &wg.w));
    DevBuf dx, dy;
    JK_TRY(dx.alloc(nx * xblock_bytes));
    JK_TRY(dy.alloc(rows * sizeof(float)));
    JK_TRY(h2d(dx.p, x, nx * xblock_bytes));
    JK_TRY(launch_gemv_q8(nullptr, wg.w->dev, dx.p, (float *)dy.p, 0, (int)rows));
    JK_TRY(d2h(out, dy.p, rows * sizeof(float)));
    return JK_OK;
}

// validate_q8_block_row_bytes (quant_q8.rs:644-664) then the single-row driver: a 1-row
// matrix, whose only row is a tail row of run_4row_chunked_gemv and so sums like `.sum()`.
static jk_status host_vec_dot_row(int quant, const void *wb, size_t w_len, const void *x, size_t nx, float *out,
                                  size_t xblock_bytes) {
    const Fmt f = fmt_of(quant);
    if (nx == 0 || w_len != nx * (size_t)f.bb)
        return fail(JK_TENSOR_BOUNDS, "weight row length %zu != expected %zu", w_len, nx * (size_t)f.bb);
    if (!wb || !x || !out) return fail(JK_TENSOR_BOUNDS, "null pointer");
    size_t shape[2] = {1, nx * (size_t)f.be};
    jk_tensor_view v = {"vec_dot_row", quant, shape, 2, wb, w_len};
    return host_gemv(quant, out, 1, &v, x, nx, xblock_bytes);
}

static jk_status host_vec_dot_f32(int quant, float *out, size_t out_len, const jk_tensor_view *w, const float *in,
                                  size_t in_len) {
    size_t rows, cols;
    JK_TRY(validate_matvec(w, quant, out_len, in_len, &rows, &cols));
    if (!in || !out) return fail(JK_TENSOR_BOUNDS, "null pointer");
    WeightGuard wg;
    JK_TRY(jk_weight_upload(nullptr, w, rows, cols, &wg.w));
    DevBuf dx, dy;
    JK_TRY(dx.alloc(cols * sizeof(float)));
    JK_TRY(dy.alloc(rows * sizeof(float)));
    JK_TRY(h2d(dx.p, in, cols * sizeof(float)));
    JK_TRY(launch_vec_dot_f32(nullptr, wg.w->dev, (const float *)dx.p, (float *)dy.p));
    JK_TRY(d2h(out, dy.p, rows * sizeof(float)));
    return JK_OK;
}

}  // namespace jk

using namespace jk;

extern "C" {

jk_status jk_host_quantize_row_q8_0(const float *x, size_t n, jk_block_q8_0 *out, size_t out_len) {
    if (n == 0 || n % 32)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_0: input length %zu must be a positive multiple of 32", n);
    if (out_len != n / 32)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_0: output block count %zu != expected %zu", out_len, n / 32);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_0: null pointer");
    DevBuf dx, dq;
    JK_TRY(dx.alloc(n * sizeof(float)));
    JK_TRY(dq.alloc(out_len * sizeof(jk_block_q8_0)));
    JK_TRY(h2d(dx.p, x, n * sizeof(float)));
    JK_TRY(launch_quantize_q8_0(nullptr, (const float *)dx.p, out_len, (jk_block_q8_0 *)dq.p));
    return d2h(out, dq.p, out_len * sizeof(jk_block_q8_0));
}

jk_status jk_host_quantize_row_q8_k(const float *x, size_t n, jk_block_q8k *out, size_t out_len) {
    if (n == 0 || n % 256)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: input length %zu must be a positive multiple of 256", n);
    if (out_len != n / 256)
        return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: output block count %zu != expected %zu", out_len, n / 256);
    if (!x || !out) return fail(JK_TENSOR_BOUNDS, "quantize_row_q8_k: null pointer");
    DevBuf dx, dq;
    JK_TRY(dx.alloc(n * sizeof(float)));
    JK_TRY(dq.alloc(out_len * sizeof(jk_block_q8k)));
    JK_TRY(h2d(dx.p, x, n * sizeof(float)));
    JK_TRY(launch_quantize_q8_k(nullptr, (const float *)dx.p, out_len, (jk_block_q8k *)dq.p));
    return d2h(out, dq.p, out_len * sizeof(jk_block_q8k));
}

jk_status jk_host_vec_dot_q4_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q4_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0));
}
jk_status jk_host_vec_dot_q8_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q8_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0));
}
jk_status jk_host_vec_dot_q4_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q4_K, w, w_len, x, nx, out, sizeof(jk_block_q8k));
}
jk_status jk_host_vec_dot_q6_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q6_K, w, w_len, x, nx, out, sizeof(jk_block_q8k));
}
jk_status jk_host_vec_dot_tq2_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_TQ2_0, w, w_len, x, nx, out, sizeof(jk_block_q8k));
}
jk_status jk_host_vec_dot_q5_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q5_0, w, w_len, x, nx, out, sizeof(jk_block_q8_0));
}
jk_status jk_host_vec_dot_q5_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_Q5_K, w, w_len, x, nx, out, sizeof(jk_block_q8k));
}
jk_status jk_host_vec_dot_tq1_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out) {
    return host_vec_dot_row(JK_TQ1_0, w, w_len, x, nx, out, sizeof(jk_block_q8k));
}

jk_status jk_host_gemv_q4_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q4_0, out, n, w, x, nx, sizeof(jk_block_q8_0));
}
jk_status jk_host_gemv_q8_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q8_0, out, n, w, x, nx, sizeof(jk_block_q8_0));
}
jk_status jk_host_gemv_q4_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q4_K, out, n, w, x, nx, sizeof(jk_block_q8k));
}
jk_status jk_host_gemv_q6_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q6_K, out, n, w, x, nx, sizeof(jk_block_q8k));
}
jk_status jk_host_gemv_tq2_0_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_TQ2_0, out, n, w, x, nx, sizeof(jk_block_q8k));
}
jk_status jk_host_gemv_q5_0_q8_0(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx) {
    return host_gemv(JK_Q5_0, out, n, w, x, nx, sizeof(jk_block_q8_0));
}
jk_status jk_host_gemv_q5_k_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_Q5_K, out, n, w, x, nx, sizeof(jk_block_q8k));
}
jk_status jk_host_gemv_tq1_0_q8_k(float *out, size_t n, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx) {
    return host_gemv(JK_TQ1_0, out, n, w, x, nx, sizeof(jk_block_q8k));
}

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

// dequantize_tensor_row (quant.rs:2492-2568) with validate_token_row_geometry (1749-1808).
jk_status jk_host_dequantize_tensor_row(const jk_tensor_view *w, size_t row, float *out, size_t out_len) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape)) return fail(JK_TENSOR_BOUNDS, "null tensor view");
    if (!fmt_known(w->quant))
        return fail(JK_CAPABILITY_MISMATCH, "dequantize_tensor_row: quant type %d is not supported", (int)w->quant);
    const size_t cols = out_len;
    if (cols == 0) return fail(JK_TENSOR_BOUNDS, "dequantize_token_row output slice cannot be empty");
    size_t total = 0;
    if (w->ndim) {
        total = 1;
        for (size_t i = 0; i < w->ndim; i++) total *= w->shape[i];
    }
    if (total == 0 || total % cols)
        return fail(JK_TENSOR_BOUNDS, "tensor element count %zu is not a positive multiple of row width %zu", total, cols);
    const size_t nrows = total / cols;
    if (w->ndim == 2 && !((w->shape[0] == cols && w->shape[1] == nrows) || (w->shape[1] == cols && w->shape[0] == nrows)))
        return fail(JK_TENSOR_BOUNDS, "tensor shape does not match row width %zu and row count %zu", cols, nrows);
    if (row >= nrows) return fail(JK_TENSOR_BOUNDS, "row index %zu out of bounds for %zu rows", row, nrows);
    const Fmt f = fmt_of(w->quant);
    if (cols % (size_t)f.be) return fail(JK_TENSOR_BOUNDS, "row width %zu is not a multiple of %d", cols, f.be);
    const size_t row_bytes = cols / (size_t)f.be * (size_t)f.bb, payload = nrows * row_bytes;
    if (w->byte_len < payload + trailer_bytes(w->quant))
        return fail(JK_TENSOR_BOUNDS, "buffer length %zu < required %zu", w->byte_len, payload + trailer_bytes(w->quant));
    if (!out) return fail(JK_TENSOR_BOUNDS, "null output");
    // Upload just this row (plus the I2_S scale trailer) as a 1-row weight.
    std::vector<uint8_t> one(row_bytes + trailer_bytes(w->quant));
    memcpy(one.data(), (const uint8_t *)w->bytes + row * row_bytes, row_bytes);
    if (trailer_bytes(w->quant)) memcpy(one.data() + row_bytes, (const uint8_t *)w->bytes + payload, 32);
    size_t shape[2] = {1, cols};
    jk_tensor_view v = {w->name, w->quant, shape, 2, one.data(), one.size()};
    WeightGuard wg;
    JK_TRY(jk_weight_upload(nullptr, &v, 1, cols, &wg.w));
    DevBuf dy;
    JK_TRY(dy.alloc(cols * sizeof(float)));
    JK_TRY(launch_dequant_rows(nullptr, wg.w->dev, 0, 1, (float *)dy.p));
    return d2h(out, dy.p, cols * sizeof(float));
}

jk_status jk_host_gemm_repacked_f32(float *out, size_t out_len, const jk_weight *w, const float *input, size_t m,
                                   size_t r0, size_t r1) {
    if (!w) return fail(JK_TENSOR_BOUNDS, "gemm_repacked_f32: null weight handle");
    if (!w->ready) return fail(JK_TENSOR_BOUNDS, "gemm_repacked_f32: the weight has not been sealed (jk_weight_seal)");
    const size_t cols = (size_t)w->dev.cols;
    if (m == 0 || !input)
        return fail(JK_TENSOR_BOUNDS, "gemm_repacked_f32: input must hold m * cols = %zu * %zu values", m, cols);
    if (r0 > r1 || r1 > (size_t)w->dev.rows)
        return fail(JK_TENSOR_BOUNDS, "gemm_repacked: row range %zu..%zu out of bounds for %d rows", r0, r1, w->dev.rows);
    if (out_len != m * (r1 - r0))
        return fail(JK_TENSOR_BOUNDS, "gemm_repacked: output len %zu != %zu * %zu", out_len, m, r1 - r0);
    if (r0 == r1) return JK_OK;
    if (!out) return fail(JK_TENSOR_BOUNDS, "null output");
    DevBuf dx, dact, dy;
    JK_TRY(dx.alloc(m * cols * sizeof(float)));
    JK_TRY(dact.alloc(jk_act_q8_bytes(m, cols)));
    JK_TRY(dy.alloc(out_len * sizeof(float)));
    JK_TRY(h2d(dx.p, input, m * cols * sizeof(float)));
    jk_act_q8 act;
    JK_TRY(jk_act_q8_bind(dact.p, jk_act_q8_bytes(m, cols), m, cols, &act));
    JK_TRY(launch_quantize_act_q8(nullptr, (const float *)dx.p, act));
    JK_TRY(launch_gemm_repacked(nullptr, w->dev, act, (float *)dy.p, (int)r0, (int)r1));
    return d2h(out, dy.p, out_len * sizeof(float));
}

// swiglu_f32 (swiglu.rs:62) / relu_squared_gate_f32 (lib.rs:1111) on host slices, with the
// reference's length check (validate_gated_activation_args, swiglu.rs:33-52).
static jk_status host_gated(int act, float *out, size_t out_len, const float *gate, size_t gate_len, const float *up,
                            size_t up_len) {
    if (gate_len == 0 || out_len != gate_len || up_len != gate_len)
        return fail(JK_TENSOR_BOUNDS, "dimension mismatch: gate=%zu, up=%zu, out=%zu", gate_len, up_len, out_len);
    if (!out || !gate || !up) return fail(JK_TENSOR_BOUNDS, "null pointer");
    const size_t b = gate_len * sizeof(float);
    DevBuf dg, du, dy;
    JK_TRY(dg.alloc(b));
    JK_TRY(du.alloc(b));
    JK_TRY(dy.alloc(b));
    JK_TRY(h2d(dg.p, gate, b));
    JK_TRY(h2d(du.p, up, b));
    JK_TRY(launch_gated(nullptr, act, (const float *)dg.p, (const float *)du.p, gate_len, (float *)dy.p));
    return d2h(out, dy.p, b);
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
    DevBuf dx, dws, di;
    JK_TRY(dx.alloc(n * sizeof(float)));
    JK_TRY(dws.alloc(argmax_ws_bytes(n)));
    JK_TRY(di.alloc(sizeof(int32_t)));
    JK_TRY(h2d(dx.p, x, n * sizeof(float)));
    JK_TRY(launch_argmax(nullptr, (const float *)dx.p, n, (int32_t *)di.p, dws.p));
    int32_t idx = -1;
    JK_TRY(d2h(&idx, di.p, sizeof idx));
    *index = idx;
    return JK_OK;
}

// bitlinear_i8_rvv (ime.rs:882-938) with validate_bitlinear_dimensions (660-763).
jk_status jk_host_bitlinear_i8(float *out, size_t out_len, const jk_tensor_view *w, const int8_t *act, size_t act_len,
                               float act_scale) {
    if (!w || (!w->bytes && w->byte_len) || (w->ndim && !w->shape)) return fail(JK_TENSOR_BOUNDS, "null tensor view");
    const int q = w->quant;
    if (!has_bitlinear(q)) return fail(JK_TENSOR_BOUNDS, "BitLinear: unsupported quant type %d", q);
    if (w->ndim == 0) return fail(JK_TENSOR_BOUNDS, "BitLinear: empty tensor shape");
    const Fmt f = fmt_of(q);
    if (w->ndim == 2) {
        const size_t d0 = w->shape[0], d1 = w->shape[1];
        if (!((out_len == d0 && act_len == d1 && d1 % (size_t)f.be == 0) ||
              (out_len == d1 && act_len == d0 && d0 % (size_t)f.be == 0)))
            return fail(JK_TENSOR_BOUNDS, "BitLinear: shape [%zu, %zu] does not match out %zu / act %zu", d0, d1, out_len,
                        act_len);
    } else {
        size_t total = 1;
        for (size_t i = 0; i < w->ndim; i++) total *= w->shape[i];
        if (act_len == 0 || out_len == 0 || act_len % (size_t)f.be || out_len * act_len != total)
            return fail(JK_TENSOR_BOUNDS, "BitLinear: tensor elements %zu do not match %zu * %zu", total, out_len, act_len);
    }
    const size_t need = out_len * act_len / (size_t)f.be * (size_t)f.bb + trailer_bytes(q);
    if (w->byte_len < need) return fail(JK_TENSOR_BOUNDS, "BitLinear: buffer length %zu < required %zu", w->byte_len, need);
    if (!act || !out) return fail(JK_TENSOR_BOUNDS, "BitLinear: null pointer");
    // The matrix is read as [out_len, act_len] row-major blocks; an explicit [rows, cols]
    // view of the same bytes keeps the orientation the validator accepted.
    size_t shape[2] = {out_len, act_len};
    jk_tensor_view v = {w->name, q, shape, 2, w->bytes, w->byte_len};
    WeightGuard wg;
    JK_TRY(jk_weight_upload(nullptr, &v, out_len, act_len, &wg.w));
    DevBuf da, ds, dy;
    JK_TRY(da.alloc(act_len));
    JK_TRY(ds.alloc(sizeof(float)));
    JK_TRY(dy.alloc(out_len * sizeof(float)));
    JK_TRY(h2d(da.p, act, act_len));
    JK_TRY(h2d(ds.p, &act_scale, sizeof(float)));
    JK_TRY(launch_bitlinear(nullptr, wg.w->dev, (const int8_t *)da.p, (const float *)ds.p, 1, (float *)dy.p));
    return d2h(out, dy.p, out_len * sizeof(float));
}

}  // extern "C"
