// jk_gemv.hip -- f32-activation matvec (vec_dot_*) and BitLinear kernels on the plane layout.
//
// Work mapping (all kernels here): a workgroup of 256 lanes covers 16 output rows;
// each 16-lane DPP row of a wave owns one output row and lane p of it processes
// blocks p, p + 16, p + 32, ... of that row. A lane computes its block's value with
// the reference's per-block arithmetic (integer dot + f32 epilogue, or sequential
// dequantize-multiply-add), then chain_add() folds the 16 block values into the row
// accumulator in block order. The result therefore equals the reference's
// sequential block-order f32 sum bit for bit.
//
// The weight stream is read once with 128-bit non-temporal loads; activation blocks
// are small and shared by all rows, so they are read through the caches.
#include "jk_device.hpp"

namespace jk {

// ----------------------------------------------------------- f32-activation block values
// Each returns dot_product_f32_scalar(dequantized block, x block) (lib.rs:770-778): one
// product and one add per element in element order, starting from +0.0.

__device__ float fv_block(const WeightDev &w, int r, int b, const float *__restrict__ x) {
    float sum = 0.0f;
    switch (w.quant) {
    case JK_Q4_0: {  // dequantize_q4_0_block (quant.rs:550-568)
        const float d = ld_dscale(w, r, b);
        const uint4 q = ld_chunk(w, 0, r, b);
        const float *xb = x + 32 * (size_t)b;
        for (int i = 0; i < 32; ++i) {
            const int nib = (int)((comp(q, (i & 15) >> 2) >> (8 * (i & 3) + (i >> 4) * 4)) & 15u);
            const float wv = d == 0.0f ? 0.0f : d * (float)(nib - 8);
            sum += wv * xb[i];
        }
        break;
    }
    case JK_Q8_0: {  // dequantize_q8_0_block (quant.rs:571-588)
        const float d = ld_dscale(w, r, b);
        const uint4 q0 = ld_chunk(w, 0, r, b), q1 = ld_chunk(w, 1, r, b);
        const float *xb = x + 32 * (size_t)b;
        for (int i = 0; i < 32; ++i) {
            const uint32_t dw = comp(i < 16 ? q0 : q1, (i & 15) >> 2);
            const int qv = (int)(int8_t)(dw >> (8 * (i & 3)));
            const float wv = d == 0.0f ? 0.0f : d * (float)qv;
            sum += wv * xb[i];
        }
        break;
    }
    case JK_Q4_K: {  // dequantize_q4_k_m_block (lib.rs:720-766)
        const uint4 h = ld_chunk(w, 0, r, b);
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        const float *xb = x + 256 * (size_t)b;
        for (int c = 0; c < 4; ++c) {
            const uint32_t scv = c < 2 ? sc_lo : sc_hi, mv = c < 2 ? m_lo : m_hi;
            const int j = (2 * c) & 3;
            const float d1 = d * (float)byte_of(scv, j), m1 = dmin * (float)byte_of(mv, j);
            const float d2 = d * (float)byte_of(scv, j + 1), m2 = dmin * (float)byte_of(mv, j + 1);
            const uint4 qa = ld_chunk(w, 1 + 2 * c, r, b), qb = ld_chunk(w, 2 + 2 * c, r, b);
            for (int l = 0; l < 32; ++l) {
                const uint32_t dw = comp(l < 16 ? qa : qb, (l & 15) >> 2);
                const float wv = d1 * (float)((dw >> (8 * (l & 3))) & 15u) - m1;
                sum += wv * xb[64 * c + l];
            }
            for (int l = 0; l < 32; ++l) {
                const uint32_t dw = comp(l < 16 ? qa : qb, (l & 15) >> 2);
                const float wv = d2 * (float)((dw >> (8 * (l & 3) + 4)) & 15u) - m2;
                sum += wv * xb[64 * c + 32 + l];
            }
        }
        break;
    }
    case JK_Q6_K: {  // dequantize_q6_k_block (quant.rs:594-648), visited in element order
        const float d = ld_dscale(w, r, b);
        const uint4 scv = ld_chunk(w, 12, r, b);
        const float *xb = x + 256 * (size_t)b;
        for (int e = 0; e < 256; ++e) {
            float wv = 0.0f;
            if (d != 0.0f) {
                const int h = e >> 7, rr = e & 127, quarter = rr >> 5, l = rr & 31;
                const int lbyte = 64 * h + l + ((quarter & 1) ? 32 : 0);
                const int qbyte = 32 * h + l;
                const uint32_t Lw = comp(ld_chunk(w, lbyte >> 4, r, b), (lbyte & 15) >> 2);
                const uint32_t Qw = comp(ld_chunk(w, 8 + (qbyte >> 4), r, b), (qbyte & 15) >> 2);
                const int L = (int)((Lw >> (8 * (lbyte & 3))) & 255u);
                const int Q = (int)((Qw >> (8 * (qbyte & 3))) & 255u);
                const int lo = quarter < 2 ? (L & 15) : (L >> 4);
                const int q = (lo | (((Q >> (2 * quarter)) & 3) << 4)) - 32;
                const int sb = 8 * h + (l >> 4) + 2 * quarter;
                const float sc = (float)(int8_t)(comp(scv, sb >> 2) >> (8 * (sb & 3)));
                wv = d * sc * (float)q;
            }
            sum += wv * xb[e];
        }
        break;
    }
    case JK_I2_S: {  // dequantize_i2_s_block (quant.rs:380-387), scale == 0 handled by the caller
        const float sc = w.tensor_scale;
        const uint4 q0 = ld_chunk(w, 0, r, b), q1 = ld_chunk(w, 1, r, b);
        const float *xb = x + 128 * (size_t)b;
        for (int e = 0; e < 128; ++e) {
            const int grp = e >> 5, g = e & 31;
            const uint32_t dw = comp(g < 16 ? q0 : q1, (g & 15) >> 2);
            const int byte = (int)((dw >> (8 * (g & 3))) & 255u);
            const int t = ((byte >> (6 - 2 * grp)) & 3) - 1;
            sum += (sc * (float)t) * xb[e];
        }
        break;
    }
    default: break;
    }
    return sum;
}

// vec_dot_{q4_0,q8_0,q6_k}_scalar (quant.rs:1401-1436, 899-934, 1012-1047),
// vec_dot_q4_k_m_scalar (lib.rs:1268-1303), vec_dot_i2_s (quant.rs:2199-2240):
// row_sum starts at +0.0 and adds each block's dot in block order.
__global__ __launch_bounds__(256) void vec_dot_f32_kernel(WeightDev w, const float *__restrict__ x,
                                                          float *__restrict__ y) {
    const int p = threadIdx.x & 15;
    const int row = (int)((blockIdx.x * 256u + threadIdx.x) >> 4);
    const bool active = row < w.rows;
    const int r = active ? row : 0;
    if (w.quant == JK_I2_S && w.tensor_scale == 0.0f) {
        if (active && p == 0) y[row] = 0.0f;
        return;
    }
    float acc = 0.0f;
    const int nb = w.nb, iters = (nb + 15) >> 4;
    for (int it = 0; it < iters; ++it) {
        const int g = min(16, nb - 16 * it);
        float v = 0.0f;
        if (p < g) v = fv_block(w, r, 16 * it + p, x);
        acc = chain_add(acc, v, g);
    }
    const int g_last = nb - 16 * (iters - 1);
    if (active && p == g_last - 1) y[row] = acc;
}

jk_status launch_vec_dot_f32(hipStream_t s, const WeightDev &w, const float *x, float *y) {
    hipLaunchKernelGGL(vec_dot_f32_kernel, dim3((unsigned)((w.rows + 15) / 16)), dim3(256), 0, s, w, x, y);
    return check_launch("vec_dot_f32_kernel");
}

// ------------------------------------------------------------------------ BitLinear
// bitlinear_i8_rvv (ime.rs:882-938) with unpack_bitlinear_block_i8 (792-871):
// row_sum += f32(dot_i32) * (block_scale * act_scale), block order, from +0.0.
__device__ __forceinline__ float bl_block_value(const WeightDev &w, int r, int b, const int8_t *__restrict__ a,
                                                float as) {
    switch (w.quant) {
    case JK_TQ2_0: {
        uint4 q[4];
        for (int c = 0; c < 4; ++c) q[c] = ld_chunk(w, c, r, b);
        const float bs = ld_dscale(w, r, b);
        const int *av = reinterpret_cast<const int *>(a + 256 * (size_t)b);
        int s = 0, sx = 0;
        for (int k = 0; k < 16; ++k) {
            const uint32_t wv = comp(q[k >> 2], k & 3);
            for (int j = 0; j < 4; ++j) {
                const int xv = av[4 * k + j];
                s = dot4((int)((wv >> (2 * j)) & 0x03030303u), xv, s);
                sx = dot4(xv, 0x01010101, sx);
            }
        }
        return (float)(s - sx) * (bs * as);
    }
    case JK_I2_S: {
        const uint4 q0 = ld_chunk(w, 0, r, b), q1 = ld_chunk(w, 1, r, b);
        const int *av = reinterpret_cast<const int *>(a + 128 * (size_t)b);
        int s = 0, sx = 0;
        for (int c = 0; c < 2; ++c)
            for (int k = 0; k < 4; ++k) {
                const uint32_t wv = comp(c ? q1 : q0, k);
                for (int grp = 0; grp < 4; ++grp) {
                    const int xv = av[8 * grp + 4 * c + k];
                    s = dot4((int)((wv >> (6 - 2 * grp)) & 0x03030303u), xv, s);
                    sx = dot4(xv, 0x01010101, sx);
                }
            }
        return (float)(s - sx) * (w.tensor_scale * as);
    }
    case JK_Q8_0: {
        const uint4 q0 = ld_chunk(w, 0, r, b), q1 = ld_chunk(w, 1, r, b);
        const float bs = ld_dscale(w, r, b);
        const int *av = reinterpret_cast<const int *>(a + 32 * (size_t)b);
        const uint32_t qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int s = 0;
        for (int i = 0; i < 8; ++i) s = dot4((int)qq[i], av[i], s);
        return (float)s * (bs * as);
    }
    default: return 0.0f;
    }
}

__global__ __launch_bounds__(256) void bitlinear_kernel(WeightDev w, const int8_t *__restrict__ act,
                                                        const float *__restrict__ act_scales, float *__restrict__ y) {
    const int p = threadIdx.x & 15;
    const int row = (int)((blockIdx.x * 256u + threadIdx.x) >> 4);
    const int m = blockIdx.y;
    const bool active = row < w.rows;
    const int r = active ? row : 0;
    const int8_t *a = act + (size_t)m * (size_t)w.cols;
    const float as = act_scales[m];
    float acc = 0.0f;
    const int nb = w.nb, iters = (nb + 15) >> 4;
    for (int it = 0; it < iters; ++it) {
        const int g = min(16, nb - 16 * it);
        float v = 0.0f;
        if (p < g) v = bl_block_value(w, r, 16 * it + p, a, as);
        acc = chain_add(acc, v, g);
    }
    const int g_last = nb - 16 * (iters - 1);
    if (active && p == g_last - 1) y[(size_t)m * (size_t)w.rows + row] = acc;
}

jk_status launch_bitlinear(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales, int m,
                           float *y) {
    hipLaunchKernelGGL(bitlinear_kernel, dim3((unsigned)((w.rows + 15) / 16), (unsigned)m), dim3(256), 0, s, w, act,
                       act_scales, y);
    return check_launch("bitlinear_kernel");
}

}  // namespace jk
