// jk_quantize.hip -- activation quantizers, bit-exact with the reference recipes.
//
// Maxima are order-independent, so they are reduced across lanes; sums that the
// reference accumulates in f32 are accumulated sequentially in one lane in the
// reference's order; integer sums are reduced across lanes.
#include "jk_device.hpp"

namespace jk {

// quantize_block_q8_0_scalar (quant_q8.rs:203-219): 32 lanes per block, one element each.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x, size_t nblocks,
                                                            jk_block_q8_0 *__restrict__ out) {
    const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int l = threadIdx.x & 31;
    const bool live = blk < nblocks;
    const float v = live ? x[blk * 32 + l] : 0.0f;
    const float amax = wave_max<32>(__builtin_isfinite(v) ? fabsf(v) : 0.0f);
    if (!live) return;
    if (amax == 0.0f || !__builtin_isfinite(amax)) {
        out[blk].qs[l] = 0;
        if (l == 0) out[blk].d = 0.0f;
        return;
    }
    const float inv = 127.0f / amax;
    out[blk].qs[l] = (int8_t)round_scaled_to_i8(v, inv);
    if (l == 0) out[blk].d = amax / 127.0f;
}

jk_status launch_quantize_q8_0(hipStream_t s, const float *x, size_t nblocks, jk_block_q8_0 *out) {
    const size_t threads = nblocks * 32;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, nblocks, out);
    return check_launch("quantize_q8_0_kernel");
}

// quantize_block_q8_k_scalar (quant_q8.rs:447-475): one wave per block, 4 elements per lane,
// bsums[j] = sum of the 16 quants of lanes 4j..4j+3.
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float *__restrict__ x, size_t nblocks,
                                                            jk_block_q8k *__restrict__ out) {
    const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int l = threadIdx.x & 63;
    const bool live = blk < nblocks;
    float v[4];
    float a = 0.0f;
    for (int i = 0; i < 4; ++i) {
        v[i] = live ? x[blk * 256 + 4 * l + i] : 0.0f;
        a = fmaxf(a, __builtin_isfinite(v[i]) ? fabsf(v[i]) : 0.0f);
    }
    const float amax = wave_max<64>(a);
    int q[4] = {0, 0, 0, 0};
    const bool zero = amax == 0.0f || !__builtin_isfinite(amax);
    if (!zero) {
        const float inv = 127.0f / amax;
        for (int i = 0; i < 4; ++i) q[i] = round_scaled_to_i8(v[i], inv);
    }
    int part = q[0] + q[1] + q[2] + q[3];
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    if (!live) return;
    uint32_t packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                      ((uint32_t)(q[3] & 255) << 24);
    *reinterpret_cast<uint32_t *>(&out[blk].qs[4 * l]) = packed;
    if ((l & 3) == 0) out[blk].bsums[l >> 2] = (int16_t)part;
    if (l == 0) out[blk].d = zero ? 0.0f : amax / 127.0f;
}

jk_status launch_quantize_q8_k(hipStream_t s, const float *x, size_t nblocks, jk_block_q8k *out) {
    const size_t threads = nblocks * 64;
    hipLaunchKernelGGL(quantize_q8_k_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, nblocks, out);
    return check_launch("quantize_q8_k_kernel");
}

// QuantizedActQ8::quantize_into (repack.rs:542-650) for one (row, 32-block) per thread:
// quantize_block32_scalar (repack.rs:175-204) with its sequential +0.0-started sum, and
// the two x_sums_16 entries of the block as Rust `.sum()` folds (from -0.0).
__global__ __launch_bounds__(256) void quantize_act_q8_kernel(const float *__restrict__ x, jk_act_q8 a) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.m * a.k_blocks32) return;
    const size_t row = idx / a.k_blocks32, b = idx % a.k_blocks32;
    const float *src = x + row * a.k;
    float clean[32];
    float absmax = 0.0f, sum = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const size_t e = b * 32 + i;
        const float v = e < a.k ? src[e] : 0.0f;
        clean[i] = __builtin_isfinite(v) ? v : 0.0f;
        sum += clean[i];
        const float av = fabsf(clean[i]);
        if (av > absmax) absmax = av;
    }
    uint32_t packed[8];
    float scale = 0.0f;
    if (absmax < 1e-30f) {
        for (int i = 0; i < 8; ++i) packed[i] = 0;
    } else {
        const float inv = 127.0f / absmax;
        scale = absmax / 127.0f;
        for (int i = 0; i < 8; ++i) {
            uint32_t p = 0;
            for (int j = 0; j < 4; ++j)
                p |= (uint32_t)(rust_round_clamp_i8(clean[4 * i + j] * inv, -127.0f, 127.0f) & 255) << (8 * j);
            packed[i] = p;
        }
    }
    uint4 *dq = reinterpret_cast<uint4 *>(a.qs + row * a.k_padded + b * 32);
    dq[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dq[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    a.scales[row * a.k_blocks32 + b] = scale;
    a.sums[row * a.k_blocks32 + b] = sum;
    for (int h = 0; h < 2; ++h) {
        float s16 = -0.0f;
        for (int i = 0; i < 16; ++i) s16 += clean[16 * h + i];
        a.sums16[row * a.k_chunks + 2 * b + h] = s16;
    }
}

// super_scales_256 (repack.rs:612-621): max of the block scales of each 256-superblock,
// starting from 0.0.
__global__ __launch_bounds__(256) void act_super_kernel(jk_act_q8 a) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.m * a.sb256) return;
    const size_t row = idx / a.sb256, sb = idx % a.sb256;
    float mx = 0.0f;
    for (size_t b = sb * 8; b < sb * 8 + 8 && b < a.k_blocks32; ++b) {
        const float sc = a.scales[row * a.k_blocks32 + b];
        if (sc > mx) mx = sc;
    }
    a.super256[idx] = mx;
}

jk_status launch_quantize_act_q8(hipStream_t s, const float *x, const jk_act_q8 &a) {
    const size_t n = a.m * a.k_blocks32;
    hipLaunchKernelGGL(quantize_act_q8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, a);
    JK_TRY(check_launch("quantize_act_q8_kernel"));
    const size_t n2 = a.m * a.sb256;
    hipLaunchKernelGGL(act_super_kernel, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, s, a);
    return check_launch("act_super_kernel");
}

// subln_quantize_absmax_i8 (lib.rs:1042-1101) per row; norm_w == nullptr gives the same
// recipe without the RMSNorm step (x_norm = x). One workgroup per row.
__global__ __launch_bounds__(256) void absmax_i8_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                        size_t k, float eps, int8_t *__restrict__ q,
                                                        float *__restrict__ scales) {
    __shared__ float s_inv;
    __shared__ float s_max[4];
    const size_t row = blockIdx.x;
    const float *src = x + row * k;
    const int t = threadIdx.x;
    if (nw) {
        if (t == 0) {
            // dot_product_f32_scalar(input, input) (lib.rs:770-778): sequential from +0.0
            float sum_sq = 0.0f;
            for (size_t i = 0; i < k; ++i) sum_sq += src[i] * src[i];
            const float mean_sq = sum_sq / (float)k;
            s_inv = 1.0f / sqrtf(mean_sq + eps);
        }
        __syncthreads();
    }
    const float inv = nw ? s_inv : 1.0f;
    float mx = 0.0f;
    for (size_t i = t; i < k; i += 256) {
        const float xn = nw ? src[i] * inv * nw[i] : src[i];
        const float av = fabsf(xn);
        if (av > mx) mx = av;
    }
    mx = wave_max<64>(mx);
    if ((t & 63) == 0) s_max[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    int8_t *dst = q + row * k;
    if (__builtin_isnan(mx) || mx < 1e-12f) {
        for (size_t i = t; i < k; i += 256) dst[i] = 0;
        if (t == 0) scales[row] = 1.0f / 127.0f;
        return;
    }
    const float scale = mx / 127.0f;
    for (size_t i = t; i < k; i += 256) {
        const float xn = nw ? src[i] * inv * nw[i] : src[i];
        dst[i] = (int8_t)rust_round_clamp_i8(xn / scale, -128.0f, 127.0f);
    }
    if (t == 0) scales[row] = scale;
}

jk_status launch_absmax_i8(hipStream_t s, const float *x, const float *norm_w, size_t m, size_t k, float eps,
                           int8_t *q, float *scales) {
    hipLaunchKernelGGL(absmax_i8_kernel, dim3((unsigned)m), dim3(256), 0, s, x, norm_w, k, eps, q, scales);
    return check_launch("absmax_i8_kernel");
}

}  // namespace jk
