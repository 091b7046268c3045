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
// bsums[j] = sum of the 16 quants of lanes 4j..4j+3. With ACT != 0 the input element is the
// gated activation gated<ACT>(x[i], up[i]) (SwiGLU or ReLU^2), computed in the load. V4: the inputs
// are 16-byte aligned and a lane reads its four elements with one load each. The block maximum and
// the bsums are DPP reductions (a maximum and an integer sum: exact in any order), with no LDS
// round trip on the launch's critical path.
template <int ACT, bool V4>
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float *__restrict__ x, const float *__restrict__ up,
                                                            size_t nblocks, jk_block_q8k *__restrict__ out) {
    const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int l = threadIdx.x & 63;
    const bool live = blk < nblocks;
    const size_t e0 = min(blk, nblocks - 1) * 256 + 4 * l;  // (clamped: in bounds for every lane)
    float g[4], u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (V4) {
        const float4 gv = *reinterpret_cast<const float4 *>(x + e0);
        g[0] = gv.x, g[1] = gv.y, g[2] = gv.z, g[3] = gv.w;
        if constexpr (ACT != 0) {
            const float4 uv = *reinterpret_cast<const float4 *>(up + e0);
            u[0] = uv.x, u[1] = uv.y, u[2] = uv.z, u[3] = uv.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g[i] = x[e0 + i];
            if constexpr (ACT != 0) u[i] = up[e0 + i];
        }
    }
    float v[4];
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = live ? gated<ACT>(g[i], u[i]) : 0.0f;
        a = fmaxf(a, __builtin_isfinite(v[i]) ? fabsf(v[i]) : 0.0f);
    }
    const float amax = wave_max64_dpp(a);
    int q[4] = {0, 0, 0, 0};
    const bool zero = amax == 0.0f || !__builtin_isfinite(amax);
    if (!zero) {
        const float inv = 127.0f / amax;
        for (int i = 0; i < 4; ++i) q[i] = round_scaled_to_i8(v[i], inv);
    }
    const int part = sum4_dpp(q[0] + q[1] + q[2] + q[3]);
    if (!live) return;
    uint32_t packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                      ((uint32_t)(q[3] & 255) << 24);
    *reinterpret_cast<uint32_t *>(&out[blk].qs[4 * l]) = packed;
    if ((l & 3) == 0) out[blk].bsums[l >> 2] = (int16_t)part;
    if (l == 0) out[blk].d = zero ? 0.0f : amax / 127.0f;
}

jk_status launch_quantize_q8_k(hipStream_t s, const float *x, size_t nblocks, jk_block_q8k *out) {
    return launch_quantize_q8_k_gated(s, kActNone, x, nullptr, nblocks, out);
}

jk_status launch_quantize_q8_k_gated(hipStream_t s, int act, const float *x, const float *up, size_t nblocks,
                                     jk_block_q8k *out) {
    const dim3 grid((unsigned)((nblocks * 64 + 255) / 256)), block(256);
    const bool v4 = (uintptr_t)x % 16 == 0 && (act == kActNone || (uintptr_t)up % 16 == 0);
    if (act == kActSwiglu) {
        if (v4) hipLaunchKernelGGL((quantize_q8_k_kernel<kActSwiglu, true>), grid, block, 0, s, x, up, nblocks, out);
        else hipLaunchKernelGGL((quantize_q8_k_kernel<kActSwiglu, false>), grid, block, 0, s, x, up, nblocks, out);
    } else if (act == kActRelu2) {
        if (v4) hipLaunchKernelGGL((quantize_q8_k_kernel<kActRelu2, true>), grid, block, 0, s, x, up, nblocks, out);
        else hipLaunchKernelGGL((quantize_q8_k_kernel<kActRelu2, false>), grid, block, 0, s, x, up, nblocks, out);
    } else {
        if (v4) hipLaunchKernelGGL((quantize_q8_k_kernel<kActNone, true>), grid, block, 0, s, x, up, nblocks, out);
        else hipLaunchKernelGGL((quantize_q8_k_kernel<kActNone, false>), grid, block, 0, s, x, up, nblocks, out);
    }
    return check_launch("quantize_q8_k_kernel");
}

// Ordered f32 fold of N consecutive lanes (N = 4 or 8) that hold four values each, in
// element order: lane j of the group computes (((prev + v0) + v1) + v2) + v3 where prev is
// lane j-1's result (init for j == 0). After N steps lane N-1 holds the group's fold.
template <int N>
__device__ __forceinline__ float lane_chain(const float (&v)[4], float init) {
    const int j = (int)(threadIdx.x & (N - 1));
    float run = init;
#pragma unroll
    for (int step = 0; step < N; ++step) {
        const float prev = __shfl_up(run, 1, N);  // lane j - 1 of the group (lane 0 keeps its own)
        const float base = j == 0 ? init : prev;
        const float r = (((base + v[0]) + v[1]) + v[2]) + v[3];
        run = j == step ? r : run;
    }
    return run;
}

// QuantizedActQ8::quantize_into (repack.rs:542-650): one wave per (row, 256-element
// superblock), lane l holding elements 4l..4l+3 (coalesced loads), 8 lanes per 32-block.
// Per block, quantize_block32_scalar (repack.rs:175-204): non-finite -> 0, absmax over the
// block (zero block below 1e-30), scale = absmax / 127, q = round(x * 127 / absmax) clamped
// to +-127, and the sequential sum from +0.0; the two x_sums_16 entries are Rust `.sum()`
// folds from -0.0; super_scales_256 (repack.rs:612-621) is the max of the superblock's
// block scales from 0.0. Elements past k (the zero-padded tail) take part as +0.0. With ACT != 0
// the element is the gated activation gated<ACT>(x, up) of the two input rows.
template <bool V4, int ACT>
__global__ __launch_bounds__(256) void quantize_act_q8_kernel(const float *__restrict__ x, const float *__restrict__ up,
                                                              jk_act_q8 a) {
    const size_t wv = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (wv >= a.m * a.sb256) return;  // wave-uniform
    const int l = (int)(threadIdx.x & 63);
    const size_t row = wv / a.sb256, sb = wv % a.sb256;
    const size_t e0 = sb * 256 + 4 * (size_t)l;
    const float *src = x + row * a.k;
    const float *usrc = ACT ? up + row * a.k : nullptr;
    float v[4];
    if constexpr (V4) {
        if (e0 + 3 < a.k) {
            const float4 f = *reinterpret_cast<const float4 *>(src + e0);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
            if constexpr (ACT != kActNone) {
                const float4 u = *reinterpret_cast<const float4 *>(usrc + e0);
                v[0] = gated<ACT>(v[0], u.x); v[1] = gated<ACT>(v[1], u.y);
                v[2] = gated<ACT>(v[2], u.z); v[3] = gated<ACT>(v[3], u.w);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = e0 + i < a.k ? gated<ACT>(src[e0 + i], ACT ? usrc[e0 + i] : 0.0f) : 0.0f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = e0 + i < a.k ? gated<ACT>(src[e0 + i], ACT ? usrc[e0 + i] : 0.0f) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_isfinite(v[i]) ? v[i] : 0.0f;
    const float absmax = max8_dpp(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const bool zero = absmax < 1e-30f;
    const float inv = zero ? 0.0f : 127.0f / absmax;
    const float scale = zero ? 0.0f : absmax / 127.0f;
    uint32_t packed = 0;
    if (!zero) {
#pragma unroll
        for (int i = 0; i < 4; ++i) packed |= (uint32_t)(rust_round_clamp_i8(v[i] * inv, -127.0f, 127.0f) & 255) << (8 * i);
    }
    const float sum = lane_chain<8>(v, 0.0f);
    const float s16 = lane_chain<4>(v, -0.0f);
    // superblock max of the block scales (lanes 8b hold block b's scale), from 0.0
    float mx = fmaxf(0.0f, scale);
    mx = fmaxf(mx, __shfl_xor(mx, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));

    const size_t b = sb * 8 + (size_t)(l >> 3);
    if (b < a.k_blocks32) {
        *reinterpret_cast<uint32_t *>(a.qs + row * a.k_padded + e0) = packed;
        const int j = l & 7;
        if (j == 0) a.scales[row * a.k_blocks32 + b] = scale;
        if (j == 7) a.sums[row * a.k_blocks32 + b] = sum;
        if ((l & 3) == 3) a.sums16[row * a.k_chunks + 2 * b + (j >> 2)] = s16;
    }
    if (l == 0) a.super256[row * a.sb256 + sb] = mx;
}

template <int ACT>
static void launch_act_q8(hipStream_t s, const float *x, const float *up, const jk_act_q8 &a) {
    const size_t waves = a.m * a.sb256;
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    const bool v4 = (a.k & 3) == 0 && ((uintptr_t)x & 15) == 0 && (!ACT || ((uintptr_t)up & 15) == 0);
    if (v4) hipLaunchKernelGGL((quantize_act_q8_kernel<true, ACT>), grid, block, 0, s, x, up, a);
    else hipLaunchKernelGGL((quantize_act_q8_kernel<false, ACT>), grid, block, 0, s, x, up, a);
}

jk_status launch_quantize_act_q8(hipStream_t s, const float *x, const jk_act_q8 &a) {
    return launch_quantize_act_q8_gated(s, kActNone, x, nullptr, a);
}

jk_status launch_quantize_act_q8_gated(hipStream_t s, int act, const float *x, const float *up, const jk_act_q8 &a) {
    if (act == kActSwiglu) launch_act_q8<kActSwiglu>(s, x, up, a);
    else if (act == kActRelu2) launch_act_q8<kActRelu2>(s, x, up, a);
    else launch_act_q8<kActNone>(s, x, up, a);
    return check_launch("quantize_act_q8_kernel");
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
