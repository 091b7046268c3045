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
#include <type_traits>

#include "jk_device.hpp"

namespace jk {

// ----------------------------------------------------------- f32-activation matvec
// vec_dot_{q4_0,q8_0,q6_k}_scalar (quant.rs:1401-1436, 899-934, 1012-1047),
// vec_dot_q4_k_m_scalar (lib.rs:1268-1303), vec_dot_q5_k_scalar (quant.rs:1181-1219),
// vec_dot_q5_0 -> vec_dot_generic_block (quant.rs:2036-2054, 1995-2029), vec_dot_i2_s
// (quant.rs:2199-2240): for each block, dot_product_f32_scalar(dequantized block, x block)
// (lib.rs:770-778) -- one product and one add per element in element order from +0.0 --
// and row_sum (from +0.0) adds the block dots in block order.
//
// Mapping: lane p of a row's LPR lanes takes blocks p, p + LPR, ...; a block's element
// chain runs in the lane, fully unrolled, on the block's bytes held in registers (16-byte
// plane loads) and the activation staged once per workgroup in LDS (or read through the
// caches when it does not fit); the block values are folded across lanes in block order.
template <int Q> struct VdFmt {
    static constexpr int E = fmt_of(Q).be;         // elements
    static constexpr int C = fmt_of(Q).chunks;     // 16-byte chunks
    static constexpr bool D = fmt_of(Q).d_off >= 0;  // f16 scale in the d-plane
    static constexpr bool H = fmt_of(Q).h_off >= 0;  // field in the word plane
};

template <int Q> struct VdBlock {
    uint4 c[VdFmt<Q>::C];
    uint32_t d;
    uint32_t h[2];
};

template <int Q>
__device__ __forceinline__ void vd_load(VdBlock<Q> &o, const WeightDev &w, int r, int b) {
#pragma unroll
    for (int c = 0; c < VdFmt<Q>::C; ++c) o.c[c] = ld_chunk(w, c, r, b);
    if constexpr (VdFmt<Q>::D) o.d = w.dplane[(size_t)r * (size_t)w.nb + (size_t)b];
    if constexpr (VdFmt<Q>::H)
#pragma unroll
        for (int i = 0; i < fmt_of(Q).h_len / 4; ++i) o.h[i] = ld_word(w, r, b, fmt_of(Q).h_len, i);
}

// Byte k (0..15 within chunk c) of the block's chunks.
template <int Q>
__device__ __forceinline__ uint32_t vd_byte(const VdBlock<Q> &o, int c, int k) {
    return (comp(o.c[c], k >> 2) >> (8 * (k & 3))) & 255u;
}

// The block's element products: added one after another from +0.0 (the reference's
// dot_product_f32_scalar), or, in tolerance mode, spread over four accumulators with fused
// multiply-adds (the chain a lane runs is a quarter as long) and added at the end.
struct VdSum {
    float s = 0.0f;
    __device__ __forceinline__ void add(float w, float x) { s += w * x; }
    __device__ __forceinline__ float get() const { return s; }
};
struct VdSumTol {
    float a = 0.0f, b = 0.0f, c = 0.0f, d = 0.0f;
    __device__ __forceinline__ void add(float w, float x) {  // (the rotation is register renaming once unrolled)
        const float n = __builtin_fmaf(w, x, a);
        a = b, b = c, c = d, d = n;
    }
    __device__ __forceinline__ float get() const { return (a + b) + (c + d); }
};

// NP > 1 (tolerance mode only): the products of part PART of NP equal runs of the block's
// elements; every element index below is a constant once unrolled, so the other parts' work
// (their dequantization and, where unused, their loads) is not emitted.
template <int Q, bool TOL = false, int NP = 1, int PART = 0>
__device__ __forceinline__ float vd_block(const VdBlock<Q> &o, const float *__restrict__ xb, float i2s_scale) {
    static_assert(NP == 1 || TOL, "a block's elements split over lanes only in tolerance mode");
    std::conditional_t<TOL, VdSumTol, VdSum> sum;
    auto add = [&](float wv, int idx) {
        if (NP == 1 || idx * NP / VdFmt<Q>::E == PART) sum.add(wv, xb[idx]);
    };
    if constexpr (Q == JK_Q4_0 || Q == JK_Q5_0 || Q == JK_Q8_0) {
        // dequantize_q4_0_block / dequantize_q8_0_block (quant.rs:550-588), dequantize_q5_0_block
        // (160-164, scale_i8_into_f32 94-102). The reference writes +0.0 for d == 0 where d * q
        // gives +-0: no sum observes the difference, since a sum that starts at +0.0 never
        // becomes -0 under round-to-nearest addition (the products are finite, so NaN cases
        // are unchanged as well).
        const float d = f16_finite(o.d);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int qv;
            if constexpr (Q == JK_Q4_0) qv = (int)((vd_byte<Q>(o, 0, i & 15) >> (i < 16 ? 0 : 4)) & 15u) - 8;
            else if constexpr (Q == JK_Q5_0)
                qv = (int)(((vd_byte<Q>(o, 0, i & 15) >> (i < 16 ? 0 : 4)) & 15u) | (((o.h[0] >> i) & 1u) << 4)) - 16;
            else qv = (int)(int8_t)vd_byte<Q>(o, i >> 4, i & 15);
            const float wv = d * (float)qv;
            add(wv, i);
        }
    } else if constexpr (Q == JK_Q4_K) {
        // dequantize_q4_k_m_block (lib.rs:720-766): y = d1 * q - m1, two roundings
        const uint4 h = o.c[0];
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t scv = c < 2 ? sc_lo : sc_hi, mv = c < 2 ? m_lo : m_hi;
            const int j = (2 * c) & 3;
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
                const float d1 = d * (float)byte_of(scv, j + hi), m1 = dmin * (float)byte_of(mv, j + hi);
#pragma unroll
                for (int l = 0; l < 32; ++l) {
                    const uint32_t q = (vd_byte<Q>(o, 1 + 2 * c + (l >> 4), l & 15) >> (4 * hi)) & 15u;
                    const float wv = d1 * (float)q - m1;
                    add(wv, 64 * c + 32 * hi + l);
                }
            }
        }
    } else if constexpr (Q == JK_Q4_1 || Q == JK_Q5_1) {
        // dequantize_q4_1_block / dequantize_q5_1_block (quant.rs:132-136, 190-195) via
        // affine_i8_into_f32 (104-113): d * q + m, or +0.0 when d and m are both zero
        const float d = f16_finite(o.h[0] & 0xFFFFu), m = f16_finite(o.h[0] >> 16);
        const bool z = d == 0.0f && m == 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            uint32_t q = (vd_byte<Q>(o, 0, i & 15) >> (i < 16 ? 0 : 4)) & 15u;
            if constexpr (Q == JK_Q5_1) q |= ((o.h[1] >> i) & 1u) << 4;
            const float wv = z ? 0.0f : d * (float)q + m;
            add(wv, i);
        }
    } else if constexpr (Q == JK_IQ4_NL) {
        // dequantize_iq4_nl_block (quant.rs:348-356): d * KVALUES_IQ4NL[nibble] (+0.0 for d == 0,
        // which no sum from +0.0 observes, as above)
        const float d = f16_finite(o.d);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = iq4nl_lookup(comp(o.c[0], k) & 0x0F0F0F0Fu);
#pragma unroll
            for (int i = 0; i < 4; ++i) add((d * (float)(int8_t)(lo >> (8 * i))), 4 * k + i);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t hi = iq4nl_lookup((comp(o.c[0], k) >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int i = 0; i < 4; ++i) add((d * (float)(int8_t)(hi >> (8 * i))), 16 + 4 * k + i);
        }
    } else if constexpr (Q == JK_Q2_K) {
        // dequantize_q2_k_block (quant.rs:238-252): element 128 half + 32 j + 16 part + l is the
        // 2-bit field 2j of qs byte 32 half + 16 part + l, times d * (sc & 15), minus dmin * (sc >> 4)
        const float d = f16_finite(o.h[0] & 0xFFFFu), dmin = f16_finite(o.h[0] >> 16);
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const uint32_t sc = vd_byte<Q>(o, 0, g);
            const float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
            const int half = g >> 3, j = (g >> 1) & 3, part = g & 1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t v = (comp(o.c[1 + 2 * half + part], k) >> (2 * j)) & 0x03030303u;
#pragma unroll
                for (int i = 0; i < 4; ++i) add((dl * (float)((v >> (8 * i)) & 3u) - ml), 16 * g + 4 * k + i);
            }
        }
    } else if constexpr (Q == JK_Q3_K) {
        // dequantize_q3_k_block (quant.rs:320-331): element 128 half + 32 j + 16 part + l is the
        // 2-bit field 2j of qs byte 32 half + 16 part + l, minus 4 when bit 4 half + j of hmask
        // byte 16 part + l is clear, times d * (scale - 32)
        const uint4 tail = o.c[6];
        const float d = f16_finite(tail.w & 0xFFFFu);
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const uint32_t lo = g < 8 ? (vd_byte<Q>(o, 6, g) & 15u) : (vd_byte<Q>(o, 6, g - 8) >> 4);
            const uint32_t hi = (vd_byte<Q>(o, 6, 8 + (g & 3)) >> (2 * (g >> 2))) & 3u;
            const float dl = d * (float)((int)(lo | (hi << 4)) - 32);
            const int half = g >> 3, j = (g >> 1) & 3, part = g & 1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t v = (comp(o.c[2 + 2 * half + part], k) >> (2 * j)) & 0x03030303u;
                const uint32_t h = (comp(o.c[part], k) >> (4 * half + j)) & 0x01010101u;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qv = (int)((v >> (8 * i)) & 3u) - ((h >> (8 * i)) & 1u ? 0 : 4);
                    add((dl * (float)qv), 16 * g + 4 * k + i);
                }
            }
        }
    } else if constexpr (Q == JK_Q5_K) {
        // dequantize_q5_k_block (quant.rs:651-706): y = d1 * q - m1 with q = nibble + 16 * bit.
        // Its d == 0 && dmin == 0 -> +0.0 case gives +-0 products here, which no sum from
        // +0.0 observes (as for Q4_0 above).
        const uint4 h = o.c[0];
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t scv = c < 2 ? sc_lo : sc_hi, mv = c < 2 ? m_lo : m_hi;
            const int j = (2 * c) & 3;
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
                const float d1 = d * (float)byte_of(scv, j + hi), m1 = dmin * (float)byte_of(mv, j + hi);
#pragma unroll
                for (int l = 0; l < 32; ++l) {
                    const uint32_t q = ((vd_byte<Q>(o, 3 + 2 * c + (l >> 4), l & 15) >> (4 * hi)) & 15u) |
                                       (((vd_byte<Q>(o, 1 + (l >> 4), l & 15) >> (2 * c + hi)) & 1u) << 4);
                    const float wv = d1 * (float)q - m1;
                    add(wv, 64 * c + 32 * hi + l);
                }
            }
        }
    } else if constexpr (Q == JK_Q6_K) {
        // dequantize_q6_k_block (quant.rs:594-648) visited in element order: (d * sc) * q
        // (its d == 0 -> +0.0 case needs no select, as for Q4_0 above)
        // Four elements at a time: bytes of 4 (q - 32) (the 6-bit field with its top bit
        // flipped, moved to the top of the byte, read back as a signed byte), times dsc / 4.
        // dsc / 4 is exact (|d * sc| is 0 or at least 2^-24) and so is 4 (q - 32), so the
        // product is dsc * (q - 32) rounded once, as in the reference.
        const float d = f16_finite(o.d);
        float dsc4[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) dsc4[j] = (d * (float)(int8_t)vd_byte<Q>(o, 12, j)) * 0.25f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int quarter = 0; quarter < 4; ++quarter) {
#pragma unroll
                for (int l = 0; l < 32; l += 4) {
                    const int lbyte = 64 * h + l + ((quarter & 1) ? 32 : 0), qbyte = 32 * h + l;
                    const uint32_t L = comp(o.c[lbyte >> 4], (lbyte & 15) >> 2);
                    const uint32_t H = comp(o.c[8 + (qbyte >> 4)], (qbyte & 15) >> 2);
                    const uint32_t v6 = ((L >> (quarter < 2 ? 0 : 4)) & 0x0F0F0F0Fu) | (((H >> (2 * quarter)) & 0x03030303u) << 4);
                    const uint32_t w4 = (v6 ^ 0x20202020u) << 2;
                    const float s4 = dsc4[8 * h + (l >> 4) + 2 * quarter];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float wv = s4 * (float)(int8_t)(w4 >> (8 * i));
                        add(wv, 128 * h + 32 * quarter + l + i);
                    }
                }
                // the chain is serial: an empty asm with a memory clobber keeps the next 32
                // activation reads from being hoisted ahead of this group (bounded live range)
                __asm__ volatile("" ::: "memory");
            }
    } else {  // JK_I2_S: dequantize_i2_s_block (quant.rs:380-387), (scale * t) * x
#pragma unroll
        for (int e = 0; e < 128; ++e) {
            const int grp = e >> 5, g = e & 31;
            const int t = (int)((vd_byte<Q>(o, g >> 4, g & 15) >> (6 - 2 * grp)) & 3u) - 1;
            add((i2s_scale * (float)t), e);
        }
    }
    return sum.get();
}

constexpr int kVdWaves = 8;
constexpr int kVdLdsMax = 60 * 1024;  // staged activation bytes

template <int Q, int LPR, bool XL, bool TOL = false>
__global__ __launch_bounds__(64 * kVdWaves) __attribute__((amdgpu_waves_per_eu(4))) void vec_dot_f32_kernel(WeightDev w, const float *__restrict__ x,
                                                                     float *__restrict__ y) {
    constexpr int RPW = 64 / LPR, E = VdFmt<Q>::E;
    extern __shared__ __align__(16) float s_xf[];
    __shared__ __align__(16) float s_red[LPR == 64 ? kVdWaves : 1][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane / LPR, p = lane % LPR;
    const int row = ((int)blockIdx.x * kVdWaves + wave) * RPW + sub;
    const int r = min(row, w.rows - 1);
    const int nb = w.nb, iters = (nb + LPR - 1) / LPR;
    if (Q == JK_I2_S && w.tensor_scale == 0.0f) {  // zero trailer scale: all outputs 0 (quant.rs:2219)
        if (row < w.rows && p == 0) y[row] = 0.0f;
        return;
    }
    VdBlock<Q> blk;
    vd_load<Q>(blk, w, r, min(p, nb - 1));
    // Staged blocks are padded by 16 bytes (XS floats apart) so that the 16-byte reads of
    // 16 lanes, each in its own block, fall on distinct LDS banks.
    constexpr int XS = XL ? E + 4 : E;
    const float *xs = x;
    if constexpr (XL) {
        const int n4 = w.cols / 4;
        for (int i = tid; i < n4; i += 64 * kVdWaves)
            reinterpret_cast<float4 *>(s_xf)[i + i / (E / 4)] = reinterpret_cast<const float4 *>(x)[i];
        __syncthreads();
        xs = s_xf;
    }
    float *red = s_red[LPR == 64 ? wave : 0];
    float acc = 0.0f;
    for (int it = 0; it < iters; ++it) {
        const int b = it * LPR + p;
        if (it > 0) vd_load<Q>(blk, w, r, min(b, nb - 1));
        const float v = b < nb ? vd_block<Q, TOL>(blk, xs + (size_t)XS * min(b, nb - 1), w.tensor_scale) : -0.0f;
        if constexpr (LPR == 16) acc = chain_add(acc, v);
        else acc = fold_wave(acc, v, red);
    }
    const int writer = LPR == 16 ? 15 : 0;
    if (row < w.rows && p == writer) y[row] = acc;
}

// Tolerance mode for rows of at most 32 blocks: the lane mapping of the 16-lane kernel (16 lanes
// per row, lane p on blocks p and p + 16), with each block's elements split in four runs over
// four waves of the workgroup (wave w: run w % 4). A lane's chain is a quarter as long and the
// launch has four times the waves (Q4_K 4096 rows: 4096 waves instead of 1024 on 128 of the
// CUs). The 16 lanes of a row and the four runs are added in any order (shuffles, then LDS).
constexpr int kVdParts = 4;
constexpr int kVdPartRows = kVdWaves / kVdParts * 4;  // rows per workgroup

// One wave's share: the runs PART of the blocks of its lanes (one or two blocks a lane), summed
// over the 16 lanes of each row into s_part.
template <int Q, int PART>
__device__ __forceinline__ void vd_parts_wave(const WeightDev &w, const float *xs, int xstride, int r, int p, int sub,
                                              float *s_part_wave) {
    const int nb = w.nb;
    VdBlock<Q> b0, b1;
    vd_load<Q>(b0, w, r, min(p, nb - 1));
    if (nb > 16) vd_load<Q>(b1, w, r, min(16 + p, nb - 1));
    float v = p < nb ? vd_block<Q, true, kVdParts, PART>(b0, xs + (size_t)xstride * p, w.tensor_scale) : 0.0f;
    if (nb > 16 && 16 + p < nb)
        v += vd_block<Q, true, kVdParts, PART>(b1, xs + (size_t)xstride * (16 + p), w.tensor_scale);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 16);
    if (p == 0) s_part_wave[sub] = v;
}

template <int Q, bool XL>
__global__ __launch_bounds__(64 * kVdWaves) __attribute__((amdgpu_waves_per_eu(4))) void vec_dot_f32_parts_kernel(
    WeightDev w, const float *__restrict__ x, float *__restrict__ y) {
    constexpr int E = VdFmt<Q>::E, XS = XL ? E + 4 : E;
    extern __shared__ __align__(16) float s_xf[];
    __shared__ float s_part[kVdWaves][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int part = wave % kVdParts, grp = wave / kVdParts;
    const int sub = lane >> 4, p = lane & 15;
    const int row0 = (int)blockIdx.x * kVdPartRows;
    const int r = min(row0 + 4 * grp + sub, w.rows - 1);
    if (Q == JK_I2_S && w.tensor_scale == 0.0f) {  // zero trailer scale: all outputs 0 (quant.rs:2219)
        if (tid < kVdPartRows && row0 + tid < w.rows) y[row0 + tid] = 0.0f;
        return;
    }
    const float *xs = x;
    if constexpr (XL) {
        const int n4 = w.cols / 4;
        for (int i = tid; i < n4; i += 64 * kVdWaves)
            reinterpret_cast<float4 *>(s_xf)[i + i / (E / 4)] = reinterpret_cast<const float4 *>(x)[i];
        __syncthreads();
        xs = s_xf;
    }
    switch (part) {  // wave-uniform
    case 0: vd_parts_wave<Q, 0>(w, xs, XS, r, p, sub, s_part[wave]); break;
    case 1: vd_parts_wave<Q, 1>(w, xs, XS, r, p, sub, s_part[wave]); break;
    case 2: vd_parts_wave<Q, 2>(w, xs, XS, r, p, sub, s_part[wave]); break;
    default: vd_parts_wave<Q, 3>(w, xs, XS, r, p, sub, s_part[wave]); break;
    }
    __syncthreads();
    if (tid < kVdPartRows && row0 + tid < w.rows) {
        const int g = tid >> 2, sr = tid & 3;
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < kVdParts; ++k) t += s_part[g * kVdParts + k][sr];
        y[row0 + tid] = t;
    }
}

template <int Q, bool TOL>
static jk_status launch_vd(hipStream_t s, const WeightDev &w, const float *x, float *y) {
    const size_t lds_need = (size_t)w.nb * (VdFmt<Q>::E + 4) * 4;  // padded blocks
    const bool xl = lds_need <= (size_t)kVdLdsMax;
    const size_t lds = xl ? lds_need : 0;
    if (TOL && w.nb <= 32) {
        const dim3 grid((unsigned)((w.rows + kVdPartRows - 1) / kVdPartRows));
        if (xl) hipLaunchKernelGGL((vec_dot_f32_parts_kernel<Q, true>), grid, dim3(64 * kVdWaves), lds, s, w, x, y);
        else hipLaunchKernelGGL((vec_dot_f32_parts_kernel<Q, false>), grid, dim3(64 * kVdWaves), 0, s, w, x, y);
    } else if (w.nb > 32) {
        const dim3 grid((unsigned)((w.rows + kVdWaves - 1) / kVdWaves));
        if (xl) hipLaunchKernelGGL((vec_dot_f32_kernel<Q, 64, true, TOL>), grid, dim3(64 * kVdWaves), lds, s, w, x, y);
        else hipLaunchKernelGGL((vec_dot_f32_kernel<Q, 64, false, TOL>), grid, dim3(64 * kVdWaves), 0, s, w, x, y);
    } else {
        const dim3 grid((unsigned)((w.rows + 4 * kVdWaves - 1) / (4 * kVdWaves)));
        if (xl) hipLaunchKernelGGL((vec_dot_f32_kernel<Q, 16, true, TOL>), grid, dim3(64 * kVdWaves), lds, s, w, x, y);
        else hipLaunchKernelGGL((vec_dot_f32_kernel<Q, 16, false, TOL>), grid, dim3(64 * kVdWaves), 0, s, w, x, y);
    }
    return check_launch("vec_dot_f32_kernel");
}

template <bool TOL>
static jk_status launch_vec_dot_f32_mode(hipStream_t s, const WeightDev &w, const float *x, float *y) {
    switch (w.quant) {
    case JK_Q4_0: return launch_vd<JK_Q4_0, TOL>(s, w, x, y);
    case JK_Q5_0: return launch_vd<JK_Q5_0, TOL>(s, w, x, y);
    case JK_Q8_0: return launch_vd<JK_Q8_0, TOL>(s, w, x, y);
    case JK_Q4_K: return launch_vd<JK_Q4_K, TOL>(s, w, x, y);
    case JK_Q5_K: return launch_vd<JK_Q5_K, TOL>(s, w, x, y);
    case JK_Q4_1: return launch_vd<JK_Q4_1, TOL>(s, w, x, y);
    case JK_Q5_1: return launch_vd<JK_Q5_1, TOL>(s, w, x, y);
    case JK_IQ4_NL: return launch_vd<JK_IQ4_NL, TOL>(s, w, x, y);
    case JK_Q2_K: return launch_vd<JK_Q2_K, TOL>(s, w, x, y);
    case JK_Q3_K: return launch_vd<JK_Q3_K, TOL>(s, w, x, y);
    case JK_Q6_K: return launch_vd<JK_Q6_K, TOL>(s, w, x, y);
    case JK_I2_S: return launch_vd<JK_I2_S, TOL>(s, w, x, y);
    default: return fail(JK_CAPABILITY_MISMATCH, "vec_dot_f32: unsupported quant %d", w.quant);
    }
}

jk_status launch_vec_dot_f32(hipStream_t s, const WeightDev &w, const float *x, float *y) {
    return launch_vec_dot_f32_mode<false>(s, w, x, y);
}

jk_status launch_vec_dot_f32_tol(hipStream_t s, const WeightDev &w, const float *x, float *y) {
    return launch_vec_dot_f32_mode<true>(s, w, x, y);
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
        float v = -0.0f;
        if (p < nb - 16 * it) v = bl_block_value(w, r, 16 * it + p, a, as);
        acc = chain_add(acc, v);
    }
    if (active && p == 15) y[(size_t)m * (size_t)w.rows + row] = acc;
}

// The ternary formats for a few tokens: a workgroup of RW rows (16 lanes each, lane p takes
// blocks p, p + 16, ... as above) issues all its weight loads first, then stages its token's
// activation row in LDS -- each block padded by 16 bytes, so the 16 lanes of a row, which
// read 16 different blocks at the same offset, hit distinct banks -- and the activation sum
// of every block once, then evaluates. Same arithmetic and block order as bitlinear_kernel.
constexpr int kBlMaxBlocks = 64;  // blocks per row (4 per lane) handled here
template <int Q> constexpr int kBlBE = Q == JK_TQ2_0 ? 256 : 128;  // elements per block
template <int Q> constexpr int kBlC = Q == JK_TQ2_0 ? 4 : 2;       // 16-byte chunks per block

template <int Q, int UF, int RW>
__global__ __launch_bounds__(16 * RW) void bitlinear_ternary_kernel(WeightDev w, const int8_t *__restrict__ act,
                                                                   const float *__restrict__ act_scales,
                                                                   float *__restrict__ y) {
    constexpr int BE = kBlBE<Q>, C = kBlC<Q>, BS = BE + 16;  // LDS stride of a block
    extern __shared__ __align__(16) uint8_t s_a[];           // nb blocks of BS bytes, then nb sums
    const int tid = threadIdx.x, p = tid & 15;
    const int row = (int)blockIdx.x * RW + (tid >> 4), m = (int)blockIdx.y;
    const int nb = w.nb, r = min(row, w.rows - 1);
    int *s_sum = reinterpret_cast<int *>(s_a + nb * BS);

    // 1. weight loads (blocks past the row end re-read the last one and are never used)
    uint4 q[UF][C];
    uint32_t dq[UF];
#pragma unroll
    for (int k = 0; k < UF; ++k) {
        const int b = min(16 * k + p, nb - 1);
#pragma unroll
        for (int c = 0; c < C; ++c) q[k][c] = ld_chunk(w, c, r, b);
        if constexpr (Q == JK_TQ2_0) dq[k] = w.dplane[(size_t)r * (size_t)nb + (size_t)b];
    }
    // 2. the token's activation row, then the sum of every block
    const uint4 *a4 = reinterpret_cast<const uint4 *>(act + (size_t)m * (size_t)w.cols);
    for (int i = tid; i < w.cols / 16; i += 16 * RW)
        *reinterpret_cast<uint4 *>(s_a + 16 * i + 16 * (16 * i / BE)) = a4[i];
    lds_barrier();
    for (int b = tid; b < nb; b += 16 * RW) {
        const int *ab = reinterpret_cast<const int *>(s_a + b * BS);
        int sx = 0;
#pragma unroll
        for (int i = 0; i < BE / 4; ++i) sx = dot4(ab[i], 0x01010101, sx);
        s_sum[b] = sx;
    }
    lds_barrier();
    // 3. block values (unpack_bitlinear_block_i8 values times the activation), block order
    const float as = act_scales[m];
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < UF; ++k) {
        if (16 * k >= nb) break;  // wave-uniform
        const int b = 16 * k + p;
        float v = -0.0f;  // past the row end: the identity of the ordered fold
        if (b < nb) {
            const int *av = reinterpret_cast<const int *>(s_a + b * BS);
            int sw = 0;
            if constexpr (Q == JK_TQ2_0) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t wv = comp(q[k][i >> 2], i & 3);
#pragma unroll
                    for (int j = 0; j < 4; ++j) sw = dot4((int)((wv >> (2 * j)) & 0x03030303u), av[4 * i + j], sw);
                }
                v = (float)(sw - s_sum[b]) * (f16_finite(dq[k]) * as);
            } else {
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t wv = comp(q[k][c], i);
#pragma unroll
                        for (int grp = 0; grp < 4; ++grp)
                            sw = dot4((int)((wv >> (6 - 2 * grp)) & 0x03030303u), av[8 * grp + 4 * c + i], sw);
                    }
                v = (float)(sw - s_sum[b]) * (w.tensor_scale * as);
            }
        }
        acc = chain_add(acc, v);
    }
    if (row < w.rows && p == 15) y[(size_t)m * (size_t)w.rows + row] = acc;
}

template <int Q, int RW>
static jk_status launch_bl_ternary(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales,
                                   int m, float *y) {
    const dim3 grid((unsigned)((w.rows + RW - 1) / RW), (unsigned)m), block(16 * RW);
    const size_t lds = (size_t)w.nb * (kBlBE<Q> + 16) + (size_t)w.nb * 4;
    if (w.nb <= 16) JK_LAUNCH("bitlinear_ternary_kernel", (bitlinear_ternary_kernel<Q, 1, RW>), grid, block, lds, s, w, act, act_scales, y);
    else if (w.nb <= 32) JK_LAUNCH("bitlinear_ternary_kernel", (bitlinear_ternary_kernel<Q, 2, RW>), grid, block, lds, s, w, act, act_scales, y);
    else JK_LAUNCH("bitlinear_ternary_kernel", (bitlinear_ternary_kernel<Q, 4, RW>), grid, block, lds, s, w, act, act_scales, y);
    return check_launch("bitlinear_ternary_kernel");
}

jk_status launch_bitlinear(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales, int m,
                           float *y) {
    // 16-byte activation rows (cols is a multiple of the block size) and up to 64 blocks a row
    const bool ternary = w.quant == JK_TQ2_0 || w.quant == JK_I2_S;
    if (ternary && w.nb <= kBlMaxBlocks && (reinterpret_cast<uintptr_t>(act) & 15u) == 0) {
        // 8 rows a workgroup; 4 when that is needed to give every CU two workgroups
        const bool narrow = (long)(w.rows + 7) / 8 * m < 512;
        if (w.quant == JK_TQ2_0)
            return narrow ? launch_bl_ternary<JK_TQ2_0, 4>(s, w, act, act_scales, m, y)
                          : launch_bl_ternary<JK_TQ2_0, 8>(s, w, act, act_scales, m, y);
        return narrow ? launch_bl_ternary<JK_I2_S, 4>(s, w, act, act_scales, m, y)
                      : launch_bl_ternary<JK_I2_S, 8>(s, w, act, act_scales, m, y);
    }
    JK_LAUNCH("bitlinear_kernel", bitlinear_kernel, dim3((unsigned)((w.rows + 15) / 16), (unsigned)m), dim3(256), 0, s, w, act,
                       act_scales, y);
    return check_launch("bitlinear_kernel");
}

}  // namespace jk
