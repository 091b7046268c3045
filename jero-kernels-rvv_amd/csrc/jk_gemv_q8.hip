// jk_gemv_q8.hip -- batch-1 quant_q8 GEMV (Q4_0/Q5_0/Q8_0 x Q8_0, Q4_K/Q5_K/Q6_K/TQ2_0 x Q8_K;
// TQ1_0 weights are held in the TQ2_0 layout).
//
// One launch serves a group of up to kMaxGemvJobs independent matrix-vector products of
// one weight format (e.g. the Q, K and V projections of a layer, or gate and up). Each
// workgroup owns a slice of output rows of one job and:
//   1. issues the 128-bit non-temporal loads of its first weight blocks,
//   2. stages the job's activation vector in LDS -- either quantizing f32 input with the
//      quantize_row_q8_0 / quantize_row_q8_k recipes (bit-exact) or copying caller
//      blocks -- while those loads are in flight,
//   3. evaluates every (row, block) with the reference's per-block arithmetic (integer
//      dot + f32 epilogue) and folds the block values of a row in block order.
// Lane mapping: LPR lanes per output row (16: one DPP row, 64: one wave); lane p takes
// blocks p, p + LPR, ... of its row. With LPR = 16 the ordered fold is chain_add over
// the DPP row; with LPR = 64 the wave's block values go through LDS and lane 0 adds
// them in order. Either way a row's result equals the reference's sequential
// block-order f32 sum bit for bit (run_4row_chunked_gemv, quant_q8.rs:1510-1560).
#include <limits.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "jk_device.hpp"

namespace jk {

// ------------------------------------------------------------ activation accessors
// Q8_K block staged in LDS: qs[256] @0, bsums i16[16] @256 (as given), d f32 @288,
// per-16 sums of qs i16[16] @304 (recomputed from qs): 336 bytes, a multiple of 16 whose
// dword stride (84) puts the 16-byte reads of 16 consecutive blocks on distinct banks.
constexpr int kXkBytes = 336;
// Q8_0 block staged in LDS: qs[32] @0, d f32 @32, sum of qs i32 @36: 48 bytes.
constexpr int kX0Bytes = 48;
constexpr int kMaxLdsX = 60 * 1024;  // staged activation; static LDS stays within the 64 KB default

struct XkLds {
    const uint8_t *p;
    __device__ int q(int i) const { return reinterpret_cast<const int *>(p)[i]; }
    __device__ int bsum(int j) const { return reinterpret_cast<const int16_t *>(p + 256)[j]; }
    __device__ float d() const { return *reinterpret_cast<const float *>(p + 288); }
    __device__ int s16(int j) const { return reinterpret_cast<const int16_t *>(p + 304)[j]; }
};

struct XkGlb {
    const jk_block_q8k *b;
    __device__ int q(int i) const { return reinterpret_cast<const int *>(b->qs)[i]; }
    __device__ int bsum(int j) const { return b->bsums[j]; }
    __device__ float d() const { return b->d; }
    __device__ int s16(int j) const {
        int s = 0;
        for (int i = 0; i < 4; ++i) s = dot4(q(4 * j + i), 0x01010101, s);
        return s;
    }
};

struct X0Lds {
    const uint8_t *p;
    __device__ int q(int i) const { return reinterpret_cast<const int *>(p)[i]; }
    __device__ float d() const { return *reinterpret_cast<const float *>(p + 32); }
    __device__ int sum() const { return *reinterpret_cast<const int *>(p + 36); }
};

struct X0Glb {
    const jk_block_q8_0 *b;
    __device__ int q(int i) const { return reinterpret_cast<const int *>(b->qs)[i]; }
    __device__ float d() const { return b->d; }
    __device__ int sum() const {
        int s = 0;
        for (int i = 0; i < 8; ++i) s = dot4(q(i), 0x01010101, s);
        return s;
    }
};

template <int Q> struct QTraits {
    static constexpr bool K = fmt_of(Q).be == 256;      // Q8_K activations
    static constexpr int XB = K ? kXkBytes : kX0Bytes;  // LDS bytes per block
    static constexpr int XE = K ? 256 : 32;             // elements per block
    static constexpr int C = fmt_of(Q).chunks;          // 16-byte weight chunks
    static constexpr bool D = fmt_of(Q).d_off >= 0;     // scale in the d-plane
    static constexpr bool H = fmt_of(Q).h_off >= 0;     // field in the word plane
    // blocks per lane per batch: about 64-144 weight bytes per lane per batch (two
    // batches are in flight per wave)
    static constexpr int U = C >= 4 ? 1 : C == 2 ? 2 : 4;
};

template <int Q> struct WReg {
    uint4 c[QTraits<Q>::C];
    uint32_t d;
    uint32_t h;
};

// Loads block b of row r with 128-bit non-temporal loads. xo (0 or 16) is XORed into
// every byte address: 16 keeps each access inside its own 128-byte line but makes it a
// distinct load (dummy loads that must not be merged with the real ones).
// Addresses are a wave-uniform plane base plus one 32-bit per-lane offset shared by all
// chunks (planes hold fewer than 2^28 blocks, checked at upload).
template <int Q>
__device__ __forceinline__ void wload(WReg<Q> &o, const WeightDev &w, int r, int b, unsigned xo = 0) {
    const uint32_t blk = (uint32_t)r * (uint32_t)w.nb + (uint32_t)b;
    const uint32_t off = (blk << 4) ^ xo;
    const size_t pstride = (size_t)w.rows * (size_t)w.nb * 16;
#pragma unroll
    for (int c = 0; c < QTraits<Q>::C; ++c) {
        const uint8_t *plane = w.planes + (size_t)c * pstride;
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(plane + off));
        o.c[c] = make_uint4(v.x, v.y, v.z, v.w);
    }
    if constexpr (QTraits<Q>::D)
        o.d = *reinterpret_cast<const uint16_t *>(reinterpret_cast<const uint8_t *>(w.dplane) + ((blk << 1) ^ (xo >> 3)));
    if constexpr (QTraits<Q>::H)
        o.h = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(w.hplane) + ((blk << 2) ^ (xo >> 2)));
}

// ------------------------------------------------------------------ block values
// dot_q4_0_q8_0_block_scalar (quant_q8.rs:672-684): nibbles are stored biased by +8, so
// sum((n - 8) * x) = sum(n * x) - 8 * sum(x), exactly.
template <class X>
__device__ __forceinline__ float val_q4_0(const WReg<JK_Q4_0> &wr, const X &x) {
    const float dw = f16_finite(wr.d);
    const float xd = x.d();
    if (dw == 0.0f || xd == 0.0f) return 0.0f;
    const uint4 q = wr.c[0];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s = dot4((int)(comp(q, i) & 0x0F0F0F0Fu), x.q(i), s);
        s = dot4((int)((comp(q, i) >> 4) & 0x0F0F0F0Fu), x.q(4 + i), s);
    }
    s -= 8 * x.sum();
    return (float)s * (dw * xd);
}

// dot_q5_0_q8_0_block_scalar (quant_q8.rs:688-703): q = (nibble | 16 * bit) - 16, so
// sum(q * x) = sum((nibble | 16 * bit) * x) - 16 * sum(x), exactly. Bit j of the word holds
// the fifth bit of element j (j < 16: low nibble of byte j; j >= 16: high nibble of byte j - 16).
template <class X>
__device__ __forceinline__ float val_q5_0(const WReg<JK_Q5_0> &wr, const X &x) {
    const float dw = f16_finite(wr.d);
    const float xd = x.d();
    if (dw == 0.0f || xd == 0.0f) return 0.0f;
    const uint4 q = wr.c[0];
    const uint32_t qh = wr.h;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t wd = comp(q, i);
        s = dot4((int)((wd & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (4 * i)) & 15u)), x.q(i), s);
        s = dot4((int)(((wd >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (16 + 4 * i)) & 15u)), x.q(4 + i), s);
    }
    s -= 16 * x.sum();
    return (float)s * (dw * xd);
}

// dot_q8_0_q8_0_block_scalar (quant_q8.rs:707-717)
template <class X>
__device__ __forceinline__ float val_q8_0(const WReg<JK_Q8_0> &wr, const X &x) {
    const float dw = f16_finite(wr.d);
    const float xd = x.d();
    if (dw == 0.0f || xd == 0.0f) return 0.0f;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = dot4((int)comp(wr.c[i >> 2], i & 3), x.q(i), s);
    return (float)s * (dw * xd);
}

// dot_q4_k_q8_k_block_scalar (quant_q8.rs:1834-1862) with the scale/min table of
// unpack_q4_q5_k_scales_mins (quant_q8.rs:1818-1830) evaluated four bytes at a time.
template <class X>
__device__ __forceinline__ float val_q4_k(const WReg<JK_Q4_K> &wr, const X &x) {
    const uint4 h = wr.c[0];
    const float xd = x.d();
    const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
    if ((d == 0.0f && dmin == 0.0f) || xd == 0.0f) return 0.0f;
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    int sumi = 0, sum_mins = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 qa = wr.c[1 + 2 * c], qb = wr.c[2 + 2 * c];
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t wd = comp(i < 4 ? qa : qb, i & 3);
            lo = dot4((int)(wd & 0x0F0F0F0Fu), x.q(16 * c + i), lo);
            hi = dot4((int)((wd >> 4) & 0x0F0F0F0Fu), x.q(16 * c + 8 + i), hi);
        }
        const uint32_t scv = c < 2 ? sc_lo : sc_hi, mv = c < 2 ? m_lo : m_hi;
        const int j = (2 * c) & 3;
        sumi += byte_of(scv, j) * lo + byte_of(scv, j + 1) * hi;
        const int bl = x.bsum(4 * c) + x.bsum(4 * c + 1);
        const int bh = x.bsum(4 * c + 2) + x.bsum(4 * c + 3);
        sum_mins += byte_of(mv, j) * bl + byte_of(mv, j + 1) * bh;
        // one 64-element chunk of activations in registers at a time
        __builtin_amdgcn_sched_barrier(0);
    }
    return (d * xd) * (float)sumi - (dmin * xd) * (float)sum_mins;
}

// dot_q5_k_q8_k_block_scalar (quant_q8.rs:1866-1899): the Q4_K evaluation with each quant's
// fifth bit, bit 2c (low nibbles) or 2c + 1 (high nibbles) of qh[l] for chunk c, at bit 4.
// Chunks: 0 the header, 1-2 qh[0..32), 3 + 2c and 4 + 2c the 32 qs bytes of chunk c.
template <class X>
__device__ __forceinline__ float val_q5_k(const WReg<JK_Q5_K> &wr, const X &x) {
    const uint4 h = wr.c[0];
    const float xd = x.d();
    const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
    if ((d == 0.0f && dmin == 0.0f) || xd == 0.0f) return 0.0f;
    const uint32_t sc_lo = h.y & 0x3F3F3F3Fu, m_lo = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    int sumi = 0, sum_mins = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 qa = wr.c[3 + 2 * c], qb = wr.c[4 + 2 * c];
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t wd = comp(i < 4 ? qa : qb, i & 3);
            const uint32_t hd = comp(wr.c[1 + (i >> 2)], i & 3);
            lo = dot4((int)((wd & 0x0F0F0F0Fu) | (((hd >> (2 * c)) & 0x01010101u) << 4)), x.q(16 * c + i), lo);
            hi = dot4((int)(((wd >> 4) & 0x0F0F0F0Fu) | (((hd >> (2 * c + 1)) & 0x01010101u) << 4)),
                      x.q(16 * c + 8 + i), hi);
        }
        const uint32_t scv = c < 2 ? sc_lo : sc_hi, mv = c < 2 ? m_lo : m_hi;
        const int j = (2 * c) & 3;
        sumi += byte_of(scv, j) * lo + byte_of(scv, j + 1) * hi;
        const int bl = x.bsum(4 * c) + x.bsum(4 * c + 1);
        const int bh = x.bsum(4 * c + 2) + x.bsum(4 * c + 3);
        sum_mins += byte_of(mv, j) * bl + byte_of(mv, j + 1) * bh;
        __builtin_amdgcn_sched_barrier(0);
    }
    return (d * xd) * (float)sumi - (dmin * xd) * (float)sum_mins;
}

// dot_q6_k_q8_k_block_scalar (quant_q8.rs:1903-1942): per 16-element group j,
// sum((q - 32) * x) = sum(q * x) - 32 * sum(x), with sum(x) from the recomputed sums.
template <class X>
__device__ __forceinline__ float val_q6_k(const WReg<JK_Q6_K> &wr, const X &x) {
    const float d = f16_finite(wr.d);
    const float xd = x.d();
    if (d == 0.0f || xd == 0.0f) return 0.0f;
    int S[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t L = comp(wr.c[(16 * h + t) >> 2], t & 3);
            const uint32_t H = comp(wr.c[(16 * h + 8 + t) >> 2], t & 3);
            const uint32_t Qh = comp(wr.c[8 + ((8 * h + t) >> 2)], t & 3);
            const int g = 8 * h + (t >> 2);
            const int q1 = (int)((L & 0x0F0F0F0Fu) | ((Qh & 0x03030303u) << 4));
            const int q2 = (int)((H & 0x0F0F0F0Fu) | (((Qh >> 2) & 0x03030303u) << 4));
            const int q3 = (int)(((L >> 4) & 0x0F0F0F0Fu) | (((Qh >> 4) & 0x03030303u) << 4));
            const int q4 = (int)(((H >> 4) & 0x0F0F0F0Fu) | (((Qh >> 6) & 0x03030303u) << 4));
            S[g] = dot4(q1, x.q(32 * h + t), S[g]);
            S[g + 2] = dot4(q2, x.q(32 * h + 8 + t), S[g + 2]);
            S[g + 4] = dot4(q3, x.q(32 * h + 16 + t), S[g + 4]);
            S[g + 6] = dot4(q4, x.q(32 * h + 24 + t), S[g + 6]);
        }
    const uint4 scv = wr.c[12];
    int sumi = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int sc = (int)(int8_t)(comp(scv, j >> 2) >> (8 * (j & 3)));
        // (24-bit multiply, exact: |sc| <= 128 and |S - 32 s16| <= 16 * 63 * 128 + 32 * 16 * 128)
        sumi += __mul24(sc, S[j] - 32 * x.s16(j));
    }
    return (d * xd) * (float)sumi;
}

// dot_tq2_0_q8_k_block_scalar (quant_q8.rs:1992-2003): sum((t - 1) * x) = sum(t * x) - sum(x).
// The device dword holds element 4j+i of activation dword j in bits 2j of byte i. TQ1_0
// weights (dot_tq1_0_q8_k_block, quant_q8.rs:1977-1988: the same arithmetic on the trits of
// unpack_tq1_0_lut) are stored in this layout and take this path.
template <class X>
__device__ __forceinline__ float val_tq2_0(const WReg<JK_TQ2_0> &wr, const X &x) {
    const float dw = f16_finite(wr.d);
    const float xd = x.d();
    if (xd == 0.0f || dw == 0.0f) return 0.0f;
    int s = 0, sx = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t wv = comp(wr.c[k >> 2], k & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j) s = dot4((int)((wv >> (2 * j)) & 0x03030303u), x.q(4 * k + j), s);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) sx += x.s16(j);
    return (float)(s - sx) * (dw * xd);
}

template <int Q, class X>
__device__ __forceinline__ float block_value(const WReg<Q> &wr, const X &x) {
    if constexpr (Q == JK_Q4_0) return val_q4_0(wr, x);
    else if constexpr (Q == JK_Q5_0) return val_q5_0(wr, x);
    else if constexpr (Q == JK_Q8_0) return val_q8_0(wr, x);
    else if constexpr (Q == JK_Q4_K) return val_q4_k(wr, x);
    else if constexpr (Q == JK_Q5_K) return val_q5_k(wr, x);
    else if constexpr (Q == JK_Q6_K) return val_q6_k(wr, x);
    else return val_tq2_0(wr, x);
}

// ------------------------------------------------------------------ LDS staging
// The activation is read into registers in rounds of ROUND dwords per workgroup, before
// any weight load of the CU (see the kernel): vector memory returns data in issue order,
// so activation loads queued behind weight loads would wait for the weight stream. With
// NW waves per workgroup, thread t holds dwords (or float4s) t + 64*NW*i of a round.
template <int NW, bool F32, int Q> struct XRegs {
    // dwords per thread per round: a 4096-wide f32 activation (16 KB) in one round, and for
    // Q6_K (whose register budget is 2 waves per SIMD) a 14336-wide one; caller blocks are
    // 4x smaller
    static constexpr int N = F32 && Q == JK_Q6_K ? (NW <= 4 ? 64 : 32) : F32 && NW <= 4 ? 16 : 8;
    static constexpr int ROUND = 64 * NW * N;
    uint32_t v[N];
};

// Round r of an f32 activation of n4 float4s (clamped, unconditional loads: entries past
// the end are never staged).
template <int NW, int Q>
__device__ __forceinline__ void xload_f32(XRegs<NW, true, Q> &xr, const float *__restrict__ x, int n4, int r) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll
    for (int i = 0; i < XRegs<NW, true, Q>::N / 4; ++i) {
        const float4 v = x4[min(r * (XRegs<NW, true, Q>::ROUND / 4) + (int)threadIdx.x + 64 * NW * i, n4 - 1)];
        xr.v[4 * i] = __float_as_uint(v.x);
        xr.v[4 * i + 1] = __float_as_uint(v.y);
        xr.v[4 * i + 2] = __float_as_uint(v.z);
        xr.v[4 * i + 3] = __float_as_uint(v.w);
    }
}

// Round r of caller blocks (ndw dwords), clamped and unconditional as above.
template <int NW, int Q>
__device__ __forceinline__ void xload_raw(XRegs<NW, false, Q> &xr, const uint32_t *__restrict__ x, int ndw, int r) {
#pragma unroll
    for (int i = 0; i < XRegs<NW, false, Q>::N; ++i) xr.v[i] = x[min(r * XRegs<NW, false, Q>::ROUND + (int)threadIdx.x + 64 * NW * i, ndw - 1)];
}

// Rust `(x * inv).round().clamp(-127.0, 127.0) as i8` for finite x (round_scaled_to_i8,
// quant_q8.rs:102-108): round-half-away-from-zero as trunc(t + copysign(0.5 - 2^-25, t)),
// exact for |t| < 2^23 and saturating beyond, a med3 clamp, and NaN -> 0 (t is NaN only
// when a subnormal block maximum makes inv infinite and x is 0).
__device__ __forceinline__ int quant_i8(float x, float inv) {
    const float t = x * inv;
    const float h = __uint_as_float((__float_as_uint(t) & 0x80000000u) | 0x3EFFFFFFu);  // +-(0.5 - 2^-25)
    const int q = (int)__builtin_amdgcn_fmed3f(__builtin_truncf(t + h), -127.0f, 127.0f);
    return t == t ? q : 0;
}

__device__ __forceinline__ uint32_t pack4(const int (&q)[4]) {
    return (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
           ((uint32_t)q[3] << 24);
}

// quantize_block_q8_k_scalar (quant_q8.rs:447-475) of one block by one wave, lane l holding
// elements 4l..4l+3 (non-finite elements count as 0, as there); bsums[j] is the sum of
// lanes 4j..4j+3.
__device__ __forceinline__ void quantize_q8_k_wave(float (&v)[4], uint8_t *dst, int l) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_isfinite(v[i]) ? v[i] : 0.0f;
    const float amax = wave_max64_dpp(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const bool zero = amax == 0.0f;  // amax is finite here
    const float inv = zero ? 0.0f : 127.0f / amax;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = quant_i8(v[i], inv);
    const int part = sum4_dpp(q[0] + q[1] + q[2] + q[3]);
    reinterpret_cast<uint32_t *>(dst)[l] = pack4(q);
    if ((l & 3) == 0) {
        reinterpret_cast<int16_t *>(dst + 256)[l >> 2] = (int16_t)part;
        reinterpret_cast<int16_t *>(dst + 304)[l >> 2] = (int16_t)part;
    }
    if (l == 0) *reinterpret_cast<float *>(dst + 288) = zero ? 0.0f : amax / 127.0f;
}

// quantize_block_q8_0_scalar (quant_q8.rs:203-219) of one block by 8 lanes, lane l (of 8)
// holding elements 4l..4l+3.
__device__ __forceinline__ void quantize_q8_0_lanes(float (&v)[4], uint8_t *dst, int l) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_isfinite(v[i]) ? v[i] : 0.0f;
    const float amax = max8_dpp(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const bool zero = amax == 0.0f;
    const float inv = zero ? 0.0f : 127.0f / amax;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = quant_i8(v[i], inv);
    const int s = sum8_dpp(q[0] + q[1] + q[2] + q[3]);
    reinterpret_cast<uint32_t *>(dst)[l] = pack4(q);
    if (l == 0) {
        *reinterpret_cast<float *>(dst + 32) = zero ? 0.0f : amax / 127.0f;
        *reinterpret_cast<int *>(dst + 36) = s;
    }
}

// Quantizes round r of f32 activations (registers) into the staged LDS blocks.
template <int Q, int NW>
__device__ __forceinline__ void xstage_f32(const XRegs<NW, true, Q> &xr, int nb, int r, uint8_t *s_x) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < XRegs<NW, true, Q>::N / 4; ++i) {
        float v[4] = {__uint_as_float(xr.v[4 * i]), __uint_as_float(xr.v[4 * i + 1]), __uint_as_float(xr.v[4 * i + 2]),
                      __uint_as_float(xr.v[4 * i + 3])};
        const int f = r * (XRegs<NW, true, Q>::ROUND / 4) + tid + 64 * NW * i;
        if constexpr (QTraits<Q>::K) {
            const int blk = f >> 6;  // uniform over the wave
            if (blk < nb) quantize_q8_k_wave(v, s_x + blk * kXkBytes, tid & 63);
        } else {
            const int blk = f >> 3;  // uniform over 8 lanes
            if (blk < nb) quantize_q8_0_lanes(v, s_x + blk * kX0Bytes, tid & 7);
        }
    }
}

// Scatters round r of caller blocks (BlockQ8K: d, qs[64], bsums[8] dwords; BlockQ8_0: d,
// qs[8]) into the staged LDS layout.
template <int Q, int NW>
__device__ __forceinline__ void xstage_raw(const XRegs<NW, false, Q> &xr, int ndw, int r, uint8_t *s_x) {
    constexpr bool K = QTraits<Q>::K;
    constexpr int DW = K ? 73 : 9, STEP = 64 * NW;
    // block / word of slot 0, then advanced by STEP dwords per slot without dividing
    const int k0 = r * XRegs<NW, false, Q>::ROUND + (int)threadIdx.x;
    int blk = k0 / DW, wd = k0 - blk * DW;
#pragma unroll
    for (int i = 0; i < XRegs<NW, false, Q>::N; ++i) {
        const int k = k0 + STEP * i;
        if (i > 0) {
            blk += STEP / DW;
            wd += STEP % DW;
            if (wd >= DW) {
                wd -= DW;
                ++blk;
            }
        }
        if (k < ndw) {
            uint8_t *dst = s_x + blk * QTraits<Q>::XB;
            int off;
            if (K) off = wd == 0 ? 288 : wd <= 64 ? 4 * (wd - 1) : 256 + 4 * (wd - 65);
            else off = wd == 0 ? 32 : 4 * (wd - 1);
            *reinterpret_cast<uint32_t *>(dst + off) = xr.v[i];
        }
        if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bounds the live address temporaries
    }
}

// Formats whose block value reads the recomputed sums of the staged caller quants: the block sum
// (Q4_0, Q5_0) or the per-16 sums (Q6_K, TQ2_0 / TQ1_0). Q8_0 reads neither, Q4_K and Q5_K read the
// caller's bsums as given.
template <int Q> constexpr bool kStagedSums = Q == JK_Q4_0 || Q == JK_Q5_0 || Q == JK_Q6_K || Q == JK_TQ2_0;

// Sums of the staged caller quants: per-16 sums (Q8_K) or the block sum (Q8_0).
template <int Q, int NW>
__device__ __forceinline__ void xstage_sums(int nb, uint8_t *s_x) {
    if constexpr (QTraits<Q>::K) {
        for (int it = threadIdx.x; it < nb * 16; it += 64 * NW) {
            uint8_t *dst = s_x + (it >> 4) * kXkBytes;
            const int j = it & 15;
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) s = dot4(reinterpret_cast<const int *>(dst)[4 * j + i], 0x01010101, s);
            reinterpret_cast<int16_t *>(dst + 304)[j] = (int16_t)s;
        }
    } else {
        for (int it = threadIdx.x; it < nb; it += 64 * NW) {
            uint8_t *dst = s_x + it * kX0Bytes;
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = dot4(reinterpret_cast<const int *>(dst)[i], 0x01010101, s);
            *reinterpret_cast<int *>(dst + 36) = s;
        }
    }
}

// The two halves of activation staging, around the weight loads issued between them.
// begin: round 0 into registers, then a barrier that puts every activation load of the
// workgroup ahead of its weight loads (it waits for no data).
template <int Q, bool F32, int NW>
__device__ __forceinline__ void stage_begin(XRegs<NW, F32, Q> &xr, const GemvJob &job, int nb) {
    using T = QTraits<Q>;
    if constexpr (F32) xload_f32<NW, Q>(xr, job.xf, nb * T::XE / 4, 0);
    else xload_raw<NW, Q>(xr, static_cast<const uint32_t *>(job.xq), nb * (T::K ? 73 : 9), 0);
    lds_barrier();
}
// finish: every round into the staged LDS layout (rounds after the first wait behind the
// weight loads), then the sums of caller blocks.
template <int Q, bool F32, int NW>
__device__ __forceinline__ void stage_finish(XRegs<NW, F32, Q> &xr, const GemvJob &job, int nb, uint8_t *s_x) {
    using T = QTraits<Q>;
    constexpr int RD = XRegs<NW, F32, Q>::ROUND;
    const int n4 = nb * T::XE / 4;         // f32 input: float4 count
    const int ndw = nb * (T::K ? 73 : 9);  // caller blocks: dword count
    const int nrounds = F32 ? (n4 + RD / 4 - 1) / (RD / 4) : (ndw + RD - 1) / RD;
    if constexpr (!F32 && kStagedSums<Q> && QTraits<Q>::K) {
        if (nrounds == 1) {
            // (kept apart from the round loop below: after that loop the compiler's wait analysis
            // treated registers its loads wrote as possibly pending and waited for every load --
            // the weights included -- before the sums reused them, so the barrier after the sums
            // held every wave of the workgroup until all their weights had arrived. Measured: Q6_K
            // 4096 x 14336 11.45 -> 11.26 us, TQ2_0 2560 x 6912 4.82 -> 4.56 us; the 32-element
            // formats keep the loop, as the split's registers cost them a wave per SIMD and
            // 0.3 us)
            xstage_raw<Q, NW>(xr, ndw, 0, s_x);
            lds_barrier();
            xstage_sums<Q, NW>(nb, s_x);
            lds_barrier();
            return;
        }
    }
    for (int rr = 0; rr < nrounds; ++rr) {
        if (rr > 0) {
            if constexpr (F32) xload_f32<NW, Q>(xr, job.xf, n4, rr);
            else xload_raw<NW, Q>(xr, static_cast<const uint32_t *>(job.xq), ndw, rr);
        }
        if constexpr (F32) xstage_f32<Q, NW>(xr, nb, rr, s_x);
        else xstage_raw<Q, NW>(xr, ndw, rr, s_x);
    }
    lds_barrier();
    if constexpr (!F32 && kStagedSums<Q>) {
        xstage_sums<Q, NW>(nb, s_x);
        lds_barrier();
    }
}

// Grid of a group launch: blockIdx.y is the job, blockIdx.x the workgroup within it (the
// grid is as wide as the largest job; workgroups past a job's own count exit at once). The
// job is known from the dispatch itself, so a workgroup's first scalar load already fetches
// its job's fields: a lookup table of first workgroups would cost a second dependent load
// round trip before the first weight load (about 0.5 us per launch on MI355X).

// ------------------------------------------------------------------ kernel
// Work unit of a wave: RPU output rows (4 with LPR 16, 1 with LPR 64) over all their
// blocks, walked in batches of U blocks per lane. A wave takes units u, u + S, u + 2S, ...
// (S = waves of its job), in pairs of batches whose loads are issued together.
template <int Q, int LPR>
struct Walker {
    using T = QTraits<Q>;
    static constexpr int RPU = 64 / LPR;
    int nb, nit, units, stride, r0, r1, rows4, sub, p;

    __device__ __forceinline__ void next(int &u, int &it0) const {
        it0 += T::U;
        if (it0 >= nit) {
            it0 = 0;
            u += stride;
        }
    }
    __device__ __forceinline__ int row_of(int u) const { return r0 + u * RPU + sub; }

    // Batch (u, it0), or with dummy set, a distinct re-read of the same lines.
    __device__ __forceinline__ void load(WReg<Q> (&wr)[T::U], const WeightDev &w, int u, int it0,
                                         bool dummy = false) const {
        const int row = row_of(u);
        const int r = row < r1 ? row : r0;
#pragma unroll
        for (int k = 0; k < T::U; ++k) wload<Q>(wr[k], w, r, min((it0 + k) * LPR + p, nb - 1), dummy ? 16u : 0u);
    }

    // Folds batch (u, it0) into acc in block order. At the unit's last batch every lane
    // parks acc in its LDS slot of the unit (slot[k * 64 + lane], k = the wave's unit
    // ordinal): a global store here would sit in a lane-divergent branch between the
    // loads, and the compiler then has to drain all outstanding loads at every wait.
    template <class Red>
    __device__ __forceinline__ float run(const WReg<Q> (&wr)[T::U], int u, int it0, float acc, const uint8_t *s_x,
                                         float *slot, int k0, Red *red) const {
        const int row = row_of(u);
        const int r = row < r1 ? row : r0;
        if (it0 == 0) acc = r < rows4 ? 0.0f : -0.0f;
        float v[T::U];
#pragma unroll
        for (int k = 0; k < T::U; ++k) {
            const int b = (it0 + k) * LPR + p;
            v[k] = -0.0f;  // past the row end: the identity of the ordered fold
            if (b < nb) {
                if constexpr (T::K) v[k] = block_value<Q>(wr[k], XkLds{s_x + b * T::XB});
                else v[k] = block_value<Q>(wr[k], X0Lds{s_x + b * T::XB});
            }
        }
#pragma unroll
        for (int k = 0; k < T::U; ++k) {
            if (it0 + k < nit) {
                if constexpr (LPR == 16) acc = chain_add(acc, v[k]);
                else acc = fold_wave(acc, v[k], red);
            }
        }
        if (it0 + T::U >= nit) slot[((u - k0) / stride) * 64 + (threadIdx.x & 63)] = acc;
        return acc;
    }

    // Lane that holds a row's result after the fold.
    __device__ __forceinline__ int writer() const { return LPR == 16 ? 15 : 0; }
};

// Register budget: 4 waves per SIMD (<= 128 VGPRs) for Q4_K / Q4_0 / Q8_0 / TQ2_0, 2 for
// Q6_K. Waves per workgroup (NW): a "full" workgroup fills a CU at that budget (16 or 8
// waves), so the activation is staged once per CU; launches with too few row units to
// give every CU a full workgroup use 4-wave workgroups instead.
template <int Q> constexpr int kWavesPerSimd = Q == JK_Q6_K ? 2 : 4;
template <int Q> constexpr int kFullWaves = 4 * kWavesPerSimd<Q>;

template <int Q, int LPR, bool F32, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd<Q>))) void
gemv_q8_group_kernel(GemvGroup grp) {
    using T = QTraits<Q>;
    extern __shared__ __align__(16) uint8_t s_x[];
    __shared__ __align__(16) float s_red[LPR == 64 ? NW : 1][64];

    const GemvJob &job = grp.job[blockIdx.y];
    if ((int)blockIdx.x >= job.nwg) return;  // (uniform over the workgroup)
    const WeightDev &w = job.w;

    // wave index as a scalar: the unit loop below must be wave-uniform control flow
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    Walker<Q, LPR> wk;
    wk.nb = w.nb;
    wk.nit = (w.nb + LPR - 1) / LPR;
    wk.units = (job.r1 - job.r0 + Walker<Q, LPR>::RPU - 1) / Walker<Q, LPR>::RPU;
    wk.stride = job.nwg * NW;
    wk.r0 = job.r0;
    wk.r1 = job.r1;
    wk.rows4 = (w.rows >> 2) << 2;
    wk.sub = lane / LPR;
    wk.p = lane % LPR;

    // 1. first round of the activation into registers (see stage_begin)
    const int nb = w.nb;
    XRegs<NW, F32, Q> xr;
    stage_begin<Q, F32, NW>(xr, job, nb);

    // 2. the first pair of weight batches. Loads are issued unconditionally -- a load that
    //    may or may not have been issued would make every later wait drain all outstanding
    //    loads. A batch position past the last unit re-reads batch A's own addresses (lines
    //    already requested), so the dummy loads neither add traffic nor pile onto one row;
    //    a wave without any unit reads a row of its own index.
    int ua = (int)blockIdx.x * NW + wave, ia = 0;
    int ub = ua, ib = ia;
    wk.next(ub, ib);
    WReg<Q> A[T::U], B[T::U];
    const int ua_ld = ua < wk.units ? ua : ua % wk.units;
    wk.load(A, w, ua_ld, ia);
    {
        const bool bd = ub >= wk.units;  // wave-uniform
        wk.load(B, w, bd ? ua_ld : ub, bd ? ia : ib, bd);
    }

    // 3. activation vector into the staged LDS layout
    stage_finish<Q, F32, NW>(xr, job, nb, s_x);

    // 4. batches in order, in pairs: both loads of a pair are issued before either batch
    //    is evaluated, and nothing is outstanding across the loop's back-edge, so every
    //    wait below is exact (for the decode shapes a wave has at most one pair).
    float acc = 0.0f;
    float *red = s_red[LPR == 64 ? wave : 0];
    float *slot = reinterpret_cast<float *>(s_x + grp.out_off) + wave * grp.upw * 64;
    const int u0 = ua;
    while (ua < wk.units) {
        acc = wk.run(A, ua, ia, acc, s_x, slot, u0, red);
        if (ub < wk.units) acc = wk.run(B, ub, ib, acc, s_x, slot, u0, red);
        ua = ub;
        ia = ib;
        wk.next(ua, ia);
        if (ua >= wk.units) break;
        ub = ua;
        ib = ia;
        wk.next(ub, ib);
        wk.load(A, w, ua, ia);
        const bool bd = ub >= wk.units;
        wk.load(B, w, bd ? ua : ub, bd ? ia : ib, bd);
    }

    // 5. results out of the LDS slots (and, for an argmax job, the key of each result row)
    wave_lds_sync();
    const int wr_lane = wk.writer();
    unsigned long long key = 0ull;
    for (int u = u0, k = 0; u < wk.units; u += wk.stride, ++k) {
        const int row = wk.row_of(u);
        if (row < wk.r1 && wk.p == wr_lane) {
            const float v = slot[k * 64 + lane];
            if (job.y) job.y[row - wk.r0] = v;
            if (job.am_slots) {
                const unsigned long long kk = argmax_key(v, (uint32_t)(row - wk.r0));
                key = kk > key ? kk : key;
            }
        }
    }
    if (job.am_slots) {
        __shared__ unsigned long long s_keys[NW];
        argmax_store_wg(key, job.am_slots + blockIdx.x, s_keys, NW);
    }
}

// ------------------------------------------------------------------ fast kernel
// Straight-line variant for launches whose rows fit in one batch per unit (nit <= UF):
// workgroup g of a job owns units [g * upg, (g + 1) * upg) and wave w of it units
// g * upg + w + NW * q (q < QPW); a wave issues all its weight loads up front, evaluates
// them and keeps the results in registers until one store pass at the end. Without a loop
// the compiler keeps every load where it is written and every wait exact.
template <int Q> constexpr int kFastU = Q == JK_Q4_0 || Q == JK_Q5_0 || Q == JK_Q8_0 ? 8 : Q == JK_TQ2_0 ? 2 : 1;

template <int Q, int LPR, bool F32, int NW, int QPW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd<Q>))) void
gemv_q8_fast_kernel(GemvGroup grp) {
    using T = QTraits<Q>;
    constexpr int RPU = 64 / LPR, UF = kFastU<Q>;
    extern __shared__ __align__(16) uint8_t s_x[];
    __shared__ __align__(16) float s_red[LPR == 64 ? NW : 1][64];

    const GemvJob &job = grp.job[blockIdx.y];
    if ((int)blockIdx.x >= job.nwg) return;  // (uniform over the workgroup)
    const WeightDev &w = job.w;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int sub = lane / LPR, p = lane % LPR;
    const int nb = w.nb, nit = (nb + LPR - 1) / LPR;  // nit <= UF
    const int r0 = job.r0, r1 = job.r1;
    const int g0 = (int)blockIdx.x * job.upg;
    const int units = min((r1 - r0 + RPU - 1) / RPU, g0 + job.upg);  // end of this workgroup's units
    const int base = g0 + wave;                                          // unit q: base + NW * q

    // 1. activation round 0, then the weight loads of the wave's first two units. A unit
    //    past the end re-reads a valid unit's lines at distinct addresses (xor 16): the
    //    loads stay unconditional, add no traffic and are never merged with the real ones.
    XRegs<NW, F32, Q> xr;
    stage_begin<Q, F32, NW>(xr, job, nb);
    const int ufb = base < units ? base : g0;  // a valid unit of the workgroup
    WReg<Q> W[QPW > 1 ? 2 : 1][UF];
    auto load_unit = [&](int q, WReg<Q>(&dst)[UF]) {
        const bool dummy = base + NW * q >= units;
        const int row = r0 + (dummy ? ufb : base + NW * q) * RPU + sub;
        const int r = min(row, r1 - 1);
#pragma unroll
        for (int k = 0; k < UF; ++k) wload<Q>(dst[k], w, r, min(k * LPR + p, nb - 1), dummy ? 16u : 0u);
    };
    load_unit(0, W[0]);
    if constexpr (QPW > 1) load_unit(1, W[1]);

    // 2. activation vector into the staged LDS layout
    stage_finish<Q, F32, NW>(xr, job, nb, s_x);

    // 3. units in order, two in flight: unit q is folded while unit q + 1 loads, then unit
    //    q + 2 is issued into the buffer just consumed. Block values fold in block order;
    //    results stay in registers.
    const int rows4 = (w.rows >> 2) << 2;
    float *red = s_red[LPR == 64 ? wave : 0];
    float out[QPW];
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
        const WReg<Q>(&Wq)[UF] = W[q & (QPW > 1 ? 1 : 0)];
        const int row = r0 + (base + NW * q) * RPU + sub;
        float acc = row < rows4 ? 0.0f : -0.0f;
        float v[UF];
#pragma unroll
        for (int k = 0; k < UF; ++k) {
            const int b = k * LPR + p;
            v[k] = -0.0f;  // past the row end: the identity of the ordered fold
            if (b < nb) {
                if constexpr (T::K) v[k] = block_value<Q>(Wq[k], XkLds{s_x + b * T::XB});
                else v[k] = block_value<Q>(Wq[k], X0Lds{s_x + b * T::XB});
            }
        }
#pragma unroll
        for (int k = 0; k < UF; ++k) {
            if (k < nit) {
                if constexpr (LPR == 16) acc = chain_add(acc, v[k]);
                else acc = fold_wave(acc, v[k], red);
            }
        }
        out[q] = acc;
        if (q + 2 < QPW) load_unit(q + 2, W[q & 1]);
    }

    // 4. stores (and, for an argmax job, the key of each result row)
    const int writer = LPR == 16 ? 15 : 0;
    unsigned long long key = 0ull;
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
        const int row = r0 + (base + NW * q) * RPU + sub;
        if (base + NW * q < units && row < r1 && p == writer) {
            if (job.y) job.y[row - r0] = out[q];
            if (job.am_slots) {
                const unsigned long long kk = argmax_key(out[q], (uint32_t)(row - r0));
                key = kk > key ? kk : key;
            }
        }
    }
    if (job.am_slots) {
        __shared__ unsigned long long s_keys[NW];
        argmax_store_wg(key, job.am_slots + blockIdx.x, s_keys, NW);
    }
}

// ------------------------------------------------------------------ repacked GEMV, 1-2 tokens
// gemm_repacked's recipe for one or two tokens (the reference's m <= 2 route, repack.rs:2892),
// shaped like the quant_q8 GEMV: 16 lanes per output row, lane p taking blocks p, p + 16, ... of
// the row from the planes into registers (two blocks in flight). A block's scale groups give their
// terms (accumulate_scaled_tile_scalar, repack.rs:3045-3093)
//     f32(sum xq * wq) * (xs * ws)  [- xsum * wm]
// with the weight values, scales and mins of repack_block_scaled_range_into_i8 (repack.rs:
// 1724-2103), and each block's terms are folded, in K order, onto the running sum passed from
// the lane of the previous block (the chain_add steps with a block's terms per step): every
// output is the GEMM's sum, in the GEMM's order, starting from 0.0. The activation quants are
// staged in LDS once per workgroup (their loads issued before the weight loads); scales and sums
// are read per lane.
constexpr int kRpNW = 4;        // waves per workgroup: 4 rows a wave
constexpr int kRpMaxLoads = 8;  // 16-byte activation loads per thread and staging round
constexpr int kRpMaxPieces = 2048;  // staged activation: MT * k_padded <= 32 KB, MT * k_blocks32 <= 2048

template <int Q> constexpr int kRpGroups = Q == JK_Q4_K || Q == JK_Q5_K ? 8 : Q == JK_Q6_K ? 16 : 1;  // scale groups per block
// LDS padding after each block's activation quants: the 16 lanes of a row read 16 consecutive
// blocks at once, and at 256 bytes a block they would all fall on the same banks; 16 more bytes
// a block put consecutive lanes on consecutive 16-byte bank groups. (32-byte blocks already do.)
template <int Q> constexpr int kRpPad = fmt_of(Q).be >= 256 ? 16 : 0;
static bool rp_kquant(int quant) { return quant == JK_Q4_K || quant == JK_Q5_K || quant == JK_Q6_K; }
static size_t rp_lds_row(int quant, size_t k_padded) {
    return k_padded + (rp_kquant(quant) ? k_padded / 256 * 16 : 0);
}

// The terms of block b of the lane's row for one token (its quants of the block in LDS, its
// scales and sums in LDS).
template <int Q>
__device__ __forceinline__ void rp_terms(const WReg<Q> &wr, const uint8_t *xq, const float *xs, const float *xm,
                                         float (&t)[kRpGroups<Q>]) {
    const int *xi = reinterpret_cast<const int *>(xq);
    if constexpr (Q == JK_Q8_0 || Q == JK_Q4_0 || Q == JK_Q5_0 || Q == JK_IQ4_NL) {
        const float ws = f16_finite(wr.d);  // repack.rs:1735-1760: the block's d
        int s = 0;
        if constexpr (Q == JK_Q8_0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) s = dot4((int)comp(wr.c[i >> 2], i & 3), xi[i], s);
        } else if constexpr (Q == JK_Q5_0) {  // (nibble | 16 bit) - 16, element j's bit j of the word (repack.rs:1830)
            int sx = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd = comp(wr.c[0], i);
                s = dot4((int)((wd & 0x0F0F0F0Fu) | bit4_of_bytes((wr.h >> (4 * i)) & 15u)), xi[i], s);
                s = dot4((int)(((wd >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes((wr.h >> (16 + 4 * i)) & 15u)), xi[4 + i], s);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) sx = dot4(xi[i], 0x01010101, sx);
            s -= 16 * sx;
        } else if constexpr (Q == JK_IQ4_NL) {  // KVALUES_IQ4NL[nibble] (repack.rs:1861)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = dot4((int)iq4nl_lookup(comp(wr.c[0], i) & 0x0F0F0F0Fu), xi[i], s);
                s = dot4((int)iq4nl_lookup((comp(wr.c[0], i) >> 4) & 0x0F0F0F0Fu), xi[4 + i], s);
            }
        } else {  // nibbles biased by +8: sum((n - 8) x) = sum(n x) - 8 sum(x), exactly
            int sx = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = dot4((int)(comp(wr.c[0], i) & 0x0F0F0F0Fu), xi[i], s);
                s = dot4((int)((comp(wr.c[0], i) >> 4) & 0x0F0F0F0Fu), xi[4 + i], s);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) sx = dot4(xi[i], 0x01010101, sx);
            s -= 8 * sx;
        }
        t[0] = (float)s * (xs[0] * ws);
    } else if constexpr (Q == JK_Q4_K || Q == JK_Q5_K) {
        // sub-block g (elements 32 g ..): quarter g / 2, low (g even) or high nibbles of planes
        // 1 + g / 2 * 2 and 2 + g / 2 * 2 (Q5_K: planes 3 + ..., 4 + ..., and bit g of the qh bytes
        // in planes 1 and 2 as the fifth bit); scale / min unpack_k4_scales_mins (repack.rs:1158-1170)
        const uint4 h = wr.c[0];
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        const uint32_t sc[2] = {h.y & 0x3F3F3F3Fu, (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u)};
        const uint32_t mv[2] = {h.z & 0x3F3F3F3Fu, ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u)};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int c = g >> 1, sh = 4 * (g & 1);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                constexpr int P = Q == JK_Q5_K ? 3 : 1;  // first quant plane
                const uint32_t wd = comp(i < 4 ? wr.c[P + 2 * c] : wr.c[P + 1 + 2 * c], i & 3);
                uint32_t v = (wd >> sh) & 0x0F0F0F0Fu;
                if constexpr (Q == JK_Q5_K) v |= ((comp(wr.c[1 + (i >> 2)], i & 3) >> g) & 0x01010101u) << 4;
                s = dot4((int)v, xi[8 * g + i], s);
            }
            const float ws = d * (float)byte_of(sc[g >> 2], g & 3);
            const float wm = dmin * (float)byte_of(mv[g >> 2], g & 3);
            t[g] = (float)s * (xs[g] * ws) - xm[g] * wm;
        }
    } else {  // JK_Q6_K
        // 16-group g of half h (elements 128 h + 16 g ..): ql plane 4 h + g % 2 + 2 (g / 2 % 2),
        // nibble g / 4, qh plane 8 + 2 h + g % 2, field g / 2; scale 8 h + g (repack.rs:1861-1874)
        const float d = f16_finite(wr.d);
        const uint4 scv = wr.c[12];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const int j = g & 1, qq = g >> 1, js = 8 * hh + g;
                const uint4 lv = wr.c[4 * hh + j + 2 * (qq & 1)], hv = wr.c[8 + 2 * hh + j];
                const int lsh = qq < 2 ? 0 : 4, hsh = 2 * qq;
                int s = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t v6 =
                        ((comp(lv, i) >> lsh) & 0x0F0F0F0Fu) | (((comp(hv, i) >> hsh) & 0x03030303u) << 4);
                    s = dot4(bytes_sub(v6, 0x20202020u), xi[32 * hh + 4 * g + i], s);
                }
                const float ws = d * (float)(int8_t)(comp(scv, js >> 2) >> (8 * (js & 3)));
                t[8 * hh + g] = (float)s * (xs[4 * hh + (g >> 1)] * ws);
            }
    }
}

template <int Q, int MT>
__global__ __launch_bounds__(64 * kRpNW) __attribute__((amdgpu_waves_per_eu(2))) void
gemv_repacked_fast_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    constexpr int G = kRpGroups<Q>, BE = fmt_of(Q).be, NT = 64 * kRpNW, PAD = kRpPad<Q>;
    constexpr bool SUMS = Q == JK_Q4_K || Q == JK_Q5_K;
    // LDS: activation quants [MT][k_padded / BE][BE + PAD] (k_padded a multiple of BE when PAD is
    // not 0), then scales [MT][k_blocks32] (and sums, Q4_K)
    extern __shared__ __align__(16) uint8_t s_xq[];
    if (MT == 1 && blockIdx.y > 0) {  // one token per workgroup row of the grid: token blockIdx.y
        a.qs += blockIdx.y * a.k_padded;
        a.scales += blockIdx.y * a.k_blocks32;
        a.sums += blockIdx.y * a.k_blocks32;
        y += blockIdx.y * (size_t)(r1 - r0);
    }
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = lane & 15, sub = lane >> 4;
    const int row = r0 + 4 * kRpNW * (int)blockIdx.x + 4 * wave + sub;
    const int r = min(row, r1 - 1);
    const int nb = w.nb, nit = (nb + 15) / 16;
    const int kp = (int)a.k_padded, kb = (int)a.k_blocks32;
    const int kpp = kp + kp / BE * PAD;  // one token's padded quants
    float *s_xs = reinterpret_cast<float *>(s_xq + MT * kpp);
    float *s_xm = s_xs + MT * kb;

    // 1. the activation -- quants in 16-byte loads, scales (and sums) in 4-byte loads -- in rounds
    //    of kRpMaxLoads per thread; round 0 is issued first (clamped, unconditional), so that it
    //    does not queue behind the weight stream
    const int n16 = MT * kp / 16, n4 = MT * kb;
    const int rounds = (max(n16, n4) + NT * kRpMaxLoads - 1) / (NT * kRpMaxLoads);
    u32x4 xr[kRpMaxLoads];  // (a plain vector type: an array of uint4 is kept in scratch)
    float sr[kRpMaxLoads], mr[kRpMaxLoads];
    auto stage_load = [&](int rd) {
#pragma unroll
        for (int i = 0; i < kRpMaxLoads; ++i) {
            const int k = min(NT * (kRpMaxLoads * rd + i) + tid, n16 - 1);
            const int m = k / (kp / 16), o = k - m * (kp / 16);
            xr[i] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint8_t *>(a.qs) + (size_t)m * a.k_padded +
                                                     16 * o);
            const int e = min(NT * (kRpMaxLoads * rd + i) + tid, n4 - 1);  // token m's scales at a.scales + m * kb
            sr[i] = a.scales[e];
            mr[i] = SUMS ? a.sums[e] : 0.0f;
        }
    };
    // every store unconditional, at the index its load was clamped to (a clamped store rewrites
    // the last element with its own value), so the stores stay one straight-line sequence
    auto stage_store = [&](int rd) {
#pragma unroll
        for (int i = 0; i < kRpMaxLoads; ++i) {
            const int k = min(NT * (kRpMaxLoads * rd + i) + tid, n16 - 1);  // piece k: block k / (BE / 16) of all MT
            *reinterpret_cast<u32x4 *>(s_xq + 16 * k + PAD * (k / (BE / 16))) = xr[i];
            const int e = min(NT * (kRpMaxLoads * rd + i) + tid, n4 - 1);
            s_xs[e] = sr[i];
            if constexpr (SUMS) s_xm[e] = mr[i];
        }
    };
    stage_load(0);
    // 2. the lane's first two blocks
    WReg<Q> W[2];
    wload<Q>(W[0], w, r, min(p, nb - 1));
    wload<Q>(W[1], w, r, min(16 + p, nb - 1));
    // 3. the activation into LDS (further rounds behind the weight loads)
    stage_store(0);
    for (int rd = 1; rd < rounds; ++rd) {
        stage_load(rd);
        stage_store(rd);
    }
    lds_barrier();

    // 4. blocks in order, two in flight: block it is folded while block it + 1 loads, then block
    //    it + 2 is issued into the buffer just consumed (clamped past the row end: the loads stay
    //    unconditional, which keeps the double buffer's waits exact -- branching around them
    //    measured slower)
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    auto fold_block = [&](const WReg<Q> &wr, int it) {
        const int b = 16 * it + p;
        const bool live = b < nb;
        const int bb = live ? b : 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float t[G];
            rp_terms<Q>(wr, s_xq + m * kpp + bb * (BE + PAD), s_xs + m * kb + bb * (BE / 32), s_xm + m * kb + bb * (BE / 32), t);
#pragma unroll
            for (int g = 0; g < G; ++g) t[g] = live ? t[g] : -0.0f;  // -0.0: the identity of the fold
            // the chain: in step s the lane of block 16 it + s folds its terms onto the sum passed
            // from the lane before it (after the 16 steps lane 15 holds the sum through the block)
#pragma unroll
            for (int st = 0; st < 16; ++st) {
                float run = row_ror1(acc[m]);
#pragma unroll
                for (int g = 0; g < G; ++g) run = run + t[g];
                acc[m] = run;
            }
        }
    };
    for (int it = 0; it < nit; it += 2) {
        fold_block(W[0], it);
        wload<Q>(W[0], w, r, min(16 * (it + 2) + p, nb - 1));
        if (it + 1 >= nit) break;
        fold_block(W[1], it + 1);
        wload<Q>(W[1], w, r, min(16 * (it + 3) + p, nb - 1));
    }
    if (p == 15 && row < r1)
#pragma unroll
        for (int m = 0; m < MT; ++m) y[(size_t)m * (size_t)(r1 - r0) + (size_t)(row - r0)] = acc[m];
}

template <int Q>
static jk_status launch_rp_fast_q(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    // Q6_K takes two tokens as two rows of one-token workgroups (both tokens in one wave need more
    // registers than it has); the second token's weight reads then mostly hit the caches
    const bool split = Q == JK_Q6_K && a.m == 2;
    const size_t mt = split ? 1 : a.m;
    const size_t lds = mt * rp_lds_row(Q, a.k_padded) + (Q == JK_Q4_K || Q == JK_Q5_K ? 2 : 1) * mt * a.k_blocks32 * sizeof(float);
    const dim3 grid((unsigned)((r1 - r0 + 4 * kRpNW - 1) / (4 * kRpNW)), split ? 2u : 1u), block(64 * kRpNW);
    if (mt == 1) JK_LAUNCH("gemv_repacked_fast_kernel<1 token>", (gemv_repacked_fast_kernel<Q, 1>), grid, block, lds, s, w, a, y, r0, r1);
    else if constexpr (Q != JK_Q6_K)
        JK_LAUNCH("gemv_repacked_fast_kernel<2 tokens>", (gemv_repacked_fast_kernel<Q, 2>), grid, block, lds, s, w, a, y, r0, r1);
    return check_launch("gemv_repacked_fast_kernel");
}

bool gemv_repacked_fast_ok(int quant, size_t m, size_t k_padded, size_t k_blocks32) {
    const bool fmt = quant == JK_Q8_0 || quant == JK_Q4_0 || quant == JK_Q5_0 || quant == JK_IQ4_NL || rp_kquant(quant);
    const bool padded = rp_kquant(quant);
    return fmt && m >= 1 && m <= 2 && k_padded % (padded ? 256 : 16) == 0 && m * k_padded / 16 <= kRpMaxPieces &&
           m * k_blocks32 <= kRpMaxPieces;
}

// (checked by the caller with gemv_repacked_fast_ok)
jk_status launch_gemv_repacked_fast(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    switch (w.quant) {
    case JK_Q8_0: return launch_rp_fast_q<JK_Q8_0>(s, w, a, y, r0, r1);
    case JK_Q4_0: return launch_rp_fast_q<JK_Q4_0>(s, w, a, y, r0, r1);
    case JK_Q5_0: return launch_rp_fast_q<JK_Q5_0>(s, w, a, y, r0, r1);
    case JK_IQ4_NL: return launch_rp_fast_q<JK_IQ4_NL>(s, w, a, y, r0, r1);
    case JK_Q4_K: return launch_rp_fast_q<JK_Q4_K>(s, w, a, y, r0, r1);
    case JK_Q5_K: return launch_rp_fast_q<JK_Q5_K>(s, w, a, y, r0, r1);
    case JK_Q6_K: return launch_rp_fast_q<JK_Q6_K>(s, w, a, y, r0, r1);
    default: return fail(JK_CAPABILITY_MISMATCH, "gemv_repacked_fast: unsupported quant %d", w.quant);
    }
}

// ------------------------------------------------------------------ global-x fallback
// Activations read from global memory (matrices whose activation exceeds the LDS budget).
template <int Q>
__global__ __launch_bounds__(256) void gemv_q8_global_kernel(WeightDev w, const void *__restrict__ x,
                                                             float *__restrict__ y, int r0, int r1,
                                                             unsigned long long *am_slots) {
    const int p = threadIdx.x & 15;
    const int row = r0 + (int)((blockIdx.x * 256u + threadIdx.x) >> 4);
    const bool active = row < r1;
    const int r = active ? row : r0;
    const int rows4 = (w.rows >> 2) << 2;
    float acc = r < rows4 ? 0.0f : -0.0f;
    const int nb = w.nb;
    const int iters = (nb + 15) >> 4;
    for (int it = 0; it < iters; ++it) {
        const int b = 16 * it + p;
        float v = -0.0f;  // past the row end: the identity of the ordered fold
        if (b < nb) {
            WReg<Q> wr;
            wload<Q>(wr, w, r, b);
            if constexpr (QTraits<Q>::K) v = block_value<Q>(wr, XkGlb{static_cast<const jk_block_q8k *>(x) + b});
            else v = block_value<Q>(wr, X0Glb{static_cast<const jk_block_q8_0 *>(x) + b});
        }
        acc = chain_add(acc, v);
    }
    if (active && p == 15 && y) y[row - r0] = acc;
    if (am_slots) {
        __shared__ unsigned long long s_keys[4];
        argmax_store_wg(active && p == 15 ? argmax_key(acc, (uint32_t)(row - r0)) : 0ull, am_slots + blockIdx.x, s_keys,
                        4);
    }
}

// ------------------------------------------------------------------ launchers

// Resident workgroups per CU of a kernel at a given dynamic LDS size (queried once).
template <class K>
static int resident_per_cu(K kernel, size_t lds, int threads) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, int> cache;
    const std::pair<const void *, size_t> key{reinterpret_cast<const void *>(kernel), lds};
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) n = 1;
    cache[key] = n;
    return n;
}

static int cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

// The argmax of each argmax job of a launched group: reduce its workgroups' keys.
static jk_status launch_group_argmax(hipStream_t s, const GemvGroup &g) {
    for (int i = 0; i < g.njobs; ++i)
        if (g.job[i].am_slots) JK_TRY(launch_argmax_slots(s, g.job[i].am_slots, g.job[i].nwg, g.job[i].am_index));
    return JK_OK;
}

template <int Q, int LPR, bool F32, int NW>
static jk_status launch_group_run(hipStream_t s, GemvGroup &g, size_t lds) {
    // (lds: the staged activation; the result slots are appended below)
    constexpr int RPU = 64 / LPR;
    auto kern = gemv_q8_group_kernel<Q, LPR, F32, NW>;
    // Size the grid to one resident round: each wave then walks ceil(units / waves) units.
    const int cap_waves = resident_per_cu(kern, lds, 64 * NW) * cu_count() * NW;
    long total = 0;
    for (int i = 0; i < g.njobs; ++i) total += (g.job[i].r1 - g.job[i].r0 + RPU - 1) / RPU;
    // (at most 16 units per wave: bigger jobs get more than one round of workgroups)
    const int upw = (int)std::min<long>(16, (total + cap_waves - 1) / cap_waves);
    g.upw = upw;
    g.out_off = (int)((lds + 15) / 16 * 16);
    lds = (size_t)g.out_off + (size_t)NW * upw * 64 * sizeof(float);
    int wgs = 0;
    for (int i = 0; i < g.njobs; ++i) {
        const int units = (g.job[i].r1 - g.job[i].r0 + RPU - 1) / RPU;
        g.job[i].nwg = (units + NW * upw - 1) / (NW * upw);
        wgs = max(wgs, g.job[i].nwg);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)wgs, (unsigned)g.njobs), dim3(64 * NW), lds, s, g);
    JK_TRY(check_launch("gemv_q8_group_kernel"));
    return launch_group_argmax(s, g);
}

// Jobs of unequal size leave part of a group launch's grid empty (its width is the largest
// job's workgroup count), and an empty workgroup still costs a dispatch. A group whose jobs
// differ in size is therefore re-cut, when it fits in kMaxGemvJobs, into jobs of the
// smallest job's workgroup count: row ranges of rpw rows per workgroup, each writing its
// own part of the original output (argmax jobs keep their shape: their slots are indexed by
// workgroup).
static void even_out_jobs(GemvGroup &g, int rpw) {
    if (g.njobs < 2) return;
    int min_wg = INT_MAX, max_wg = 0, pieces = 0;
    for (int i = 0; i < g.njobs; ++i) {
        if (g.job[i].am_slots) return;
        const int n = (g.job[i].r1 - g.job[i].r0 + rpw - 1) / rpw;
        min_wg = min(min_wg, n);
        max_wg = max(max_wg, n);
    }
    if (max_wg == min_wg) return;
    const int span = min_wg * rpw;  // rows of one piece
    for (int i = 0; i < g.njobs; ++i) pieces += (g.job[i].r1 - g.job[i].r0 + span - 1) / span;
    if (pieces > kMaxGemvJobs) return;
    GemvGroup out = g;
    out.njobs = 0;
    for (int i = 0; i < g.njobs; ++i) {
        const GemvJob &j = g.job[i];
        for (int r = j.r0; r < j.r1; r += span) {
            GemvJob p = j;
            p.r0 = r;
            p.r1 = min(j.r1, r + span);
            if (j.y) p.y = j.y + (r - j.r0);
            out.job[out.njobs++] = p;
        }
    }
    g = out;
}

template <int Q, int LPR, bool F32, int NW, int QPW>
static jk_status launch_fast_run(hipStream_t s, GemvGroup &g, size_t lds, int upg) {
    constexpr int RPU = 64 / LPR;
    even_out_jobs(g, upg * RPU);
    int wgs = 0;
    for (int i = 0; i < g.njobs; ++i) {
        const int units = (g.job[i].r1 - g.job[i].r0 + RPU - 1) / RPU;
        g.job[i].upg = upg;
        g.job[i].nwg = (units + upg - 1) / upg;
        wgs = max(wgs, g.job[i].nwg);
    }
    hipLaunchKernelGGL((gemv_q8_fast_kernel<Q, LPR, F32, NW, QPW>), dim3((unsigned)wgs, (unsigned)g.njobs), dim3(64 * NW),
                       lds, s, g);
    JK_TRY(check_launch("gemv_q8_fast_kernel"));
    return launch_group_argmax(s, g);
}

// Fast-kernel launch. Measured on MI355X: 8-wave workgroups with one unit per wave (about
// 3.5 workgroups per CU for the gate + up launch) beat one 16-wave workgroup per CU and
// two units per wave -- workgroups that start and stage their activation at different
// times keep the memory pipeline fuller. Launches with at most 4 units per CU use 4-wave
// workgroups, one per CU.
template <int Q, int LPR, bool F32>
static jk_status launch_fast(hipStream_t s, GemvGroup &g, size_t lds) {
    constexpr int RPU = 64 / LPR;
    long units = 0;
    for (int i = 0; i < g.njobs; ++i) units += (g.job[i].r1 - g.job[i].r0 + RPU - 1) / RPU;
    const long ncu = cu_count();
    const int upg = (int)std::max<long>(1, (units + ncu - 1) / ncu);
    if (upg <= 4) return launch_fast_run<Q, LPR, F32, 4, 1>(s, g, lds, upg);
    return launch_fast_run<Q, LPR, F32, 8, 1>(s, g, lds, 8);
}

// One job on the global-activation kernel (caller blocks only; validated by the callers).
template <int Q>
static jk_status launch_global_job(hipStream_t s, const GemvJob &j) {
    const int nwg = (j.r1 - j.r0 + 15) / 16;
    hipLaunchKernelGGL(gemv_q8_global_kernel<Q>, dim3((unsigned)nwg), dim3(256), 0, s, j.w, j.xq, j.y, j.r0, j.r1,
                       j.am_slots);
    JK_TRY(check_launch("gemv_q8_global_kernel"));
    if (j.am_slots) JK_TRY(launch_argmax_slots(s, j.am_slots, nwg, j.am_index));
    return JK_OK;
}

// One launch of jobs whose activations all fit the LDS budget and share an activation kind.
template <int Q>
static jk_status launch_staged_group(hipStream_t s, GemvGroup &g) {
    using T = QTraits<Q>;
    int max_nb = 0;
    for (int i = 0; i < g.njobs; ++i) max_nb = max(max_nb, g.job[i].w.nb);
    const size_t lds = (size_t)max_nb * T::XB;
    const bool f32 = g.job[0].xf != nullptr;
    const bool wide = T::K && max_nb > 32;  // one wave per row for long K-quant rows
    const int lpr = wide ? 64 : 16;
    if ((max_nb + lpr - 1) / lpr <= kFastU<Q>) {
        if (wide && f32) return launch_fast<Q, 64, true>(s, g, lds);
        if (wide) return launch_fast<Q, 64, false>(s, g, lds);
        if (f32) return launch_fast<Q, 16, true>(s, g, lds);
        return launch_fast<Q, 16, false>(s, g, lds);
    }
    // full workgroups when every CU gets at least one
    const int rpu = wide ? 1 : 4;
    long units = 0;
    for (int i = 0; i < g.njobs; ++i) units += (g.job[i].r1 - g.job[i].r0 + rpu - 1) / rpu;
    const bool full = units >= (long)cu_count() * kFullWaves<Q>;
    constexpr int FW = kFullWaves<Q>;
    if (wide && f32) return full ? launch_group_run<Q, 64, true, FW>(s, g, lds) : launch_group_run<Q, 64, true, 4>(s, g, lds);
    if (wide) return full ? launch_group_run<Q, 64, false, FW>(s, g, lds) : launch_group_run<Q, 64, false, 4>(s, g, lds);
    if (f32) return full ? launch_group_run<Q, 16, true, FW>(s, g, lds) : launch_group_run<Q, 16, true, 4>(s, g, lds);
    return full ? launch_group_run<Q, 16, false, FW>(s, g, lds) : launch_group_run<Q, 16, false, 4>(s, g, lds);
}

// Each job goes to the staged kernels when its own activation fits the LDS budget, else (caller
// blocks only: f32 jobs beyond the budget are refused by the callers before any launch) to the
// global-activation kernel. Staged jobs are launched together in runs of one activation kind.
template <int Q>
static jk_status launch_group_q(hipStream_t s, const GemvJob *jobs, int n) {
    using T = QTraits<Q>;
    GemvGroup g;
    memset(&g, 0, sizeof g);
    for (int i = 0; i < n; ++i) {
        const GemvJob &j = jobs[i];
        if ((size_t)j.w.nb * T::XB > (size_t)kMaxLdsX) {
            JK_TRY(launch_global_job<Q>(s, j));
            continue;
        }
        if (g.njobs > 0 && (g.njobs == kMaxGemvJobs || (g.job[0].xf != nullptr) != (j.xf != nullptr))) {
            JK_TRY(launch_staged_group<Q>(s, g));
            memset(&g, 0, sizeof g);
        }
        g.job[g.njobs++] = j;
    }
    if (g.njobs > 0) JK_TRY(launch_staged_group<Q>(s, g));
    return JK_OK;
}

size_t gemv_f32_max_cols(int q) {
    const int xb = fmt_of(q).be == 256 ? kXkBytes : kX0Bytes;
    return (size_t)(kMaxLdsX / xb) * (size_t)fmt_of(q).be;
}

// All jobs share one weight format and have r1 > r0 (checked by the callers).
jk_status launch_gemv_group(hipStream_t s, const GemvJob *jobs, int n) {
    if (n <= 0) return JK_OK;
    switch (jobs[0].w.quant) {
    case JK_Q4_0: return launch_group_q<JK_Q4_0>(s, jobs, n);
    case JK_Q5_0: return launch_group_q<JK_Q5_0>(s, jobs, n);
    case JK_Q8_0: return launch_group_q<JK_Q8_0>(s, jobs, n);
    case JK_Q4_K: return launch_group_q<JK_Q4_K>(s, jobs, n);
    case JK_Q5_K: return launch_group_q<JK_Q5_K>(s, jobs, n);
    case JK_Q6_K: return launch_group_q<JK_Q6_K>(s, jobs, n);
    case JK_TQ2_0: return launch_group_q<JK_TQ2_0>(s, jobs, n);
    default: return fail(JK_CAPABILITY_MISMATCH, "gemv: unsupported quant %d", jobs[0].w.quant);
    }
}

jk_status launch_gemv_q8(hipStream_t s, const WeightDev &w, const void *x, float *y, int r0, int r1) {
    GemvJob j;
    memset(&j, 0, sizeof j);
    j.w = w;
    j.xq = x;
    j.y = y;
    j.r0 = r0;
    j.r1 = r1;
    return launch_gemv_group(s, &j, 1);
}

}  // namespace jk
