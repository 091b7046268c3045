// jk_device.hpp -- device helpers shared by the libjk kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jk_internal.hpp"

namespace jk {

// f16_to_f32_finite (lib.rs:676-717): exact decode, NaN/Inf -> +0.0, signed zero kept. The low
// 16 bits of h are the f16. The hardware conversion is exact for every f16, subnormals included
// (the kernels run with f16 denormals preserved), so the decode is one conversion and a select.
__device__ __forceinline__ float f16_finite(uint32_t h) {
    const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    return __builtin_isfinite(f) ? f : 0.0f;
}

// Signed 4 x i8 dot product accumulated into c (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Value of the lane one position lower in the same 16-lane DPP row (lane 0 takes lane 15).
__device__ __forceinline__ float row_ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false));
}

// Ordered f32 accumulation across the 16 lanes of a DPP row: in step s the lane at row
// position s computes acc = acc(position s-1) + v, so after the 16 straight-line steps
// position 15 holds (((acc_in + v0) + v1) + ...) + v15 with acc_in taken from position 15.
// A row of g < 16 values passes -0.0 in positions g..15: x + (-0.0) == x for every x
// (+0 and -0 included), so position 15 then holds exactly the sum of the g values.
// Every lane of the wave must execute this.
__device__ __forceinline__ float chain_add(float acc, float v) {
#pragma unroll
    for (int s = 0; s < 16; ++s) acc = row_ror1(acc) + v;
    return acc;
}

// Chunk c of block b of row r in the plane layout.
__device__ __forceinline__ const uint4 *chunk_ptr(const WeightDev &w, int c, int r, int b) {
    return reinterpret_cast<const uint4 *>(
        w.planes + ((((size_t)c * (size_t)w.rows + (size_t)r) * (size_t)w.nb + (size_t)b) << 4));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Weight chunks are streamed exactly once per call: non-temporal 128-bit load.
__device__ __forceinline__ uint4 ld_chunk(const WeightDev &w, int c, int r, int b) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(chunk_ptr(w, c, r, b)));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ld_dscale(const WeightDev &w, int r, int b) {
    return f16_finite(w.dplane[(size_t)r * (size_t)w.nb + (size_t)b]);
}

// Byte i of a dword, and dword i of a 16-byte chunk.
__device__ __forceinline__ int byte_of(uint32_t v, int i) { return (int)((v >> (8 * i)) & 255u); }

__device__ __forceinline__ uint32_t comp(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Bytewise a - k for bytes that may borrow (k < 128 per byte): result bytes are the
// two's-complement i8 values of (byte - k).
__device__ __forceinline__ int bytes_sub(uint32_t a, uint32_t k) {
    return (int)(((a | 0x80808080u) - k) ^ 0x80808080u);
}

// Four 2-bit fields f (one per byte, values 0..3) to the signed bytes f - 1 by one byte permute:
// selector byte f picks byte f of 0x020100FF (v_perm_b32 reads selectors 0..3 from its second
// operand).
__device__ __forceinline__ uint32_t crumbs_minus1(uint32_t f) { return __builtin_amdgcn_perm(0u, 0x020100FFu, f); }

// Bits 0..3 of n moved to bit 4 of bytes 0..3 (the four shifted copies of n occupy
// disjoint bit ranges, so the multiply has no carries): the fifth bit of four 5-bit quants.
__device__ __forceinline__ uint32_t bit4_of_bytes(uint32_t n) { return ((n * 0x00204081u) & 0x01010101u) << 4; }

// KVALUES_IQ4NL (quant.rs:76-78) of four 4-bit indices, one per byte: two byte permutes over
// the 16-byte table (v_perm_b32 picks bytes 0..3 from its second source and 4..7 from its
// first, by the low 3 bits of each selector byte), then a per-byte select on index bit 3.
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t idx) {
    const uint32_t t0 = 0xBFAD9881u, t1 = 0xF6EADDCFu;  // -127 -104 -83 -65 | -49 -35 -22 -10
    const uint32_t t2 = 0x26190D01u, t3 = 0x71594535u;  //    1   13  25  38 |  53  69  89 113
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel), hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

// Word i of block b of row r in the word plane (fields of h_len bytes).
__device__ __forceinline__ uint32_t ld_word(const WeightDev &w, int r, int b, int h_len, int i) {
    return w.hplane[((size_t)r * (size_t)w.nb + (size_t)b) * (size_t)(h_len / 4) + (size_t)i];
}

// Rust `v.round().clamp(lo, hi) as i8`: round half away from zero, NaN -> 0.
__device__ __forceinline__ int rust_round_clamp_i8(float v, float lo, float hi) {
    float r = roundf(v);
    if (__builtin_isnan(r)) return 0;
    r = r < lo ? lo : r;
    r = r > hi ? hi : r;
    return (int)r;
}

// round_scaled_to_i8 (quant_q8.rs:102-108)
__device__ __forceinline__ int round_scaled_to_i8(float v, float inv) {
    if (!__builtin_isfinite(v)) return 0;
    return rust_round_clamp_i8(v * inv, -127.0f, 127.0f);
}

// DPP lane permutations (GFX9 encodings), all lanes of the row taking part:
// quad_perm [1,0,3,2] = lane ^ 1, quad_perm [2,3,0,1] = lane ^ 2, row_half_mirror
// (lane i <-> 7 - i within 8), row_mirror (lane i <-> 15 - i within 16).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// Maximum / sum over aligned groups of 4, 8 or 16 lanes; every lane of a group gets it.
__device__ __forceinline__ float max8_dpp(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}
__device__ __forceinline__ int sum4_dpp(int v) {
    v += dpp_i<kDppXor1>(v);
    return v + dpp_i<kDppXor2>(v);
}
__device__ __forceinline__ int sum8_dpp(int v) {
    v = sum4_dpp(v);
    return v + dpp_i<kDppHalfMirror>(v);
}

// Maximum over the whole wave (all lanes active), returned wave-uniform.
__device__ __forceinline__ float wave_max64_dpp(float v) {
    v = max8_dpp(v);
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float e = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, e));
}
// Sum over the whole wave (all lanes active), returned wave-uniform.
__device__ __forceinline__ int wave_sum64_dpp(int v) {
    v = sum8_dpp(v);
    v += dpp_i<kDppMirror>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

template <int W>
__device__ __forceinline__ float wave_max(float v) {
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, W));
    return v;
}

// Ordered workgroup barrier for LDS traffic only: outstanding global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Makes this wave's LDS writes visible to the other lanes of the same wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Ordered fold of one value per lane over a whole wave: lane 0 adds the values of lanes
// 0..63 in lane order to acc (acc lives in lane 0); lanes past the row end pass -0.0, the
// exact identity of f32 addition. red: 64 floats of 16-byte aligned LDS for this wave, read
// 16 at a time with the next 16 requested before the current 16 are added.
__device__ __forceinline__ float fold_wave(float acc, float v, float *red) {
    const int l = threadIdx.x & 63;
    red[l] = v;
    wave_lds_sync();
    if (l == 0) {
        const float4 *r4 = reinterpret_cast<const float4 *>(red);
        float4 cur[4], nxt[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) cur[i] = r4[i];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (c < 3)
#pragma unroll
                for (int i = 0; i < 4; ++i) nxt[i] = r4[4 * (c + 1) + i];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = (((acc + cur[i].x) + cur[i].y) + cur[i].z) + cur[i].w;
            if (c < 3)
#pragma unroll
                for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
        }
    }
    wave_lds_sync();
    return acc;
}

// ------------------------------------------------------------ gated activations
// swiglu_f32_scalar (swiglu.rs:98-121) and relu_squared_gate_scalar (lib.rs:1140-1147) of one
// element; ACT 0 passes g through. expf is the library's single-precision exponential.
constexpr int kActNone = 0, kActSwiglu = 1, kActRelu2 = 2;
template <int ACT>
__device__ __forceinline__ float gated(float g, float u) {
    if constexpr (ACT == kActSwiglu) {
        const float silu = g < -20.0f ? 0.0f : (g > 20.0f ? g : g / (1.0f + expf(-g)));
        return silu * u;
    } else if constexpr (ACT == kActRelu2) {
        const float relu = g > 0.0f ? g : 0.0f;
        return relu * relu * u;
    } else {
        return g;
    }
}

// ------------------------------------------------------------ argmax keys
// argmax_f32_scalar (lib.rs:555-568) as a maximum over 64-bit keys: the high word orders the
// values (sign-magnitude bits mapped to an unsigned order, -0.0 folded onto +0.0 because the
// two compare equal), the low word is ~index so that among equal values the lowest index has
// the largest key. NaN maps to 0, below every value's key (-inf's key is 0x007FFFFF << 32).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    if (__builtin_isnan(v)) return 0ull;
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ int argmax_index(unsigned long long key) {
    return key == 0ull ? -1 : (int)(0xFFFFFFFFu - (uint32_t)key);
}
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long t = __shfl_xor(k, o, 64);
        k = t > k ? t : k;
    }
    return k;
}

// Workgroup maximum of every thread's key, stored by thread 0 to *slot (plain store: the slots
// of a launch are reduced by the next kernel on the stream, after this launch has completed --
// no device-scope atomics or fences, which on this part would serialize across the XCDs' L2s).
// Every thread of the workgroup must call it. s_keys: one LDS slot per wave; nw waves.
__device__ __forceinline__ void argmax_store_wg(unsigned long long key, unsigned long long *slot,
                                                unsigned long long *s_keys, int nw) {
    key = wave_max_key(key);
    const int t = threadIdx.x;
    if ((t & 63) == 0) s_keys[t >> 6] = key;
    __syncthreads();
    if (t == 0) {
        unsigned long long k = 0ull;
        for (int i = 0; i < nw; ++i) k = s_keys[i] > k ? s_keys[i] : k;
        *slot = k;
    }
}

// ------------------------------------------------- global-to-LDS loads (no staging registers)
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

// One global-to-LDS load of 16 (or 4) bytes per lane into the LDS span starting at byte lds
// (M0). Written as inline asm so that the compiler's wait insertion, which cannot tell the two
// stages' loads apart across the loop, does not drain the other stage's loads before every
// read of this one; the kernel waits for its own loads explicitly (vmcnt) instead. No
// compiler-issued global load shares the loop, so those explicit counts are exact.
__device__ __forceinline__ void lds_dma16(const void *src, const lds_u8_t *lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"((unsigned)(size_t)lds) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *src, const lds_u8_t *lds) {
    asm volatile("global_load_lds_dword %0, off" ::"v"(src), "{m0}"((unsigned)(size_t)lds) : "memory");
}

// s_waitcnt vmcnt(n) (GFX9 encoding; expcnt and lgkmcnt left unconstrained)
#define JK_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | ((((n) >> 4) & 3) << 14) | (7 << 4) | (15 << 8))
// Workgroup barrier between the stage phases with the waits made explicit: a wave has already
// waited for its own loads into the stage (vmcnt) and waits here for its own LDS reads (lgkmcnt);
// the compiler-only fences keep memory accesses on their side of the barrier. (A release fence
// would also wait for the loads into the other stage: LDS-bound loads count as LDS writes.)
__device__ __forceinline__ void stage_barrier() {
    __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace jk
