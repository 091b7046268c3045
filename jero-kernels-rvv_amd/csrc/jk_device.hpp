// jk_device.hpp -- device helpers shared by the libjk kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jk_internal.hpp"

namespace jk {

// f16_to_f32_finite (lib.rs:676-717): exact decode, NaN/Inf -> +0.0, signed zero kept.
__device__ __forceinline__ float f16_finite(uint32_t h) {
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u, s = (h & 0x8000u) << 16;
    if (e == 31u) return 0.0f;
    if (e == 0u) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-24f));
    return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
}

// Signed 4 x i8 dot product accumulated into c (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Value of the lane one position lower in the same 16-lane DPP row (lane 0 takes lane 15).
__device__ __forceinline__ float row_ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false));
}

// Ordered f32 accumulation across the 16 lanes of a DPP row: for s in 0..g, the lane at
// row position s computes acc = acc(position s-1) + v, so after g steps position g-1
// holds (((acc_in + v0) + v1) + ...) + v(g-1) with acc_in taken from position 15.
// Every lane of the wave must execute this (g is wave-uniform).
__device__ __forceinline__ float chain_add(float acc, float v, int g) {
    for (int s = 0; s < g; ++s) acc = row_ror1(acc) + v;
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

// Bytewise a - k for bytes that may borrow (k < 128 per byte): result bytes are the
// two's-complement i8 values of (byte - k).
__device__ __forceinline__ int bytes_sub(uint32_t a, uint32_t k) {
    return (int)(((a | 0x80808080u) - k) ^ 0x80808080u);
}

}  // namespace jk
