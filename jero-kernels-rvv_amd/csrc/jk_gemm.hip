// jk_gemm.hip -- prefill GEMM on int8 MFMA for the repacked (block-scaled i8) model.
//
// out[m][n] = sum over scale groups g, in K order, starting from 0.0:
//     acc += f32(sum_k xq[m][k] * wq[n][k]) * (xs[m][b32(g)] * ws[n][g])  [- xsum * wm]
// (execute_gemm_repacked_rows, repack.rs:2718-3042, accumulate_scaled_tile_scalar
// 3045-3093). One MFMA covers exactly one scale group (v_mfma_i32_32x32x32_i8 for the
// 32-element groups, v_mfma_i32_32x32x16_i8 for Q6_K's 16-element groups), so every
// group's integer partial is exact and the f32 epilogue runs per group in K order: each
// output keeps the reference's arithmetic and order, bit for bit.
//
// Tiling: a workgroup computes a TN (weight rows) x TM (tokens) tile with 2 TN threads, two
// per weight row when staging. Each wave computes up to 64 x 32 outputs as 32x32 MFMA tiles.
// K advances in chunks of 128 elements (4 steps of 32; half a super-block of the
// 256-element formats). While the 4 steps of a chunk are evaluated from LDS, the next chunk
// is loaded into registers with coalesced reads -- every thread a share of both tiles -- and
// after a barrier it is unpacked to i8 and written to LDS. LDS rows are padded from 128 to
// 144 bytes so the 16-byte fragment reads of 16 lanes land on distinct banks.
// Tile shapes: 128 x 64 (4 waves, 35 KB of LDS, <= 168 VGPRs: three workgroups per CU, so
// while one waits at its barrier or on its loads the others compute) for large launches;
// 64 x 64 (2 waves) and 32 x 32 (1 wave) when the large tiles would leave CUs idle.
#include <string.h>

#include "jk_device.hpp"

namespace jk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

// Integer MFMA results as f32 without a conversion instruction: the accumulator starts at the
// bit pattern of 1.5 * 2^23, so the i32 sum adds the group's dot product d to that float's
// mantissa. |d| <= 32 * 128 * 128 < 2^22 keeps it in the binade [2^23, 2^24), where the float
// is exactly 1.5 * 2^23 + d, and one exact subtraction recovers d -- cheaper to issue than
// v_cvt_f32_i32. The bias registers are never written (the MFMA's result goes elsewhere), at
// 16 VGPRs: used where the epilogue's issue time dominates and registers allow (the 512-token
// tolerance tiles; measured slower in the split-K and the bit-exact tiles, whose register
// budgets it crowds).
constexpr int kMagicBits = 0x4B400000;
constexpr float kMagicF = 12582912.0f;  // 1.5 * 2^23
__device__ __forceinline__ v16i magic_acc() {
    v16i m;
#pragma unroll
    for (int v = 0; v < 16; ++v) m[v] = kMagicBits;
    return m;
}
__device__ __forceinline__ float unbias(int c) { return __int_as_float(c) - kMagicF; }

constexpr int kKC = 128;      // K elements per chunk
constexpr int kSteps = 4;     // 32-element steps per chunk
constexpr int kRowB = 144;    // padded LDS bytes per 128-byte row

template <int Q> struct GemmFmt {
    static constexpr int GK = Q == JK_Q6_K || Q == JK_Q3_K || Q == JK_Q2_K ? 16 : 32;  // elements per scale group
    static constexpr bool MINS = Q == JK_Q4_K || Q == JK_Q5_K || Q == JK_Q4_1 || Q == JK_Q5_1 || Q == JK_Q2_K;
    static constexpr int NG = 128 / GK;                 // scale groups per chunk
    static constexpr int NM = MINS ? NG : 1;            // min / activation-sum rows staged per chunk
    // 32-element blocks, 4 per chunk, staged like Q4_0
    static constexpr bool B32 = Q == JK_Q8_0 || Q == JK_Q4_0 || Q == JK_Q5_0 || Q == JK_Q4_1 || Q == JK_Q5_1 ||
                                Q == JK_IQ4_NL;
};

template <int TN, int TM> struct Tile {
    static constexpr int THREADS = 2 * TN;        // two staging threads per weight row
    static constexpr int WAVES = THREADS / 64;
    static constexpr int RW = TN < 64 ? TN : 64;  // weight rows per wave
    static constexpr int NT = RW / 32;            // 32-row MFMA blocks per wave
    static constexpr int WR = TN / RW;            // waves along the rows
    static constexpr int WM = TM < 32 ? 1 : TM / 32;  // waves along the tokens
    static constexpr int XL = 8 * TM / THREADS;   // activation loads per thread and chunk
    static constexpr int XS = 4 * TM / THREADS;   // activation scales per thread and chunk
    static constexpr int XS16 = 8 * TM / THREADS; // activation 16-sums per thread and chunk (Q2_K)
    static constexpr int WPE = TN == 128 ? 3 : 2;  // waves per SIMD the register budget allows
    // (a wave covers 32 tokens, or 64 in the tolerance kernel's 128 x 128 tiles)
    static_assert((WR * WM) % WAVES == 0 && XL >= 1 && XS >= 1 && XS <= 4, "tile shape");
};

template <int Q, int TN, int TM> struct GemmChunk {
    static constexpr int NM = GemmFmt<Q>::NM;
    uint8_t a[TN * kRowB];  // weights, i8, [row][k]
    uint8_t b[TM * kRowB];  // activations, i8, [token][k]
    float ws[8][TN];        // weight scale per scale group of the chunk
    float wm[NM][TN];       // weight min per scale group (formats with mins)
    float xs[4][TM];        // activation scale per 32-block
    float xm[NM][TM];       // activation sum per scale group: per 32-block, or per 16 (Q2_K)
};

// Writes of 16 i8 values (K elements koff .. koff + 15 of one tile row) into a chunk's LDS
// tiles: the i8 tiles keep them as bytes in padded rows.
template <int Q, int TN, int TM>
__device__ __forceinline__ void put_a(GemmChunk<Q, TN, TM> &c, int row, int koff, uint4 v) {
    *reinterpret_cast<uint4 *>(c.a + row * kRowB + koff) = v;
}
template <int Q, int TN, int TM>
__device__ __forceinline__ void put_b(GemmChunk<Q, TN, TM> &c, int tok, int koff, uint4 v) {
    *reinterpret_cast<uint4 *>(c.b + tok * kRowB + koff) = v;
}

// One 16-byte global load without the streaming hint: a weight tile is read once per
// token tile, so its lines are meant to stay in L2 for the neighbouring workgroups.
__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ __forceinline__ const uint8_t *plane_ptr(const WeightDev &w, int c, int r, int b) {
    return w.planes + ((((size_t)c * (size_t)w.rows + (size_t)r) * (size_t)w.nb + (size_t)b) << 4);
}

// Raw bytes of one thread's share of a chunk, exactly as stored in the plane layout, plus
// raw f16 scales. Loading and unpacking are separate so that every global load of a chunk
// is in flight while the previous chunk is evaluated; nothing between the loads depends on
// a loaded value. Every thread stages part of both tiles, so the four waves (one per SIMD)
// carry the same load and unpack work.
//  Q8_0 / Q4_0 / Q5_0: a chunk is 4 blocks, 64 contiguous bytes per (plane, row); 4
//   consecutive lanes read one such segment (piece t % 4 = block 4kc + t % 4), load i covers
//   rows t / 4 + TN/2 (i % 2) of plane i / 2 (Q5_0: with the word of the same block).
//   Scales: row t / 2, blocks 4kc + 2 (t % 2) ...
//  K-quants, TQ2_0 (256-element blocks): chunk kc is half h = kc % 2 of block kc / 2;
//   I2_S (128-element blocks): chunk kc is block kc. Thread t takes row t / 2 and part
//   j = t % 2 of the chunk's planes.
//  Activations: load i covers token t / 8 + (threads / 8) i, piece t % 8 of its 128-byte
//   row; scale j (and sum) of entry e = XS t + j: token e / 4, block 4kc + e % 4.
template <int TN, int TM> struct Stage {
    uint4 w[5];                         // weight plane bytes
    uint32_t wd[2];                     // weight scales: f16 d (or the d | m word) of two blocks; K-formats: d
    uint32_t wh[2];                     // Q5_0 / Q5_1: high-bit words of the blocks of w[0], w[1]
    uint4 x[Tile<TN, TM>::XL];          // activation bytes
    uint32_t xd[2][Tile<TN, TM>::XS];   // activation scale, sum per 32-block
    uint32_t x16[Tile<TN, TM>::XS16];   // activation sums per 16 (Q2_K)
};

// Blocks past the row end (a partial last chunk) are read clamped and never used; rows
// past r1 are read clamped to r1 - 1 and never stored.
// XV (whole chunks, nb % 4 == 0): the two f16 scales of a thread's blocks in one 4-byte load.
template <int Q, int TN, int TM, bool XV = false>
__device__ __forceinline__ void chunk_w_load(const WeightDev &w, int n0, int r1, int kc, Stage<TN, TM> &r) {
    const int nb = w.nb, t = (int)threadIdx.x % Tile<TN, TM>::THREADS;
    if constexpr (GemmFmt<Q>::B32) {
        constexpr int HW = fmt_of(Q).h_len / 4;  // words per block in the word plane
        const int b = min(4 * kc + (t & 3), nb - 1);
#pragma unroll
        for (int i = 0; i < (Q == JK_Q8_0 ? 4 : 2); ++i) {
            const int n = min(n0 + (t >> 2) + TN / 2 * (i & 1), r1 - 1);
            r.w[i] = ldg16(plane_ptr(w, i >> 1, n, b));
            if constexpr (Q == JK_Q5_0) r.wh[i] = w.hplane[(size_t)n * (size_t)nb + (size_t)b];
            if constexpr (Q == JK_Q5_1) r.wh[i] = w.hplane[((size_t)n * (size_t)nb + (size_t)b) * 2 + 1];
        }
        const size_t srow = (size_t)min(n0 + (t >> 1), r1 - 1) * (size_t)nb;
        if constexpr (XV && Q != JK_Q4_1 && Q != JK_Q5_1) {
            const uint32_t dd = *reinterpret_cast<const uint32_t *>(w.dplane + srow + (size_t)(4 * kc + 2 * (t & 1)));
            r.wd[0] = dd & 0xFFFFu;
            r.wd[1] = dd >> 16;
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const size_t blk = srow + (size_t)min(4 * kc + 2 * (t & 1) + j, nb - 1);
                if constexpr (Q == JK_Q4_1 || Q == JK_Q5_1) r.wd[j] = w.hplane[blk * HW];  // d | m << 16
                else r.wd[j] = w.dplane[blk];
            }
        }
    } else {
        const int n = min(n0 + (t >> 1), r1 - 1), j = t & 1;
        if constexpr (Q == JK_I2_S) {
            r.w[0] = ldg16(plane_ptr(w, j, n, min(kc, nb - 1)));
            return;
        }
        const int h = kc & 1, b = kc >> 1;
        if constexpr (Q == JK_Q4_K) {
            r.w[0] = ldg16(plane_ptr(w, 0, n, b));  // d, dmin, 12 packed 6-bit scales / mins
            r.w[1] = ldg16(plane_ptr(w, 1 + 2 * (2 * h + j), n, b));
            r.w[2] = ldg16(plane_ptr(w, 2 + 2 * (2 * h + j), n, b));
        } else if constexpr (Q == JK_Q5_K) {
            r.w[0] = ldg16(plane_ptr(w, 0, n, b));  // d, dmin, 12 packed 6-bit scales / mins
            r.w[1] = ldg16(plane_ptr(w, 3 + 2 * (2 * h + j), n, b));
            r.w[2] = ldg16(plane_ptr(w, 4 + 2 * (2 * h + j), n, b));
            r.w[3] = ldg16(plane_ptr(w, 1, n, b));  // qh[0..16)
            r.w[4] = ldg16(plane_ptr(w, 2, n, b));  // qh[16..32)
        } else if constexpr (Q == JK_Q2_K) {
            r.w[0] = ldg16(plane_ptr(w, 0, n, b));          // 16 scale / min bytes
            r.w[1] = ldg16(plane_ptr(w, 1 + 2 * h, n, b));  // qs of the half, bytes 0..15
            r.w[2] = ldg16(plane_ptr(w, 2 + 2 * h, n, b));  // qs of the half, bytes 16..31
            r.wd[0] = w.hplane[(size_t)n * (size_t)nb + (size_t)b];  // d | dmin << 16
        } else if constexpr (Q == JK_Q3_K) {
            r.w[0] = ldg16(plane_ptr(w, 0, n, b));          // hmask bytes 0..15
            r.w[1] = ldg16(plane_ptr(w, 1, n, b));          // hmask bytes 16..31
            r.w[2] = ldg16(plane_ptr(w, 2 + 2 * h, n, b));  // qs of the half, bytes 0..15
            r.w[3] = ldg16(plane_ptr(w, 3 + 2 * h, n, b));  // qs of the half, bytes 16..31
            r.w[4] = ldg16(plane_ptr(w, 6, n, b));          // 12 packed scales, d
        } else if constexpr (Q == JK_Q6_K) {
            r.w[0] = ldg16(plane_ptr(w, 4 * h + j, n, b));      // ql, quarters 0 and 2
            r.w[1] = ldg16(plane_ptr(w, 4 * h + j + 2, n, b));  // ql, quarters 1 and 3
            r.w[2] = ldg16(plane_ptr(w, 8 + 2 * h + j, n, b));  // qh
            r.w[3] = ldg16(plane_ptr(w, 12, n, b));             // i8 scales
            r.wd[0] = w.dplane[(size_t)n * (size_t)nb + (size_t)b];
        } else {  // JK_TQ2_0
            r.w[0] = ldg16(plane_ptr(w, 2 * h + j, n, b));
            r.wd[0] = w.dplane[(size_t)n * (size_t)nb + (size_t)b];
        }
    }
}

// XV: a thread's XS (2 or 4) scale entries are consecutive blocks of one token, read with one
// 8- or 16-byte load per array instead of XS loads that each touch a different line per lane.
// The caller guarantees whole chunks, k_blocks32 % 4 == 0 and 16-byte aligned scales / sums.
template <int Q, int TN, int TM, bool XV = false>
__device__ __forceinline__ void chunk_x_load(const jk_act_q8 &a, int m0, int M, int kc, Stage<TN, TM> &r) {
    using T = Tile<TN, TM>;
    const int t = (int)threadIdx.x % T::THREADS;
    int k = kKC * kc + 16 * (t & 7);
    if (k >= (int)a.k_padded) k = 0;  // past the row end (partial chunk): in bounds, unused
#pragma unroll
    for (int i = 0; i < T::XL; ++i) {
        const int m = min(m0 + (t >> 3) + T::THREADS / 8 * i, M - 1);
        r.x[i] = ldg16(reinterpret_cast<const uint8_t *>(a.qs) + (size_t)m * a.k_padded + k);
    }
    constexpr bool SUMS = GemmFmt<Q>::MINS && GemmFmt<Q>::GK == 32;
    if constexpr (XV && (T::XS == 2 || T::XS == 4)) {
        const int e = T::XS * t;
        const size_t sidx = (size_t)min(m0 + (e >> 2), M - 1) * a.k_blocks32 + (size_t)(4 * kc + (e & 3));
        if constexpr (T::XS == 4) {
            const float4 v = *reinterpret_cast<const float4 *>(a.scales + sidx);
            r.xd[0][0] = __float_as_uint(v.x), r.xd[0][1] = __float_as_uint(v.y);
            r.xd[0][2] = __float_as_uint(v.z), r.xd[0][3] = __float_as_uint(v.w);
            if constexpr (SUMS) {
                const float4 u = *reinterpret_cast<const float4 *>(a.sums + sidx);
                r.xd[1][0] = __float_as_uint(u.x), r.xd[1][1] = __float_as_uint(u.y);
                r.xd[1][2] = __float_as_uint(u.z), r.xd[1][3] = __float_as_uint(u.w);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) r.xd[1][j] = 0u;
            }
        } else {
            const float2 v = *reinterpret_cast<const float2 *>(a.scales + sidx);
            r.xd[0][0] = __float_as_uint(v.x), r.xd[0][1] = __float_as_uint(v.y);
            if constexpr (SUMS) {
                const float2 u = *reinterpret_cast<const float2 *>(a.sums + sidx);
                r.xd[1][0] = __float_as_uint(u.x), r.xd[1][1] = __float_as_uint(u.y);
            } else {
                r.xd[1][0] = r.xd[1][1] = 0u;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < T::XS; ++j) {
            const int e = T::XS * t + j;
            const size_t sidx =
                (size_t)min(m0 + (e >> 2), M - 1) * a.k_blocks32 + (size_t)min(4 * kc + (e & 3), (int)a.k_blocks32 - 1);
            r.xd[0][j] = __float_as_uint(a.scales[sidx]);
            r.xd[1][j] = SUMS ? __float_as_uint(a.sums[sidx]) : 0u;
        }
    }
    if constexpr (GemmFmt<Q>::MINS && GemmFmt<Q>::GK == 16) {  // x_sums_16 (repack.rs:3061-3066)
#pragma unroll
        for (int j = 0; j < T::XS16; ++j) {
            const int e = T::XS16 * t + j;
            const size_t sidx = (size_t)min(m0 + (e >> 3), M - 1) * a.k_chunks +
                                (size_t)min(8 * kc + (e & 7), (int)a.k_chunks - 1);
            r.x16[j] = __float_as_uint(a.sums16[sidx]);
        }
    }
}

// Global loads of chunk kc into this thread's staging registers.
template <int Q, bool XV = false, int TN, int TM>
__device__ __forceinline__ void chunk_load(Stage<TN, TM> &r, const WeightDev &w, const jk_act_q8 &a, int n0, int r1,
                                           int m0, int M, int kc) {
    chunk_w_load<Q, TN, TM, XV>(w, n0, r1, kc, r);
    chunk_x_load<Q, TN, TM, XV>(a, m0, M, kc, r);
}

__device__ __forceinline__ uint4 nib4(uint4 v, int sh, uint32_t bias) {
    return make_uint4((uint32_t)bytes_sub((v.x >> sh) & 0x0F0F0F0Fu, bias), (uint32_t)bytes_sub((v.y >> sh) & 0x0F0F0F0Fu, bias),
                      (uint32_t)bytes_sub((v.z >> sh) & 0x0F0F0F0Fu, bias), (uint32_t)bytes_sub((v.w >> sh) & 0x0F0F0F0Fu, bias));
}
__device__ __forceinline__ uint4 crumb4(uint4 v, int sh) {
    return make_uint4(crumbs_minus1((v.x >> sh) & 0x03030303u), crumbs_minus1((v.y >> sh) & 0x03030303u),
                      crumbs_minus1((v.z >> sh) & 0x03030303u), crumbs_minus1((v.w >> sh) & 0x03030303u));
}

// Unpack the staging registers to i8 with repack_block_scaled_range_into_i8's values
// (repack.rs:1724-2103) and write them, with the scale (and min) of each scale group, to
// the chunk's LDS tiles.
template <int Q, int TN, int TM, class Chunk>
__device__ __forceinline__ void chunk_store(const WeightDev &w, const Stage<TN, TM> &r, Chunk &c, int kc) {
    using T = Tile<TN, TM>;
    using F = GemmFmt<Q>;
    const int t = (int)threadIdx.x % T::THREADS;
    {  // activations
#pragma unroll
        for (int i = 0; i < T::XL; ++i) put_b(c, (t >> 3) + T::THREADS / 8 * i, 16 * (t & 7), r.x[i]);
#pragma unroll
        for (int j = 0; j < T::XS; ++j) {
            const int e = T::XS * t + j;
            c.xs[e & 3][e >> 2] = __uint_as_float(r.xd[0][j]);
            if constexpr (F::MINS && F::GK == 32) c.xm[e & 3][e >> 2] = __uint_as_float(r.xd[1][j]);
        }
        if constexpr (F::MINS && F::GK == 16)
#pragma unroll
            for (int j = 0; j < T::XS16; ++j) {
                const int e = T::XS16 * t + j;
                c.xm[e & 7][e >> 3] = __uint_as_float(r.x16[j]);
            }
    }
    if constexpr (F::B32) {
        const int piece = t & 3;
#pragma unroll
        for (int i = 0; i < (Q == JK_Q8_0 ? 4 : 2); ++i) {
            const int arow = (t >> 2) + TN / 2 * (i & 1), k0 = 32 * piece;
            if constexpr (Q == JK_Q8_0) {
                put_a(c, arow, k0 + 16 * (i >> 1), r.w[i]);
            } else if constexpr (Q == JK_Q4_1) {  // unpack_q4_1_block_i8 (quant.rs:117-129): the nibbles
                put_a(c, arow, k0, nib4(r.w[i], 0, 0u));
                put_a(c, arow, k0 + 16, nib4(r.w[i], 4, 0u));
            } else if constexpr (Q == JK_Q5_1) {  // unpack_q5_1_block_i8 (quant.rs:168-187): nibble | 16 * bit
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t v = comp(r.w[i], k), qh = r.wh[i];
                    lo[k] = (v & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (4 * k)) & 15u);
                    hi[k] = ((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (16 + 4 * k)) & 15u);
                }
                put_a(c, arow, k0, make_uint4(lo[0], lo[1], lo[2], lo[3]));
                put_a(c, arow, k0 + 16, make_uint4(hi[0], hi[1], hi[2], hi[3]));
            } else if constexpr (Q == JK_IQ4_NL) {  // unpack_iq4_nl_block_i8 (quant.rs:333-345)
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    lo[k] = iq4nl_lookup(comp(r.w[i], k) & 0x0F0F0F0Fu);
                    hi[k] = iq4nl_lookup((comp(r.w[i], k) >> 4) & 0x0F0F0F0Fu);
                }
                put_a(c, arow, k0, make_uint4(lo[0], lo[1], lo[2], lo[3]));
                put_a(c, arow, k0 + 16, make_uint4(hi[0], hi[1], hi[2], hi[3]));
            } else if constexpr (Q == JK_Q5_0) {
                // unpack_q5_0_block_i8 (quant.rs:139-157): (nibble | 16 * bit) - 16, bit j of
                // the word for element j
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t v = comp(r.w[i], k), qh = r.wh[i];
                    lo[k] = (uint32_t)bytes_sub((v & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (4 * k)) & 15u), 0x10101010u);
                    hi[k] = (uint32_t)bytes_sub(((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes((qh >> (16 + 4 * k)) & 15u),
                                                0x10101010u);
                }
                put_a(c, arow, k0, make_uint4(lo[0], lo[1], lo[2], lo[3]));
                put_a(c, arow, k0 + 16, make_uint4(hi[0], hi[1], hi[2], hi[3]));
            } else {
                put_a(c, arow, k0, nib4(r.w[i], 0, 0x08080808u));
                put_a(c, arow, k0 + 16, nib4(r.w[i], 4, 0x08080808u));
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            c.ws[2 * (t & 1) + j][t >> 1] = f16_finite(r.wd[j] & 0xFFFFu);
            if constexpr (Q == JK_Q4_1 || Q == JK_Q5_1) {  // repack.rs:1814-1860: min stored as -m
                const float m = f16_finite(r.wd[j] >> 16);
                c.wm[2 * (t & 1) + j][t >> 1] = m == 0.0f ? 0.0f : -m;
            }
        }
        return;
    }
    const int row = t >> 1, j = t & 1, h = kc & 1;
    if constexpr (Q == JK_Q4_K) {
        // unpack_k4_scales_mins (repack.rs:1158-1170); qs planes (1 + 2c', 2 + 2c') of
        // super-block quarter c' = 2h + j hold elements 64j .. 64j + 63 of the half: low
        // nibbles of both planes, then high nibbles
        const uint4 hd = r.w[0];
        const float d = f16_finite(hd.x & 0xFFFFu), dmin = f16_finite(hd.x >> 16);
        const uint32_t sc = h == 0 ? (hd.y & 0x3F3F3F3Fu) : ((hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u));
        const uint32_t mv = h == 0 ? (hd.z & 0x3F3F3F3Fu) : (((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int g = 2 * j + e;
            c.ws[g][row] = d * (float)((sc >> (8 * g)) & 255u);
            c.wm[g][row] = dmin * (float)((mv >> (8 * g)) & 255u);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            put_a(c, row, 64 * j + 32 * hh, nib4(r.w[1], 4 * hh, 0u));
            put_a(c, row, 64 * j + 32 * hh + 16, nib4(r.w[2], 4 * hh, 0u));
        }
    } else if constexpr (Q == JK_Q5_K) {
        // The Q4_K arm with the Q5_K bits (repack.rs:1959-2002): quarter c' = 2h + j takes qs
        // planes 3 + 2c', 4 + 2c'; element l (l < 32) of its low half adds 16 * bit 2c' of
        // qh[l], element 32 + l of its high half bit 2c' + 1
        const uint4 hd = r.w[0];
        const float d = f16_finite(hd.x & 0xFFFFu), dmin = f16_finite(hd.x >> 16);
        const uint32_t sc = h == 0 ? (hd.y & 0x3F3F3F3Fu) : ((hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u));
        const uint32_t mv = h == 0 ? (hd.z & 0x3F3F3F3Fu) : (((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int g = 2 * j + e;
            c.ws[g][row] = d * (float)((sc >> (8 * g)) & 255u);
            c.wm[g][row] = dmin * (float)((mv >> (8 * g)) & 255u);
        }
        const int qsh = 2 * (2 * h + j);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint4 qv = r.w[1 + p], hv = r.w[3 + p];
                uint32_t o[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[k] = ((comp(qv, k) >> (4 * hh)) & 0x0F0F0F0Fu) | (((comp(hv, k) >> (qsh + hh)) & 0x01010101u) << 4);
                put_a(c, row, 64 * j + 32 * hh + 16 * p, make_uint4(o[0], o[1], o[2], o[3]));
            }
    } else if constexpr (Q == JK_Q2_K) {
        // unpack_q2_k_block_i8 (quant.rs:197-235), repack.rs:1876-1895: 16-group g = 2 jq + part of
        // the half (jq = 2j .. 2j + 1 here) is the 2-bit field 2 jq of qs bytes 16 part .. of the half;
        // scale d * (sc & 15), min dmin * (sc >> 4) with sc = scales[8h + g]
        const float d = f16_finite(r.wd[0] & 0xFFFFu), dmin = f16_finite(r.wd[0] >> 16);
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
            const int jq = 2 * j + jo;
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const int g = 2 * jq + part;
                const uint32_t sc = (comp(r.w[0], (8 * h + g) >> 2) >> (8 * ((8 * h + g) & 3))) & 255u;
                c.ws[g][row] = d * (float)(sc & 15u);
                c.wm[g][row] = dmin * (float)(sc >> 4);
                const uint4 qv = r.w[1 + part];
                put_a(c, row, 32 * jq + 16 * part,
                      make_uint4((qv.x >> (2 * jq)) & 0x03030303u, (qv.y >> (2 * jq)) & 0x03030303u,
                                 (qv.z >> (2 * jq)) & 0x03030303u, (qv.w >> (2 * jq)) & 0x03030303u));
            }
        }
    } else if constexpr (Q == JK_Q3_K) {
        // unpack_q3_k_block_i8 (quant.rs:254-317), repack.rs:1896-1911: 16-group g = 2 jq + part of
        // the half takes the 2-bit field 2 jq of qs bytes 16 part .. of the half, minus 4 where bit
        // 4h + jq of hmask byte 16 part + l is clear; scale d * (6-bit scale 8h + g - 32)
        const uint4 tail = r.w[4];
        const float d = f16_finite(tail.w & 0xFFFFu);
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
            const int jq = 2 * j + jo;
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const int g = 2 * jq + part, is = 8 * h + g;
                const uint32_t lb = (comp(tail, (is & 7) >> 2) >> (8 * (is & 3))) & 255u;
                const uint32_t lo = is < 8 ? (lb & 15u) : (lb >> 4);
                const uint32_t hi = (((tail.z >> (8 * (is & 3))) & 255u) >> (2 * (is >> 2))) & 3u;
                c.ws[g][row] = d * (float)((int)(lo | (hi << 4)) - 32);
                const uint4 qv = r.w[2 + part], hv = r.w[part];
                uint32_t o[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t v = (comp(qv, k) >> (2 * jq)) & 0x03030303u;
                    const uint32_t hb = (comp(hv, k) >> (4 * h + jq)) & 0x01010101u;
                    o[k] = (uint32_t)bytes_sub(v | (hb << 2), 0x04040404u);
                }
                put_a(c, row, 32 * jq + 16 * part, make_uint4(o[0], o[1], o[2], o[3]));
            }
        }
    } else if constexpr (Q == JK_Q6_K) {
        // dequantize_q6_k_block's element order (quant.rs:594-648): 16-group g = j + 2 qq of
        // half h (quarter qq) takes ql bytes 16j + 32(qq % 2) of the half, qh bytes 16j, the
        // low / high nibble and 2-bit field by quarter, scale 8h + g
        const float d = f16_finite(r.wd[0]);
        const uint4 scv = r.w[3], hv = r.w[2];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int g = j + 2 * qq, js = 8 * h + g;
            c.ws[g][row] = d * (float)(int8_t)(comp(scv, js >> 2) >> (8 * (js & 3)));
            const uint4 lv = r.w[qq & 1];
            const int lsh = qq < 2 ? 0 : 4, hsh = 2 * qq;
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t v6 = ((comp(lv, i) >> lsh) & 0x0F0F0F0Fu) | (((comp(hv, i) >> hsh) & 0x03030303u) << 4);
                o[i] = (uint32_t)bytes_sub(v6, 0x20202020u);
            }
            put_a(c, row, 16 * g, make_uint4(o[0], o[1], o[2], o[3]));
        }
    } else if constexpr (Q == JK_TQ2_0) {
        // plane 2h + j: its dword k holds elements 64j + 16k .. 64j + 16k + 15, the 2-bit
        // fields of each byte in order
        const float d = f16_finite(r.wd[0]);
        c.ws[2 * j][row] = d;
        c.ws[2 * j + 1][row] = d;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t wv = comp(r.w[0], k);
            put_a(c, row, 64 * j + 16 * k,
                  make_uint4(crumbs_minus1(wv & 0x03030303u), crumbs_minus1((wv >> 2) & 0x03030303u),
                             crumbs_minus1((wv >> 4) & 0x03030303u), crumbs_minus1((wv >> 6) & 0x03030303u)));
        }
    } else {  // JK_I2_S: 32-group g is 2-bit field g (shift 6 - 2g) of planes 0 (first 16) and 1
        c.ws[2 * j][row] = w.tensor_scale;
        c.ws[2 * j + 1][row] = w.tensor_scale;
#pragma unroll
        for (int g = 0; g < 4; ++g) put_a(c, row, 32 * g + 16 * j, crumb4(r.w[0], 6 - 2 * g));
    }
}

// GB: 32-element steps per scale block. 1 for the repacked GEMM (per-32 activation scales,
// one epilogue per step); for BitLinear (one scale per token and per weight block: 256
// elements for TQ2_0, 128 for I2_S, 32 for Q8_0) the block's MFMAs accumulate in i32 and the
// epilogue runs once per block.
// TOL: tolerance mode -- each group's exact integer partial enters the accumulator through one
// fused multiply-add, acc = fma(f32(c), xs * ws, acc), and formats with mins add -(xsum * wm) with
// the K = 1 outer-product MFMA accumulating into the accumulators (one rounding each), instead of
// the reference's separately rounded products and sums. The 1e-5-of-the-row-L2-norm tolerance
// the port is held to for f32 products allows it; the bit-exact kernel is TOL = false.
template <int Q, int GB, int TN, int TM, bool TOL = false>
__global__ __launch_bounds__(2 * TN) __attribute__((amdgpu_waves_per_eu(Tile<TN, TM>::WPE))) void
gemm_repacked_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    using F = GemmFmt<Q>;
    using T = Tile<TN, TM>;
    constexpr int NT = T::NT, RW = T::RW;
    static_assert(GB == 1 || F::GK == 32, "block accumulation needs 32-element steps");
    __shared__ __align__(16) GemmChunk<Q, TN, TM> cs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % T::WR, wmi = wave / T::WR;  // wave tile: rows RW * wn .., tokens 32 * wmi ..
    // Workgroup i runs on XCD i % 8. Tile order: the token tiles of one weight row tile go
    // to consecutive workgroups of one XCD, so they run together and share the row tile's
    // weights in that XCD's L2; row tiles are dealt round-robin over the XCDs.
    const int ntn = (r1 - r0 + TN - 1) / TN, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;  // padding workgroups of the last round-robin group
    const int n0 = r0 + tn * TN, m0 = tm * TM;
    const int M = (int)a.m;
    const int steps = w.cols / 32;
    const int nchunks = (steps + kSteps - 1) / kSteps;
    const int hl = lane >> 5, jl = lane & 31;
    const int tok = 32 * wmi + jl;

    float acc[NT][16];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[nt][v] = 0.0f;
    v16f tacc[NT];  // TOL: the accumulators of each 32-row block, in the MFMA result layout
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) tacc[nt] = v16f{0};
    static_assert(!TOL || (F::GK == 32 && GB == 1), "tolerance mode: 32-element groups, one per step");

    v16i cacc[NT];  // i32 partials of the current scale block (GB > 1)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) cacc[nt] = v16i{0};
    // the scale-product MFMA covers two 32-row blocks; lane l supplies row RW wn + srow
    const int srow = RW * wn + (NT == 2 ? lane : jl);
    // chunk kc from LDS
    auto step = [&](int kc, int st) {
        const float xs = cs.xs[st][tok];
        const float xsum32 = F::MINS && F::GK == 32 ? cs.xm[st][tok] : 0.0f;
        if constexpr (TOL) {
            // One 32-row block at a time: its integer partial, its scale products as a K = 2 f32
            // outer product (lanes 32..63 supply the zero second column, so each is the single
            // rounded product xs * ws), then one fused multiply-add per output; formats with mins
            // add -(xsum * wm) through the same outer product accumulating into the block.
            const v4i bq = *reinterpret_cast<const v4i *>(cs.b + tok * kRowB + 32 * st + 16 * hl);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int r = RW * wn + 32 * nt + jl;
                const v4i aq = *reinterpret_cast<const v4i *>(cs.a + r * kRowB + 32 * st + 16 * hl);
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
                const v16f p =
                    __builtin_amdgcn_mfma_f32_32x32x2f32(hl ? 0.0f : cs.ws[st][r], hl ? 0.0f : xs, v16f{0}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) tacc[nt][v] = __builtin_fmaf((float)c[v], p[v], tacc[nt][v]);
                if constexpr (F::MINS)
                    tacc[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(hl ? 0.0f : -cs.wm[st][r], hl ? 0.0f : xsum32,
                                                                    tacc[nt], 0, 0, 0);
            }
            return;
        }
#pragma unroll
        for (int gg = 0; gg < 32 / F::GK; ++gg) {
            v16i c[NT];
            if constexpr (F::GK == 32) {
                const v4i bq = *reinterpret_cast<const v4i *>(cs.b + tok * kRowB + 32 * st + 16 * hl);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const v4i aq =
                        *reinterpret_cast<const v4i *>(cs.a + (RW * wn + 32 * nt + jl) * kRowB + 32 * st + 16 * hl);
                    if constexpr (GB == 1) c[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
                    else c[nt] = cacc[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, cacc[nt], 0, 0, 0);
                }
                if constexpr (GB > 1) {
                    if ((kSteps * kc + st) % GB != GB - 1) continue;  // block not complete: no epilogue yet
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) cacc[nt] = v16i{0};
                }
            } else {
                const long bq = *reinterpret_cast<const long *>(cs.b + tok * kRowB + 32 * st + 16 * gg + 8 * hl);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const long aq = *reinterpret_cast<const long *>(cs.a + (RW * wn + 32 * nt + jl) * kRowB +
                                                                    32 * st + 16 * gg + 8 * hl);
                    c[nt] = __builtin_amdgcn_mfma_i32_32x32x16_i8(aq, bq, v16i{0}, 0, 0, 0);
                }
            }
            // Scale products xs * ws (and xsum * wm) of all 64 x 32 outputs as two 32 x 32
            // f32 outer products (K = 1, zero accumulator): each is the single rounded f32
            // product, as a VALU multiply gives, except that -0 comes out +0 -- which the
            // accumulation cannot observe, as an accumulator that starts at +0.0 never
            // becomes -0. Lane l supplies the scale of row srow (block l / 32 = nt; with
            // one block per wave both halves repeat it) and of token tok. Both results share
            // c's layout: lane holds token column jl, weight rows 8 * (v / 4) + 4 * hl + v % 4
            // of block nt in element 16 nt + v.
            const int g = (32 / F::GK) * st + gg;
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.ws[g][srow], xs, v32f{0}, 0, 0, 0);
            v32f pm;
            // mins: per 32-group with the 32-block activation sum, or per 16-group (Q2_K) with
            // the 16-element sum (accumulate_scaled_tile_scalar, repack.rs:3061-3077)
            if constexpr (F::MINS && F::GK == 32)
                pm = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.wm[st][srow], xsum32, v32f{0}, 0, 0, 0);
            if constexpr (F::MINS && F::GK == 16)
                pm = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.wm[g][srow], cs.xm[g][tok], v32f{0}, 0, 0, 0);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float t = (float)c[nt][v] * p[16 * nt + v];
                    if constexpr (F::MINS) acc[nt][v] += t - pm[16 * nt + v];
                    else acc[nt][v] += t;
                }
        }
    };
    auto compute = [&](int kc) {
        const int nst = min(kSteps, steps - kSteps * kc);
        for (int st = 0; st < nst; ++st) step(kc, st);
    };

    Stage<TN, TM> rg;
    chunk_load<Q>(rg, w, a, n0, r1, m0, M, 0);
    chunk_store<Q>(w, rg, cs, 0);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) chunk_load<Q>(rg, w, a, n0, r1, m0, M, kc + 1);
        compute(kc);
        if (more) {
            __syncthreads();
            chunk_store<Q>(w, rg, cs, kc + 1);
            __syncthreads();
        }
    }

    const int m = m0 + tok;
    if (m < M) {
        const size_t ld = (size_t)(r1 - r0);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int n = n0 + RW * wn + 32 * nt + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (n < r1) y[(size_t)m * ld + (size_t)(n - r0)] = TOL ? tacc[nt][v] : acc[nt][v];
            }
    }
}

// Tolerance-mode prefill tiles for the 32-element-group formats: a workgroup computes 128
// weight rows x 128 tokens with four waves, each 64 rows x 64 tokens (2 x 2 blocks of 32 x 32),
// at two waves per SIMD. Per scale group a wave issues four integer MFMAs, one two-block f32
// outer product of the scale products per token block (each the single rounded xs * ws), and
// one fused multiply-add per output, acc = fma(f32(c), xs * ws, acc); formats with mins add
// -(xsum * wm) through an outer product accumulating into the accumulators. Against the
// 128 x 64 tiles at three waves per SIMD the tile count halves (a 512-token launch fits the
// GPU's 512 resident workgroups in one round instead of 1.17) and each staged weight byte
// feeds twice the MFMAs.
template <int Q>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gemm_tol_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    using F = GemmFmt<Q>;
    constexpr int TN = 128, TM = 128;
    static_assert(F::GK == 32, "32-element scale groups");
    __shared__ __align__(16) GemmChunk<Q, TN, TM> cs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave & 1, wmi = wave >> 1;  // wave tile: rows 64 wn .., tokens 64 wmi ..
    // tile order as gemm_repacked_kernel: a row tile's token tiles on one XCD
    const int ntn = (r1 - r0 + TN - 1) / TN, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;
    const int n0 = r0 + tn * TN, m0 = tm * TM;
    const int M = (int)a.m;
    const int steps = w.cols / 32;
    const int nchunks = (steps + kSteps - 1) / kSteps;
    const int hl = lane >> 5, jl = lane & 31;
    const int arow = 64 * wn + jl;  // A operand row of block 0 (block 1: + 32)

    v32f tacc[2];  // [token block]: both 32-row blocks, element 16 nt + v
    tacc[0] = tacc[1] = v32f{0};
    // A step's MFMA operands, read from LDS one step ahead of their use (the scales are read
    // where they are used)
    struct Ops {
        v4i aq[2], bq[2];
    };
    auto load_ops = [&](int st) {
        Ops o;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            o.aq[nt] = *reinterpret_cast<const v4i *>(cs.a + (arow + 32 * nt) * kRowB + 32 * st + 16 * hl);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
            o.bq[tb] = *reinterpret_cast<const v4i *>(cs.b + (64 * wmi + 32 * tb + jl) * kRowB + 32 * st + 16 * hl);
        return o;
    };
    auto compute = [&](const Ops &o, int st) {
        const float ws = cs.ws[st][64 * wn + lane];  // lane l: row of block l / 32
        [[maybe_unused]] const float wm = F::MINS ? -cs.wm[st][64 * wn + lane] : 0.0f;
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int tok = 64 * wmi + 32 * tb + jl;
            v16i c[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) c[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.aq[nt], o.bq[tb], v16i{0}, 0, 0, 0);
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(ws, cs.xs[st][tok], v32f{0}, 0, 0, 0);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    tacc[tb][16 * nt + v] = __builtin_fmaf((float)c[nt][v], p[16 * nt + v], tacc[tb][16 * nt + v]);
            if constexpr (F::MINS) tacc[tb] = __builtin_amdgcn_mfma_f32_32x32x1f32(wm, cs.xm[st][tok], tacc[tb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // the four steps of a whole chunk, unrolled, each step's operands read during the previous one
    // (a loop, not unrolled: unrolled, the register allocation of the four steps spills)
    auto chunk4 = [&]() {
        Ops cur = load_ops(0);
#pragma unroll 1
        for (int st = 0; st < kSteps; ++st) {
            const Ops nxt = load_ops(st + 1 < kSteps ? st + 1 : st);
            compute(cur, st);
            cur = nxt;
        }
    };

    Stage<TN, TM> rg;
    chunk_load<Q>(rg, w, a, n0, r1, m0, M, 0);
    chunk_store<Q>(w, rg, cs, 0);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) chunk_load<Q>(rg, w, a, n0, r1, m0, M, kc + 1);
        chunk4();  // (K is a multiple of 128 on this kernel)
        if (more) {
            __syncthreads();
            chunk_store<Q>(w, rg, cs, kc + 1);
            __syncthreads();
        }
    }

    const size_t ld = (size_t)(r1 - r0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int m = m0 + 64 * wmi + 32 * tb + jl;
        if (m >= M) continue;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int n = n0 + 64 * wn + 32 * nt + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (n < r1) y[(size_t)m * ld + (size_t)(n - r0)] = tacc[tb][16 * nt + v];
            }
    }
}

// The integer scales of a staged 16-element-group chunk kc (Q6_K: int8 scale 8h + g; Q3_K: 6-bit
// scale 8h + g minus 32) and the block's d, as chunk_store unpacks them: staging thread t has row
// t / 2 and half j = t % 2 of the chunk's 8 groups.
template <int Q, int TN, int TM>
__device__ __forceinline__ void tol16_scales(const Stage<TN, TM> &r, int kc, int t, int (*sc)[TN], float *d) {
    const int row = t >> 1, j = t & 1, h = kc & 1;
    if constexpr (Q == JK_Q6_K) {
        const uint4 scv = r.w[3];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int g = j + 2 * qq, js = 8 * h + g;
            sc[g][row] = (int)(int8_t)(comp(scv, js >> 2) >> (8 * (js & 3)));
        }
        if (j == 0) d[row] = f16_finite(r.wd[0]);
    } else {  // Q3_K (repack.rs:1896-1911)
        const uint4 tail = r.w[4];
#pragma unroll
        for (int jo = 0; jo < 2; ++jo)
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const int g = 2 * (2 * j + jo) + part, is = 8 * h + g;
                const uint32_t lb = (comp(tail, (is & 7) >> 2) >> (8 * (is & 3))) & 255u;
                const uint32_t lo = is < 8 ? (lb & 15u) : (lb >> 4);
                const uint32_t hi = (((tail.z >> (8 * (is & 3))) & 255u) >> (2 * (is >> 2))) & 3u;
                sc[g][row] = (int)(lo | (hi << 4)) - 32;
            }
        if (j == 0) d[row] = f16_finite(tail.w & 0xFFFFu);
    }
}

// Tolerance-mode prefill for Q6_K and Q3_K (16-element scale groups, no mins): the tiles, staging
// and loop of gemm_tol_kernel. A 32-element step holds two groups of one weight block with integer
// scales sc0, sc1 and the block's d (dequantize_q6_k_block, quant.rs:594-648: y = d * sc * (q - 32);
// dequantize_q3_k_block, quant.rs:320-331: y = d * (scale - 32) * q3).
// Each group's exact i32 dot comes from a K = 16 MFMA; with tokens as the MFMA's A operand and
// weights as its B operand a lane holds one weight row, so the two groups combine in integers,
// sc0 * c0 + sc1 * c1 (24-bit multiplies: |c| <= 16 * 32 * 127 and |sc| <= 128, so the sum stays
// below 2^24 and converts to f32 exactly), and enter the accumulator through one fused
// multiply-add by xs * d -- four VALU instructions per output and step where the reference's
// recipe takes six. Outputs are within the tolerance of the bit-exact recipe as for the other
// tolerance kernels: per step the scale product xs * d and the fused multiply-add round once
// each, where the reference rounds two products and a sum per group (d * sc is exact either way).
template <int Q>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gemm_tol16_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    static_assert(Q == JK_Q6_K || Q == JK_Q3_K, "Q6_K, Q3_K");
    constexpr int TN = 128, TM = 128;
    __shared__ __align__(16) GemmChunk<Q, TN, TM> cs;
    __shared__ int s_sc[8][TN];  // the chunk's 8 group scales per row
    __shared__ float s_d[TN];    // the rows' block scale d
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave & 1, wmi = wave >> 1;  // wave tile: rows 64 wn .., tokens 64 wmi ..
    const int ntn = (r1 - r0 + TN - 1) / TN, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;
    const int n0 = r0 + tn * TN, m0 = tm * TM;
    const int M = (int)a.m;
    const int nchunks = w.cols / kKC;  // (K is a multiple of 128 on this kernel)
    const int hl = lane >> 5, jl = lane & 31;

    v32f tacc[2];  // [token block]: rows of block nt at element 16 nt + v (lane: row jl of the block)
    tacc[0] = tacc[1] = v32f{0};
    // the scales of the staged chunk kc: thread t has row t / 2, half j = t % 2 of the chunk's
    // groups (g = j + 2 qq), as chunk_store unpacks them
    auto store_scales = [&](const Stage<TN, TM> &r, int kc) { tol16_scales<Q>(r, kc, (int)threadIdx.x, s_sc, s_d); };
    auto step = [&](int st) {
        // lane l (half hl) supplies token jl's scale (A) and the d of row 64 wn + 32 hl + jl (B):
        // p[16 nt + v] = xs(token 8 (v / 4) + 4 hl + v % 4 of the token block) * d(row jl of block nt)
        const float dr = s_d[64 * wn + 32 * hl + jl];
        int sc[2][2];  // [nt][group]
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) sc[nt][gg] = s_sc[2 * st + gg][64 * wn + 32 * nt + jl];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int tok = 64 * wmi + 32 * tb + jl;
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.xs[st][tok], dr, v32f{0}, 0, 0, 0);
            long bq[2];
#pragma unroll
            for (int gg = 0; gg < 2; ++gg)
                bq[gg] = *reinterpret_cast<const long *>(cs.b + tok * kRowB + 32 * st + 16 * gg + 8 * hl);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int arow = 64 * wn + 32 * nt + jl;
                v16i c[2];
#pragma unroll
                for (int gg = 0; gg < 2; ++gg) {
                    const long aq = *reinterpret_cast<const long *>(cs.a + arow * kRowB + 32 * st + 16 * gg + 8 * hl);
                    c[gg] = __builtin_amdgcn_mfma_i32_32x32x16_i8(bq[gg], aq, v16i{0}, 0, 0, 0);
                }
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int comb = __mul24(c[0][v], sc[nt][0]) + __mul24(c[1][v], sc[nt][1]);
                    tacc[tb][16 * nt + v] = __builtin_fmaf((float)comb, p[16 * nt + v], tacc[tb][16 * nt + v]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    Stage<TN, TM> rg;
    chunk_load<Q>(rg, w, a, n0, r1, m0, M, 0);
    chunk_store<Q>(w, rg, cs, 0);
    store_scales(rg, 0);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) chunk_load<Q>(rg, w, a, n0, r1, m0, M, kc + 1);
#pragma unroll 1
        for (int st = 0; st < kSteps; ++st) step(st);
        if (more) {
            __syncthreads();
            chunk_store<Q>(w, rg, cs, kc + 1);
            store_scales(rg, kc + 1);
            __syncthreads();
        }
    }

    // element v of block nt: token 8 (v / 4) + 4 hl + v % 4 of token block tb, row jl of block nt
    const size_t ld = (size_t)(r1 - r0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int n = n0 + 64 * wn + 32 * nt + jl;
            if (n >= r1) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + 64 * wmi + 32 * tb + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (m < M) y[(size_t)m * ld + (size_t)(n - r0)] = tacc[tb][16 * nt + v];
            }
        }
}

// Q8_0 tolerance-mode prefill, the same tiles and arithmetic as gemm_tol_kernel with its loads
// made asynchronous: Q8_0 quants need no unpacking, so every tile goes from global memory
// straight into LDS (global_load_lds: lane l of a load writes bytes 16 l.. of a 1 KB LDS
// span), two chunk stages deep, with no staging registers. While chunk kc is evaluated from
// one stage, chunk kc + 1 streams into the other. The stages are separate LDS objects, so
// the compiler's dependency tracking keeps the reads of one stage free of the loads into the
// other; each wave waits for its own loads of a stage (vmcnt) before a barrier publishes it.
// A stage (35 KB): weights [row][8 x 16 B] and activation quants [token][8 x 16 B] with the
// 16-byte piece p of row r at slot p ^ ((r >> 1) & 7) (16 consecutive rows or tokens of an MFMA
// operand read, which the LDS serves together, then fall on 16 distinct 16-byte bank groups: with
// slot p ^ (r & 7) rows r and r + 8 collided, and the counters put bank conflicts in 58% of the
// LDS-active cycles), the f16 scales of the chunk's four blocks per row, and the f32 activation
// scales per token.
template <int TN> struct alignas(16) Q8Stage {
    uint8_t a[TN * 128];
    uint8_t x[128 * 128];
    uint16_t ws[TN * 4];
    float xs[128 * 4];
};
// loads per wave and stage (NW = TN / 32 waves): 4 weight, 16 / NW activation, 1 scale, 8 / NW act scale
template <int TN> constexpr int kQ8DmaPerWave = 4 + 16 / (TN / 32) + 1 + 8 / (TN / 32);

// EXACT: the reference's epilogue instead, bit for bit -- the integer MFMA from zero, the scale
// product from the outer-product MFMA, then acc = acc + f32(dot) * (xs * ws), each rounded, in K order.
template <int TN, bool EXACT = false>
__device__ __forceinline__ void gemm_q8_0_tol_dma(const WeightDev &w, const jk_act_q8 &a, float *__restrict__ y, int r0,
                                                  int r1) {
    constexpr int TM = 128, NW = TN / 32, WR = TN / 64;  // waves; waves along the rows (64 rows each)
    constexpr int XPW = 16 / NW, SPW = 8 / NW;          // activation / activation-scale loads per wave
    __shared__ Q8Stage<TN> sA;
    __shared__ Q8Stage<TN> sB;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn = wave % WR, wmi = wave / WR;  // wave tile: rows 64 wn .., tokens 64 wmi ..
    const int ntn = (r1 - r0 + TN - 1) / TN, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;
    const int n0 = r0 + tn * TN, m0 = tm * TM;
    const int M = (int)a.m, nb = w.nb;
    const int nchunks = w.cols / 128;  // (K is a multiple of 128 on this kernel)
    const int hl = lane >> 5, jl = lane & 31;
    const size_t pstride = (size_t)w.rows * (size_t)nb * 16;

    // this lane's share of a stage's loads (addresses of chunk 0; chunk kc adds a fixed offset)
    const int rr = lane >> 3, slot = lane & 7;
    const uint8_t *asrc[4];
    const uint8_t *xsrc[XPW];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = 8 * (4 * wave + i) + rr, p = slot ^ ((n >> 1) & 7);
        const int gn = min(n0 + n, r1 - 1);
        asrc[i] = w.planes + (size_t)(p & 1) * pstride + ((size_t)gn * (size_t)nb + (size_t)(p >> 1)) * 16;
    }
#pragma unroll
    for (int i = 0; i < XPW; ++i) {
        const int t = 8 * (XPW * wave + i) + rr, q = slot ^ ((t >> 1) & 7);
        const int gt = min(m0 + t, M - 1);
        xsrc[i] = reinterpret_cast<const uint8_t *>(a.qs) + (size_t)gt * a.k_padded + (size_t)(16 * q);
    }
    const int wsd = 64 * wave + lane;  // dword of the scale span: row wsd / 2, blocks 2 (wsd % 2) ..
    const uint8_t *wssrc = reinterpret_cast<const uint8_t *>(w.dplane) +
                           ((size_t)min(n0 + (wsd >> 1), r1 - 1) * (size_t)nb + (size_t)(2 * (wsd & 1))) * 2;
    const uint8_t *xssrc[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        const int d = 64 * (SPW * wave + i) + lane;  // token d / 4, block d % 4
        xssrc[i] = reinterpret_cast<const uint8_t *>(a.scales) +
                   ((size_t)min(m0 + (d >> 2), M - 1) * a.k_blocks32 + (size_t)(d & 3)) * 4;
    }
    auto issue = [&](Q8Stage<TN> &S, int kc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(asrc[i] + (size_t)kc * 64, (lds_u8_t *)S.a + 1024 * (4 * wave + i));
#pragma unroll
        for (int i = 0; i < XPW; ++i) lds_dma16(xsrc[i] + (size_t)kc * 128, (lds_u8_t *)S.x + 1024 * (XPW * wave + i));
        lds_dma4(wssrc + (size_t)kc * 8, (lds_u8_t *)S.ws + 256 * wave);
#pragma unroll
        for (int i = 0; i < SPW; ++i) lds_dma4(xssrc[i] + (size_t)kc * 16, (lds_u8_t *)S.xs + 256 * (SPW * wave + i));
    };

    v32f tacc[2];
    tacc[0] = tacc[1] = v32f{0};
    const v16i bias = magic_acc();
    const int arow = 64 * wn + jl;
    auto chunk_tol = [&](const Q8Stage<TN> &S) {
#pragma unroll 1
        for (int st = 0; st < kSteps; ++st) {
            const int pc = 2 * st + hl;  // 16-byte piece: block st, half hl
            v4i aq[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int r = arow + 32 * nt;
                aq[nt] = *reinterpret_cast<const v4i *>(S.a + r * 128 + ((pc ^ ((r >> 1) & 7)) << 4));
            }
            const float ws = f16_finite(S.ws[(64 * wn + lane) * 4 + st]);  // lane l: row of block l / 32
            const float wsb = ws * -kMagicF;  // exact: 1.5 * 2^23 times an 11-bit significand
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const int t = 64 * wmi + 32 * tb + jl;
                const v4i bq = *reinterpret_cast<const v4i *>(S.x + t * 128 + ((pc ^ ((t >> 1) & 7)) << 4));
                const float xs = S.xs[t * 4 + st];
                v16i c[2];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) c[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq[nt], bq, bias, 0, 0, 0);
                const v32f pr = __builtin_amdgcn_mfma_f32_32x32x1f32(ws, xs, v32f{0}, 0, 0, 0);
                // the bias's share of the group, B * ws * xs, taken off the accumulators on the matrix
                // core, so each output costs one fused multiply-add of the biased bits
                tacc[tb] = __builtin_amdgcn_mfma_f32_32x32x1f32(wsb, xs, tacc[tb], 0, 0, 0);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        tacc[tb][16 * nt + v] =
                            __builtin_fmaf(__int_as_float(c[nt][v]), pr[16 * nt + v], tacc[tb][16 * nt + v]);
            }
        }
    };

    // Bit-exact mode: the chunk's 8 (step, token block) pairs software-pipelined, the MFMAs of pair
    // t + 1 issued before the epilogue of pair t on a ring of two register sets, a scheduling barrier
    // after each pair so the compiler keeps that shape (unconstrained, it hoists further and spills);
    // each output still takes its groups in K order. 146.1 against 150.7 us at 512 tokens.
    auto chunk_exact = [&](const Q8Stage<TN> &S) {
        v16i c[2][2];
        v32f pr[2];
        auto mfmas = [&](int t, int slot) {
            const int st = t >> 1, tb = t & 1, pc = 2 * st + hl;
            v4i aq[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int r = arow + 32 * nt;
                aq[nt] = *reinterpret_cast<const v4i *>(S.a + r * 128 + ((pc ^ ((r >> 1) & 7)) << 4));
            }
            const float ws = f16_finite(S.ws[(64 * wn + lane) * 4 + st]);
            const int tk = 64 * wmi + 32 * tb + jl;
            const v4i bq = *reinterpret_cast<const v4i *>(S.x + tk * 128 + ((pc ^ ((tk >> 1) & 7)) << 4));
            const float xs = S.xs[tk * 4 + st];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) c[slot][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq[nt], bq, v16i{0}, 0, 0, 0);
            pr[slot] = __builtin_amdgcn_mfma_f32_32x32x1f32(ws, xs, v32f{0}, 0, 0, 0);
        };
        auto epilogue = [&](int t, int slot) {
            const int tb = t & 1;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    tacc[tb][16 * nt + v] = tacc[tb][16 * nt + v] + (float)c[slot][nt][v] * pr[slot][16 * nt + v];
        };
        mfmas(0, 0);
#pragma unroll
        for (int t = 0; t < 2 * kSteps; ++t) {
            if (t + 1 < 2 * kSteps) mfmas(t + 1, (t + 1) & 1);
            epilogue(t, t & 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // One barrier per chunk: the barrier that publishes chunk kc (every wave has waited for its own
    // loads into the stage) also shows every wave done with chunk kc - 1, whose stage is then
    // refilled with chunk kc + 1 while chunk kc is evaluated.
    issue(sA, 0);
    if (nchunks > 1) issue(sB, 1);
    for (int kc = 0; kc < nchunks; kc += 2) {
        if (kc == 0 && nchunks > 1) JK_WAIT_VMCNT(kQ8DmaPerWave<TN>);  // chunk 1 stays in flight
        else JK_WAIT_VMCNT(0);
        stage_barrier();
        if (kc >= 2 && kc + 1 < nchunks) issue(sB, kc + 1);
        if constexpr (EXACT) chunk_exact(sA);
        else chunk_tol(sA);
        if (kc + 1 >= nchunks) break;
        JK_WAIT_VMCNT(0);
        stage_barrier();
        if (kc + 2 < nchunks) issue(sA, kc + 2);
        if constexpr (EXACT) chunk_exact(sB);
        else chunk_tol(sB);
    }

    const size_t ld = (size_t)(r1 - r0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int m = m0 + 64 * wmi + 32 * tb + jl;
        if (m >= M) continue;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int n = n0 + 64 * wn + 32 * nt + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (n < r1) y[(size_t)m * ld + (size_t)(n - r0)] = tacc[tb][16 * nt + v];
            }
    }
}

// (a plain kernel around the body: the host stub of a kernel template with this body is not
// emitted)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gemm_q8_0_tol_dma_128(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    gemm_q8_0_tol_dma<128>(w, a, y, r0, r1);
}

// The bit-exact Q8_0 prefill on the same staging (launched where it measured faster than the
// register-staged 128 x 64 tiles; see launch_gemm)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
gemm_q8_0_exact_dma_128(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    gemm_q8_0_tol_dma<128, true>(w, a, y, r0, r1);
}

static long cu_count() {
    static long n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        n = hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v
                : 256;
    }
    return n;
}

// Small launches: one wave computes 32 weight rows x 16 tokens as two 16 x 16 tiles
// (v_mfma_i32_16x16x32_i8 per 32-element group; lane l supplies row / token l % 16 and K
// bytes 8 (l / 16) .. + 7, and holds token l % 16, rows 4 (l / 16) + r of each tile). The
// scale products are VALU multiplies (8 a group), the reference's single rounded products.
// Each wave's serial chain per group is about half that of a 32 x 32 tile, and the launch
// has twice the waves. (Q6_K's 16-element groups stay on the 32 x 32 tiles: measured slower here.)
template <int Q, int GB>
__global__ __launch_bounds__(64) void gemm16_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0, int r1) {
    using F = GemmFmt<Q>;
    constexpr int TN = 32, TM = 16;
    static_assert(F::GK == 32, "32-element scale groups");
    __shared__ __align__(16) GemmChunk<Q, TN, TM> cs;
    const int lane = threadIdx.x;
    const int ntn = (r1 - r0 + TN - 1) / TN, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;  // as gemm_repacked_kernel
    if (tn >= ntn) return;
    const int n0 = r0 + tn * TN, m0 = tm * TM;
    const int M = (int)a.m;
    const int steps = w.cols / 32;
    const int nchunks = (steps + kSteps - 1) / kSteps;
    const int jl = lane & 15, kq = lane >> 4;

    float acc[2][4];
    v4i cacc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        cacc[nt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[nt][r] = 0.0f;
    }
    auto step = [&](int kc, int st) {
        const int off = 32 * st + 8 * kq;
        const long bq = *reinterpret_cast<const long *>(cs.b + jl * kRowB + off);
        v4i c[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const long aq = *reinterpret_cast<const long *>(cs.a + (16 * nt + jl) * kRowB + off);
            if constexpr (GB == 1) c[nt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, bq, v4i{0, 0, 0, 0}, 0, 0, 0);
            else c[nt] = cacc[nt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, bq, cacc[nt], 0, 0, 0);
        }
        if constexpr (GB > 1) {
            if ((kSteps * kc + st) % GB != GB - 1) return;  // block not complete: no epilogue yet
            cacc[0] = cacc[1] = v4i{0, 0, 0, 0};
        }
        const float xs = cs.xs[st][jl];
        const float xsum = F::MINS ? cs.xm[st][jl] : 0.0f;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const float4 ws4 = *reinterpret_cast<const float4 *>(&cs.ws[st][16 * nt + 4 * kq]);
            float4 wm4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if constexpr (F::MINS) wm4 = *reinterpret_cast<const float4 *>(&cs.wm[st][16 * nt + 4 * kq]);
            const float wsr[4] = {ws4.x, ws4.y, ws4.z, ws4.w};
            [[maybe_unused]] const float wmr[4] = {wm4.x, wm4.y, wm4.z, wm4.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float t = (float)c[nt][r] * (xs * wsr[r]);
                if constexpr (F::MINS) acc[nt][r] += t - xsum * wmr[r];
                else acc[nt][r] += t;
            }
        }
    };

    Stage<TN, TM> rg;
    chunk_load<Q>(rg, w, a, n0, r1, m0, M, 0);
    chunk_store<Q>(w, rg, cs, 0);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) chunk_load<Q>(rg, w, a, n0, r1, m0, M, kc + 1);
        const int nst = min(kSteps, steps - kSteps * kc);
        for (int st = 0; st < nst; ++st) step(kc, st);
        if (more) {
            __syncthreads();
            chunk_store<Q>(w, rg, cs, kc + 1);
            __syncthreads();
        }
    }

    const int m = m0 + jl;
    if (m < M) {
        const size_t ld = (size_t)(r1 - r0);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = n0 + 16 * nt + 4 * kq + r;
                if (n < r1) y[(size_t)m * ld + (size_t)(n - r0)] = acc[nt][r];
            }
    }
}

// One or two tokens (the reference's m <= 2 GEMV route, repack.rs:2892): the same per-group
// arithmetic without MFMA, shaped for streaming. A workgroup owns 32 weight rows and all of K;
// its NW waves take the 128-element chunks round-robin (wave v: chunks v, v + NW, ...), each
// staging its chunk through the GEMM's loads (kGemvDepth chunks in flight) and unpacking into a
// chunk of LDS of its own.
// Each lane evaluates the terms of half the chunk's scale groups for one row and every token,
//     term = f32(sum xq * wq) * (xs * ws)  [- xsum * wm],
// the reference's per-group addend (accumulate_scaled_tile_scalar, repack.rs:3045-3093), into
// an LDS table; after a barrier, wave 0 (lane: row l % 32 of token l / 32) adds the round's
// terms to its accumulator in K order. Each output is therefore the same sum, in the same
// order, as the GEMM's.
constexpr int kGemvNW = 8;     // waves per workgroup (chunk LDS plus term tables: 99-142 KB of the 160 KB)
constexpr int kGemvDepth = 2;  // chunks in flight per wave (4 measured slower: register pressure)

template <int Q>
__global__ __launch_bounds__(64 * kGemvNW) void gemv_repacked_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y,
                                                                     int r0, int r1) {
    using F = GemmFmt<Q>;
    using Ch = GemmChunk<Q, 32, 16>;
    constexpr int NW = kGemvNW, NG = F::NG, GPL = NG / 2;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    Ch &cs = reinterpret_cast<Ch *>(smem)[wave];
    float *terms = reinterpret_cast<float *>(smem + NW * sizeof(Ch));  // [2 rounds][2 tokens][NW][NG][32]
    const int n0 = r0 + 32 * (int)blockIdx.x;
    const int M = (int)a.m;
    const int steps = w.cols / 32, nchunks = (steps + kSteps - 1) / kSteps, rounds = (nchunks + NW - 1) / NW;
    const int row = lane & 31, hs = lane >> 5;
    float acc = 0.0f;  // wave 0: row n0 + row of token hs

    // kGemvDepth chunks in flight per wave: round rd's chunk is staged in set rd % kGemvDepth
    // (the loop is unrolled so that each staging set is a fixed set of registers)
    Stage<32, 16> rg[kGemvDepth];
#pragma unroll
    for (int d = 0; d < kGemvDepth; ++d)
        if (wave + NW * d < nchunks) chunk_load<Q>(rg[d], w, a, n0, r1, 0, M, wave + NW * d);
    auto round = [&](int rd, Stage<32, 16> &stg) {
        const int kc = NW * rd + wave;  // wave-uniform
        float *tb = terms + (rd & 1) * (2 * NW * NG * 32);
        if (kc < nchunks) {
            chunk_store<Q>(w, stg, cs, kc);
            wave_lds_sync();
            if (kc + kGemvDepth * NW < nchunks) chunk_load<Q>(stg, w, a, n0, r1, 0, M, kc + kGemvDepth * NW);
            const int ng = min(kSteps, steps - kSteps * kc) * 32 / F::GK;  // groups of this chunk
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int q = 0; q < GPL; ++q) {
                    const int g = GPL * hs + q, st = g * F::GK / 32;
                    if (g < ng) {
                        const uint8_t *pa = cs.a + row * kRowB + F::GK * g, *pb = cs.b + m * kRowB + F::GK * g;
                        int c = 0;
#pragma unroll
                        for (int i = 0; i < F::GK / 16; ++i) {
                            const uint4 va = *reinterpret_cast<const uint4 *>(pa + 16 * i);
                            const uint4 vb = *reinterpret_cast<const uint4 *>(pb + 16 * i);
                            c = dot4((int)va.x, (int)vb.x, c);
                            c = dot4((int)va.y, (int)vb.y, c);
                            c = dot4((int)va.z, (int)vb.z, c);
                            c = dot4((int)va.w, (int)vb.w, c);
                        }
                        float term = (float)c * (cs.xs[st][m] * cs.ws[g][row]);
                        if constexpr (F::MINS && F::GK == 32) term = term - cs.xm[st][m] * cs.wm[st][row];
                        if constexpr (F::MINS && F::GK == 16) term = term - cs.xm[g][m] * cs.wm[g][row];
                        tb[((m * NW + wave) * NG + g) * 32 + row] = term;
                    }
                }
            }
        }
        __syncthreads();
        if (wave == 0 && hs < M) {
            // every term of the round read first (independent LDS reads in flight together),
            // then added in K order; slots past the last chunk are read but never added
            float t[NW * NG];
#pragma unroll
            for (int i = 0; i < NW * NG; ++i) t[i] = tb[(hs * NW * NG + i) * 32 + row];
#pragma unroll
            for (int v = 0; v < NW; ++v) {
                const int kv = NW * rd + v;
                const int ng = kv < nchunks ? min(kSteps, steps - kSteps * kv) * 32 / F::GK : 0;
#pragma unroll
                for (int g = 0; g < NG; ++g)
                    if (g < ng) acc += t[v * NG + g];
            }
        }
    };
    for (int rd = 0; rd < rounds; rd += kGemvDepth) {
#pragma unroll
        for (int d = 0; d < kGemvDepth; ++d)
            if (rd + d < rounds) round(rd + d, rg[d]);
    }
    if (wave == 0 && hs < M && n0 + row < r1) y[(size_t)hs * (size_t)(r1 - r0) + (size_t)(n0 + row - r0)] = acc;
}

template <int Q>
static jk_status launch_gemv_repacked_q(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0,
                                        int r1) {
    constexpr size_t lds =
        kGemvNW * sizeof(GemmChunk<Q, 32, 16>) + 2 * 2 * kGemvNW * GemmFmt<Q>::NG * 32 * sizeof(float);
    static_assert(lds <= 160 * 1024, "GEMV LDS budget (160 KB per workgroup on gfx950)");
    if (t_plan.dry) {
        t_plan.kernel = "gemv_repacked_kernel";
        return JK_OK;
    }
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(gemv_repacked_kernel<Q>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return hip_fail(attr, "gemv_repacked_kernel LDS");
    hipLaunchKernelGGL(gemv_repacked_kernel<Q>, dim3((unsigned)((r1 - r0 + 31) / 32)), dim3(64 * kGemvNW), lds, s, w, a,
                       y, r0, r1);
    return check_launch("gemv_repacked_kernel");
}

// m <= 2 of the repacked GEMM entry points (both modes: the result is the bit-exact one).
static jk_status launch_gemv_repacked(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    if (gemv_repacked_fast_ok(w.quant, a.m, a.k_padded, a.k_blocks32))
        return launch_gemv_repacked_fast(s, w, a, y, r0, r1);
    switch (w.quant) {
    case JK_Q8_0: return launch_gemv_repacked_q<JK_Q8_0>(s, w, a, y, r0, r1);
    case JK_Q4_0: return launch_gemv_repacked_q<JK_Q4_0>(s, w, a, y, r0, r1);
    case JK_Q5_0: return launch_gemv_repacked_q<JK_Q5_0>(s, w, a, y, r0, r1);
    case JK_Q4_K: return launch_gemv_repacked_q<JK_Q4_K>(s, w, a, y, r0, r1);
    case JK_Q5_K: return launch_gemv_repacked_q<JK_Q5_K>(s, w, a, y, r0, r1);
    case JK_Q4_1: return launch_gemv_repacked_q<JK_Q4_1>(s, w, a, y, r0, r1);
    case JK_Q5_1: return launch_gemv_repacked_q<JK_Q5_1>(s, w, a, y, r0, r1);
    case JK_IQ4_NL: return launch_gemv_repacked_q<JK_IQ4_NL>(s, w, a, y, r0, r1);
    case JK_Q2_K: return launch_gemv_repacked_q<JK_Q2_K>(s, w, a, y, r0, r1);
    case JK_Q3_K: return launch_gemv_repacked_q<JK_Q3_K>(s, w, a, y, r0, r1);
    case JK_Q6_K: return launch_gemv_repacked_q<JK_Q6_K>(s, w, a, y, r0, r1);
    case JK_TQ2_0: return launch_gemv_repacked_q<JK_TQ2_0>(s, w, a, y, r0, r1);
    case JK_I2_S: return launch_gemv_repacked_q<JK_I2_S>(s, w, a, y, r0, r1);
    default: return fail(JK_CAPABILITY_MISMATCH, "gemm: unsupported quant %d", w.quant);
    }
}

// Tolerance-mode products of a few tokens (3 up to a few hundred) for the 32-element-group
// formats, where the tiled kernels have too few tiles to fill the GPU: K is split instead. A
// workgroup owns 32 weight rows x TM tokens (TM = 32 or 64) and all of K; its NW waves take the
// 128-element chunks round-robin (wave v: chunks v, v + NW, ...). Each wave stages its chunks
// through the GEMM's coalesced loads and unpacking into an LDS chunk of its own -- two chunks in
// flight per wave, no barrier with the other waves -- and accumulates a partial tile; the NW
// partial tiles are added in wave order through LDS at the end. Per 32-element step: one
// integer MFMA per 32-token block; the scale products from one two-block f32 outer product
// (TM = 64: the two token blocks; TM = 32: two steps, held in the two halves of the partial tile
// until the end); one fused multiply-add per output; formats with mins add -(xsum * wm) through
// a second outer product accumulating into the partial tile.
template <int Q, int TM, int NW> union SplitkSmem {
    GemmChunk<Q, 32, TM> cs[NW];  // while the chunks are evaluated: one per wave
    float red[NW][TM][33];        // then the partial tiles [wave][token][row], rows padded to 33
};

template <int Q, int TM>
__device__ __forceinline__ void sk_compute(const GemmChunk<Q, 32, TM> &cs, v32f &acc, int lane) {
    constexpr bool MINS = GemmFmt<Q>::MINS;
    const int hl = lane >> 5, jl = lane & 31;
    const uint8_t *pa = cs.a + jl * kRowB + 16 * hl;
    if constexpr (TM == 64) {
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const v4i aq = *reinterpret_cast<const v4i *>(pa + 32 * st);
            // lane l: row jl and token l (token block l / 32)
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.ws[st][jl], cs.xs[st][lane], v32f{0}, 0, 0, 0);
            // both token blocks' MFMAs ahead of their rescaling (one more v16i live: 236 VGPRs);
            // across steps the MFMAs stay in order (interleaving them spills)
            v16i c[2];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const v4i bq = *reinterpret_cast<const v4i *>(cs.b + (32 * tb + jl) * kRowB + 32 * st + 16 * hl);
                c[tb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[16 * tb + v] = __builtin_fmaf((float)c[tb][v], p[16 * tb + v], acc[16 * tb + v]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (MINS)
                acc = __builtin_amdgcn_mfma_f32_32x32x1f32(-cs.wm[st][jl], cs.xm[st][lane], acc, 0, 0, 0);
        }
    } else {
        const uint8_t *pb = cs.b + jl * kRowB + 16 * hl;
#pragma unroll
        for (int st = 0; st < kSteps; st += 2) {
            // lanes 0..31 carry step st, lanes 32..63 step st + 1 into the outer products
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.ws[st + hl][jl], cs.xs[st + hl][jl], v32f{0}, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const v4i aq = *reinterpret_cast<const v4i *>(pa + 32 * (st + e));
                const v4i bq = *reinterpret_cast<const v4i *>(pb + 32 * (st + e));
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[16 * e + v] = __builtin_fmaf((float)c[v], p[16 * e + v], acc[16 * e + v]);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (MINS)
                acc = __builtin_amdgcn_mfma_f32_32x32x1f32(-cs.wm[st + hl][jl], cs.xm[st + hl][jl], acc, 0, 0, 0);
        }
    }
}

// sk_compute for the 16-element-group formats without mins (Q6_K, Q3_K), 64 tokens: the two
// groups of a step each get their exact i32 dot from a K = 16 MFMA with the tokens as the A operand
// and the weights as the B operand (a lane holds weight row jl), combine in integers with the row's
// scales (below 2^24, exact in f32), and enter the accumulator through one fused multiply-add by
// xs * d. acc[16 tb + v]: token 32 tb + 8 (v / 4) + 4 hl + v % 4, row jl.
template <int Q>
__device__ __forceinline__ void sk16_compute(const GemmChunk<Q, 32, 64> &cs, const int (*sc)[32], const float *d,
                                             v32f &acc, int lane) {
    const int hl = lane >> 5, jl = lane & 31;
    const float dr = d[jl];
#pragma unroll 1
    for (int st = 0; st < kSteps; ++st) {  // (rolled: unrolled, the steps' registers spill)
        const int sc0 = sc[2 * st][jl], sc1 = sc[2 * st + 1][jl];
        // block b of the outer product: token 32 b + i (lane 32 b + i supplies its scale) times row jl's d
        const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.xs[st][lane], dr, v32f{0}, 0, 0, 0);
        long aq[2];
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) aq[gg] = *reinterpret_cast<const long *>(cs.a + jl * kRowB + 32 * st + 16 * gg + 8 * hl);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            v16i c[2];
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
                const long bq = *reinterpret_cast<const long *>(cs.b + (32 * tb + jl) * kRowB + 32 * st + 16 * gg + 8 * hl);
                c[gg] = __builtin_amdgcn_mfma_i32_32x32x16_i8(bq, aq[gg], v16i{0}, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
                acc[16 * tb + v] =
                    __builtin_fmaf((float)(__mul24(c[0][v], sc0) + __mul24(c[1][v], sc1)), p[16 * tb + v], acc[16 * tb + v]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int Q, int TM, int NW, bool XV>
__global__ __launch_bounds__(64 * NW) void gemm_tol_splitk_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y,
                                                                  int r0, int r1) {
    // 16-element groups (Q6_K, Q3_K) combine a step's two groups in integers: 64-token tiles
    constexpr bool G16 = GemmFmt<Q>::GK == 16;
    static_assert((TM == 32 || TM == 64) && (!G16 || (TM == 64 && !GemmFmt<Q>::MINS)),
                  "32-element groups on 32 or 64 tokens; 16-element groups without mins on 64");
    __shared__ __align__(16) SplitkSmem<Q, TM, NW> sm;
    __shared__ int s_sc16[G16 ? NW : 1][8][32];  // (G16) each wave's chunk: group scales per row
    __shared__ float s_d16[G16 ? NW : 1][32];    // and the rows' block scale d
    // (wave read as a scalar: the chunk loop's branches are then uniform, not exec-masked)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hl = lane >> 5, jl = lane & 31;
    // tile order as gemm_repacked_kernel: a row tile's token tiles on one XCD
    const int ntn = (r1 - r0 + 31) / 32, ntm = ((int)a.m + TM - 1) / TM;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;  // workgroup-uniform: the whole workgroup leaves before any barrier
    const int n0 = r0 + 32 * tn, m0 = TM * tm, M = (int)a.m;
    const int nchunks = w.cols / kKC;
    GemmChunk<Q, 32, TM> &cs = sm.cs[wave];

    v32f acc = v32f{0};
    // Chunks of this wave: wave, wave + NW, ... Every load is unconditional (a chunk past the
    // wave's last is read as its last again, from L2) so that the loads in flight are the same on
    // every path and each staging buffer's wait leaves the other buffer's loads in flight.
    const int cnt = (nchunks - wave + NW - 1) / NW;
    if (cnt > 0) {
        const int last = wave + NW * (cnt - 1);
        auto ck = [&](int i) { return min(wave + NW * i, last); };
        Stage<32, TM> ra, rb;
        // (the scheduling barriers keep each phase in place: the waits count loads in issue order,
        // so a buffer loaded out of turn -- here or in the loop -- would drain the other one too)
        chunk_load<Q, XV>(ra, w, a, n0, r1, m0, M, ck(0));
        __builtin_amdgcn_sched_barrier(0);
        chunk_load<Q, XV>(rb, w, a, n0, r1, m0, M, ck(1));
        __builtin_amdgcn_sched_barrier(0);
        auto store = [&](const Stage<32, TM> &r, int kc) {
            chunk_store<Q>(w, r, cs, kc);
            if constexpr (G16) tol16_scales<Q>(r, kc, lane, s_sc16[wave], s_d16[wave]);
        };
        auto compute = [&]() {
            if constexpr (G16) sk16_compute<Q>(cs, s_sc16[wave], s_d16[wave], acc, lane);
            else sk_compute(cs, acc, lane);
        };
        for (int i = 0; i < cnt; i += 2) {
            store(ra, ck(i));
            wave_lds_sync();
            __builtin_amdgcn_sched_barrier(0);
            chunk_load<Q, XV>(ra, w, a, n0, r1, m0, M, ck(i + 2));
            __builtin_amdgcn_sched_barrier(0);
            compute();
            wave_lds_sync();  // the chunk's LDS reads are done before the next store
            __builtin_amdgcn_sched_barrier(0);
            store(rb, ck(i + 1));
            wave_lds_sync();
            __builtin_amdgcn_sched_barrier(0);
            chunk_load<Q, XV>(rb, w, a, n0, r1, m0, M, ck(i + 3));
            __builtin_amdgcn_sched_barrier(0);
            if (i + 1 < cnt) compute();
            wave_lds_sync();
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    __syncthreads();  // every wave is done with its chunk before the partial tiles overwrite them
    // element v of block e: row 8 (v / 4) + 4 hl + v % 4; token jl of token block e (TM = 64)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 8 * (v >> 2) + 4 * hl + (v & 3);
        if constexpr (G16) {  // element 16 tb + v: token 32 tb + 8 (v / 4) + 4 hl + v % 4, row jl
            sm.red[wave][row][jl] = acc[v];
            sm.red[wave][32 + row][jl] = acc[16 + v];
        } else if constexpr (TM == 64) {
            sm.red[wave][jl][row] = acc[v];
            sm.red[wave][32 + jl][row] = acc[16 + v];
        } else {
            sm.red[wave][jl][row] = acc[v] + acc[16 + v];
        }
    }
    __syncthreads();
    const size_t ld = (size_t)(r1 - r0);
    for (int o = (int)threadIdx.x; o < TM * 32; o += 64 * NW) {
        const int tok = o >> 5, row = o & 31;
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < NW; ++v) s += sm.red[v][tok][row];
        if (m0 + tok < M && n0 + row < r1) y[(size_t)(m0 + tok) * ld + (size_t)(n0 + row - r0)] = s;
    }
}

// waves per workgroup (K = 4096: 32 chunks, 8 per wave): two workgroups per CU by registers, and
// eight waves per workgroup measured slower (their 1.75 rounds over the CUs against one)
constexpr int kSplitkNW = 4;

template <int Q, int TM, bool XV>
static void launch_splitk_t(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    const size_t ntn = (size_t)(r1 - r0 + 31) / 32, ntm = (a.m + TM - 1) / TM;
    JK_LAUNCH(TM == 32 ? "gemm_tol_splitk_kernel<32 tokens>" : "gemm_tol_splitk_kernel<64 tokens>",
              (gemm_tol_splitk_kernel<Q, TM, kSplitkNW, XV>), dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)),
                       dim3(64 * kSplitkNW), 0, s, w, a, y, r0, r1);
}

// (w.cols % 128 == 0, checked by the caller)
template <int Q>
static jk_status launch_splitk(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    // one load per thread for its chunk's activation scales (and sums), and one for its two weight
    // scales, when the rows allow it (w.nb % 4 == 0 follows from whole chunks)
    const bool xv = a.k_blocks32 % 4 == 0 && (uintptr_t)a.scales % 16 == 0 && (uintptr_t)a.sums % 16 == 0 &&
                    (uintptr_t)w.dplane % 4 == 0;
    if (a.m <= 32) {
        if (xv) launch_splitk_t<Q, 32, true>(s, w, a, y, r0, r1);
        else launch_splitk_t<Q, 32, false>(s, w, a, y, r0, r1);
    } else {
        if (xv) launch_splitk_t<Q, 64, true>(s, w, a, y, r0, r1);
        else launch_splitk_t<Q, 64, false>(s, w, a, y, r0, r1);
    }
    return check_launch("gemm_tol_splitk_kernel");
}

// Bit-exact block-scaled products with few row tiles (BitLinear at 16 or more tokens: TQ2_0 with
// GB = 8 32-element steps per weight block, I2_S with GB = 4), K split over the waves of a
// workgroup with the reference's order of additions kept. A workgroup owns 32 weight rows x 32
// tokens; the weight blocks go round-robin to its NW waves (round r: wave v takes block NW r + v).
// Per block a wave stages the block's chunks through the GEMM's coalesced loads (two chunks in
// flight), accumulates the exact i32 dot over its GB steps with MFMA, and writes the block's
// addend f32(dot) * (ws * xs) -- the scale product the single rounded f32 product, from an
// outer-product MFMA -- to an LDS table. After a barrier every thread adds the round's addends,
// for its outputs, in wave order, i.e. in block order, to an accumulator that started at 0.0:
// the same sum in the same order as gemm_repacked_kernel, bit for bit. The table is kept per
// round parity, so one barrier per round suffices.
template <int Q, int GB, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_block_splitk_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y,
                                                                    int r0, int r1) {
    static_assert(GemmFmt<Q>::GK == 32 && !GemmFmt<Q>::MINS && (GB == 4 || GB == 8), "blocks of 4 or 8 steps");
    static_assert(NW >= 4, "each thread adds four of the tile's 32 x 32 outputs");
    constexpr int UC = GB / 4;  // chunks per weight block
    __shared__ __align__(16) GemmChunk<Q, 32, 32> css[NW];
    __shared__ float tab[2][NW][32][33];  // [round parity][wave][token][row], rows padded to 33
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hl = lane >> 5, jl = lane & 31;
    const int ntn = (r1 - r0 + 31) / 32, ntm = ((int)a.m + 31) / 32;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;  // workgroup-uniform: the whole workgroup leaves before any barrier
    const int n0 = r0 + 32 * tn, m0 = 32 * tm, M = (int)a.m;
    const int nblocks = w.cols / (32 * GB), rounds = (nblocks + NW - 1) / NW;
    GemmChunk<Q, 32, 32> &cs = css[wave];

    // This wave's chunks in order: block wave + NW i, chunk c of it. Every wave loads, stages and
    // evaluates a block in every round -- past its last block (or with none: K below NW blocks)
    // it repeats a valid one whose addend is not used -- so that the loads in flight are the same
    // on every path and each staging buffer's wait leaves the other buffer's loads in flight.
    const int nmine = (nblocks - wave + NW - 1) / NW, lastq = max(nmine * UC - 1, 0);
    auto kc_of = [&](int q) {
        q = min(q, lastq);
        return nmine > 0 ? (wave + NW * (q / UC)) * UC + q % UC : q % UC;
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // outputs threadIdx.x + 64 NW i of the tile
    Stage<32, 32> ra, rb;
    chunk_load<Q>(ra, w, a, n0, r1, m0, M, kc_of(0));
    __builtin_amdgcn_sched_barrier(0);
    chunk_load<Q>(rb, w, a, n0, r1, m0, M, kc_of(1));
    __builtin_amdgcn_sched_barrier(0);
    v16i cacc = v16i{0};
    // one chunk: staged from r (which then loads chunk q + 2), its GB / UC = 4 steps added to cacc
    auto chunk = [&](Stage<32, 32> &r, int q) {
        chunk_store<Q>(w, r, cs, kc_of(q));
        wave_lds_sync();
        __builtin_amdgcn_sched_barrier(0);
        chunk_load<Q>(r, w, a, n0, r1, m0, M, kc_of(q + 2));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const v4i aq = *reinterpret_cast<const v4i *>(cs.a + jl * kRowB + 32 * st + 16 * hl);
            const v4i bq = *reinterpret_cast<const v4i *>(cs.b + jl * kRowB + 32 * st + 16 * hl);
            cacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, cacc, 0, 0, 0);
        }
    };
    // round rd: this wave's block NW rd + wave (chunks rd UC .. rd UC + UC - 1), then the ordered
    // addition; the staging buffer of chunk q is ra when q is even, so the caller passes the
    // buffers in chunk order (fixed registers on every path)
    auto round = [&](int rd, Stage<32, 32> &b0, Stage<32, 32> &b1) {
        chunk(b0, rd * UC);
        if constexpr (UC == 2) chunk(b1, rd * UC + 1);
        if (NW * rd + wave < nblocks) {  // wave-uniform; false only in the last round
            // the block's addend: lane l supplies the scale of row jl and of token jl (both halves
            // repeat them), so p[v] = ws(row 8 (v / 4) + 4 hl + v % 4) * xs(token jl)
            const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(cs.ws[kSteps - 1][jl], cs.xs[kSteps - 1][jl], v32f{0}, 0,
                                                                0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v)
                tab[rd & 1][wave][jl][8 * (v >> 2) + 4 * hl + (v & 3)] = (float)cacc[v] * p[v];
        }
        cacc = v16i{0};
        // LDS wait and barrier without a fence: the chunk loads in flight stay in flight
        stage_barrier();
        const int nv = min(NW, nblocks - NW * rd);  // blocks of this round
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (int)threadIdx.x + 64 * NW * i, tok = o >> 5, row = o & 31;
            if (o < 32 * 32)
                for (int v = 0; v < nv; ++v) acc[i] += tab[rd & 1][v][tok][row];
        }
    };
    if constexpr (UC == 2) {
        for (int rd = 0; rd < rounds; ++rd) round(rd, ra, rb);
    } else {
        // (pairs of rounds, the odd last one after the loop: the loop's back edge then always
        // follows the same loads, so the waits at its head stay exact)
        int rd = 0;
        for (; rd + 1 < rounds; rd += 2) {
            round(rd, ra, rb);
            round(rd + 1, rb, ra);
        }
        if (rd < rounds) round(rd, ra, rb);
    }
    const size_t ld = (size_t)(r1 - r0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int o = (int)threadIdx.x + 64 * NW * i, tok = o >> 5, row = o & 31;
        if (o < 32 * 32 && m0 + tok < M && n0 + row < r1) y[(size_t)(m0 + tok) * ld + (size_t)(n0 + row - r0)] = acc[i];
    }
}

// BitLinear token batches, one wave per 32 weight rows x 32 tokens with all of K in block order:
// each output has one owner, so the reference's order of additions needs no table or barrier.
// Per block the wave loads its rows' plane bytes and its tokens' activation bytes straight into
// registers (two blocks in flight; loads clamped past the ends and unconditional), unpacks each
// step's weight operand in registers (TQ2_0: dword 2 (st % 2) + hl of plane 2 (st / 4) +
// (st % 4) / 2 holds the step's 16 values of half hl, the 2-bit fields of its bytes in order;
// I2_S: field 6 - 2 st of plane hl), accumulates the exact i32 dot over the block's GB steps with
// MFMA and adds f32(dot) * (xs * ws) -- the scale product from an outer-product MFMA, a single
// rounded f32 product -- to an accumulator that started at 0.0 (ime.rs:882-938). Activations are
// the MFMA's A operand and weights its B operand, so a lane holds one weight row and a store
// instruction writes 32 consecutive rows of two tokens.
template <int Q> struct BlRegs {
    u32x4 w[Q == JK_TQ2_0 ? 4 : 1];  // TQ2_0: the block's four planes; I2_S: plane hl
    u32x4 x[Q == JK_TQ2_0 ? 8 : 4];  // step st: token jl's bytes 32 st + 16 hl ..
    uint32_t d;                      // TQ2_0: the block's f16 scale
};

template <int Q>
__global__ __launch_bounds__(64) void bitlinear_wave_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y, int r0,
                                                            int r1) {
    static_assert(Q == JK_TQ2_0 || Q == JK_I2_S, "ternary formats");
    constexpr int GB = Q == JK_TQ2_0 ? 8 : 4, BE = 32 * GB;  // steps and elements per weight block
    const int lane = threadIdx.x & 63, hl = lane >> 5, jl = lane & 31;
    const int ntn = (r1 - r0 + 31) / 32, ntm = ((int)a.m + 31) / 32;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;
    const int n0 = r0 + 32 * tn, m0 = 32 * tm, M = (int)a.m, nb = w.nb;
    const int row = min(n0 + jl, r1 - 1), tok = min(m0 + jl, M - 1);
    const uint8_t *xrow = reinterpret_cast<const uint8_t *>(a.qs) + (size_t)tok * a.k_padded + 16 * hl;
    const float xs = a.scales[(size_t)tok * a.k_blocks32];  // the token's scale (k_blocks32 = 1)
    // the row's planes (TQ2_0: all four; I2_S: plane hl) and scales, advanced by the block index
    constexpr int NP = Q == JK_TQ2_0 ? 4 : 1;
    const uint8_t *pbase[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) pbase[p] = plane_ptr(w, Q == JK_TQ2_0 ? p : hl, row, 0);
    const uint16_t *dbase = Q == JK_TQ2_0 ? w.dplane + (size_t)row * (size_t)nb : nullptr;
    auto load = [&](BlRegs<Q> &R, int b) {
        b = min(b, nb - 1);
#pragma unroll
        for (int p = 0; p < NP; ++p) R.w[p] = *reinterpret_cast<const u32x4 *>(pbase[p] + 16 * b);
        if constexpr (Q == JK_TQ2_0) R.d = dbase[b];
        const uint8_t *xb = xrow + (size_t)b * BE;
#pragma unroll
        for (int st = 0; st < GB; ++st) R.x[st] = *reinterpret_cast<const u32x4 *>(xb + 32 * st);
    };
    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    auto block = [&](const BlRegs<Q> &R) {
        v16i c = v16i{0};
#pragma unroll
        for (int st = 0; st < GB; ++st) {
            u32x4 wq;
            if constexpr (Q == JK_TQ2_0) {
                const uint32_t wv = R.w[2 * (st >> 2) + ((st & 3) >> 1)][2 * (st & 1) + hl];
                wq = u32x4{crumbs_minus1(wv & 0x03030303u), crumbs_minus1((wv >> 2) & 0x03030303u),
                           crumbs_minus1((wv >> 4) & 0x03030303u), crumbs_minus1((wv >> 6) & 0x03030303u)};
            } else {
                const int sh = 6 - 2 * st;
#pragma unroll
                for (int k = 0; k < 4; ++k) wq[k] = crumbs_minus1((R.w[0][k] >> sh) & 0x03030303u);
            }
            c = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, R.x[st]), __builtin_bit_cast(v4i, wq), c, 0,
                                                      0, 0);
        }
        const float ws = Q == JK_TQ2_0 ? f16_finite(R.d) : w.tensor_scale;
        // p[v] = xs(token 8 (v / 4) + 4 hl + v % 4) * ws(row jl)
        const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(xs, ws, v32f{0}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] += (float)c[v] * p[v];
    };
    BlRegs<Q> R0, R1;
    load(R0, 0);
    load(R1, 1);
    for (int b = 0; b < nb; b += 2) {
        block(R0);
        load(R0, b + 2);
        if (b + 1 >= nb) break;
        block(R1);
        load(R1, b + 3);
    }
    const size_t ld = (size_t)(r1 - r0);
    if (n0 + jl < r1)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = m0 + 8 * (v >> 2) + 4 * hl + (v & 3);
            if (m < M) y[(size_t)m * ld + (size_t)(n0 + jl - r0)] = acc[v];
        }
}

template <int Q>
static jk_status launch_bitlinear_wave(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y) {
    const size_t ntn = (size_t)(w.rows + 31) / 32, ntm = (a.m + 31) / 32;
    JK_LAUNCH("bitlinear_wave_kernel", bitlinear_wave_kernel<Q>, dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(64), 0, s, w, a, y, 0,
                       w.rows);
    return check_launch("bitlinear_wave_kernel");
}

// Tolerance-mode BitLinear token batches (jk_bitlinear_i8_tol). The order of the per-block
// addends is free here, so K is split over the waves of a workgroup: a workgroup owns 32 RT
// weight rows x 32 tokens with RT x KS waves; wave (rt, kq) computes rows 32 rt .. of the tile
// over the weight blocks kq, kq + KS, ... (at most MB of them), and the KS partial tiles of each
// row sub-tile are added through LDS at the end.
//  - Weights: the row's plane bytes straight into registers, unpacked per step as in
//    bitlinear_wave_kernel: I2_S (16 bytes a block) all of a wave's blocks at the start, TQ2_0
//    (64 bytes a block) one round ahead, which keeps it at 128 VGPRs or fewer.
//  - Activations: one round ahead. In round r the workgroup stages block kq + KS r of every K
//    slice kq for its 32 tokens in LDS (the RT waves of a slice share the slab and load a share of
//    it each), coalesced -- consecutive lanes read one token's contiguous bytes, so a load
//    instruction touches 4 (TQ2_0) or 8 (I2_S) cache lines instead of one line per lane -- with
//    the 16-byte piece p of token t at slot p ^ (t % (BE / 16)), so the 32 tokens of an MFMA
//    operand read fall on distinct banks in each group of 16 lanes. Two slab buffers; one barrier
//    per round (with one row sub-tile the slab is the wave's own, and a wave-level sync does).
//  - I2_S: every block shares the tensor scale, so a wave's dot over all its blocks accumulates
//    in the MFMA's i32 accumulator and the partials add in i32: the whole K sum is exact
//    (|sum| <= 128 K) and converted once, y = f32(sum) * (ts * xs). TQ2_0: one fused
//    multiply-add per block, acc = fma(f32(dot), d, acc) (d is the lane's row's block scale), and
//    the token's scale once at the end, y = acc * xs.
// Within 1e-5 of each token's output-row L2 norm of the reference's per-block order
// (ime.rs:882-938).
template <int Q> struct BlTolRegs {
    u32x4 w[Q == JK_TQ2_0 ? 4 : 1];  // TQ2_0: the block's four planes of row jl; I2_S: plane hl
    uint32_t d;                      // TQ2_0: the block's f16 scale
};
// blocks of weights a wave holds in registers
template <int Q> constexpr int kBlTolMaxBlocks = Q == JK_TQ2_0 ? 4 : 8;

template <int Q, int RT, int KS>
__global__ __launch_bounds__(64 * RT * KS) void bitlinear_tol_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y) {
    static_assert(Q == JK_TQ2_0 || Q == JK_I2_S, "ternary formats");
    constexpr int GB = Q == JK_TQ2_0 ? 8 : 4, BE = 32 * GB;  // steps and elements (bytes) per weight block
    constexpr int PR = BE / 16;                              // 16-byte pieces per token and block
    constexpr int XL = BE / 32 / RT;                         // pieces per lane: a slab is shared by RT waves
    static_assert(XL >= 1, "slab pieces per lane");
    constexpr int MB = kBlTolMaxBlocks<Q>;
    constexpr bool EXACT = Q == JK_I2_S;  // the partials are exact i32 sums
    constexpr int NW = RT * KS;
    union Smem {
        uint8_t x[2][KS][32 * BE];  // [round parity][K slice]: the block's 32 token rows, swizzled
        float part[NW][32][33];     // after the loop: [wave][token][row] (I2_S: i32 bits)
    };
    __shared__ __align__(16) Smem sm;
    const int lane = threadIdx.x & 63, hl = lane >> 5, jl = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int rt = wave % RT, kq = wave / RT;  // row sub-tile, K slice
    const int ntn = (w.rows + 32 * RT - 1) / (32 * RT), ntm = ((int)a.m + 31) / 32;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / ntm) * 8 + (wg & 7), tm = local % ntm;
    if (tn >= ntn) return;  // workgroup-uniform: the whole workgroup leaves before the barriers
    const int n0 = 32 * RT * tn + 32 * rt, m0 = 32 * tm, M = (int)a.m, nb = w.nb;
    const int row = min(n0 + jl, w.rows - 1);
    const int rounds = (nb + KS - 1) / KS;  // <= MB (the launcher's choice of KS)
    // every block of this wave's share into registers (past the last block a valid block is
    // re-read and not used)
    constexpr int NP = Q == JK_TQ2_0 ? 4 : 1;
    constexpr bool PRE = Q == JK_I2_S;  // all blocks' weights at the start (TQ2_0: one round ahead)
    BlTolRegs<Q> W[PRE ? MB : 2];
    const uint8_t *pbase[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) pbase[p] = plane_ptr(w, Q == JK_TQ2_0 ? p : hl, row, 0);
    const uint16_t *dbase = Q == JK_TQ2_0 ? w.dplane + (size_t)row * (size_t)nb : nullptr;
    auto wload = [&](BlTolRegs<Q> &R, int r) {
        const int b = min(kq + KS * r, nb - 1);
#pragma unroll
        for (int p = 0; p < NP; ++p) R.w[p] = *reinterpret_cast<const u32x4 *>(pbase[p] + 16 * b);
        if constexpr (Q == JK_TQ2_0) R.d = dbase[b];
    };
    if constexpr (PRE) {
#pragma unroll
        for (int r = 0; r < MB; ++r) wload(W[r], r);
    } else {
        wload(W[0], 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // this wave's share of its K slice's slab: piece f = 64 (RT i + rt) + lane is piece f % PR of
    // token f / PR
    const uint8_t *xsrc[XL];
    int xdst[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int f = 64 * (RT * i + rt) + lane, t = f / PR, p = f % PR;
        xsrc[i] = reinterpret_cast<const uint8_t *>(a.qs) + (size_t)min(m0 + t, M - 1) * a.k_padded + 16 * p;
        xdst[i] = t * BE + 16 * (p ^ (t & (PR - 1)));
    }
    u32x4 xr[XL];
    auto xload = [&](int r) {
        const int b = min(kq + KS * r, nb - 1);
#pragma unroll
        for (int i = 0; i < XL; ++i) xr[i] = *reinterpret_cast<const u32x4 *>(xsrc[i] + (size_t)b * BE);
    };
    v16i cacc = v16i{0};  // I2_S: the wave's i32 dot over all its blocks
    float acc[16];        // TQ2_0: sum of f32(dot) * d over the wave's blocks
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    xload(0);
    // round r: this wave's share of the slab (in xr) into buffer r % 2, barrier, the next round's
    // activation loads, then the block. The buffer written in round r was last read in round
    // r - 2, before every wave passed round r - 1's barrier.
#pragma unroll
    for (int r = 0; r < MB; ++r) {
        if (r >= rounds) break;  // workgroup-uniform
        uint8_t *xs = sm.x[r & 1][kq];
#pragma unroll
        for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4 *>(xs + xdst[i]) = xr[i];
        if constexpr (RT == 1) wave_lds_sync();  // the slab is this wave's own
        else lds_barrier();
        xload(r + 1);
        if constexpr (!PRE) wload(W[(r + 1) & 1], r + 1);
        __builtin_amdgcn_sched_barrier(0);  // (left to itself the compiler sinks the loads below the MFMAs)
        const BlTolRegs<Q> &Wr = W[PRE ? r : r & 1];
        v16i c = EXACT ? cacc : v16i{0};
#pragma unroll
        for (int st = 0; st < GB; ++st) {
            const int pc = 2 * st + hl;
            const v4i xq = *reinterpret_cast<const v4i *>(xs + jl * BE + 16 * (pc ^ (jl & (PR - 1))));
            u32x4 wq;
            if constexpr (Q == JK_TQ2_0) {
                const uint32_t wv = Wr.w[2 * (st >> 2) + ((st & 3) >> 1)][2 * (st & 1) + hl];
                wq = u32x4{crumbs_minus1(wv & 0x03030303u), crumbs_minus1((wv >> 2) & 0x03030303u),
                           crumbs_minus1((wv >> 4) & 0x03030303u), crumbs_minus1((wv >> 6) & 0x03030303u)};
            } else {
                const int sh = 6 - 2 * st;
#pragma unroll
                for (int k = 0; k < 4; ++k) wq[k] = crumbs_minus1((Wr.w[0][k] >> sh) & 0x03030303u);
            }
            c = __builtin_amdgcn_mfma_i32_32x32x32_i8(xq, __builtin_bit_cast(v4i, wq), c, 0, 0, 0);
        }
        if (kq + KS * r < nb) {  // wave-uniform: false for a repeated block past this slice's last one
            if constexpr (EXACT) {
                cacc = c;
            } else {
                const float d = f16_finite(Wr.d);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[v] = __builtin_fmaf((float)c[v], d, acc[v]);
            }
        }
    }
    __syncthreads();  // every wave done with the slabs before the partials overwrite them
    // lane holds row jl of tokens 8 (v / 4) + 4 hl + v % 4 of its sub-tile
#pragma unroll
    for (int v = 0; v < 16; ++v)
        sm.part[wave][8 * (v >> 2) + 4 * hl + (v & 3)][jl] = EXACT ? __int_as_float(cacc[v]) : acc[v];
    __syncthreads();
    const size_t ld = (size_t)w.rows;
    const int nbase = 32 * RT * tn;
    for (int o = (int)threadIdx.x; o < RT * 32 * 32; o += 64 * NW) {
        const int sub = o >> 10, t = (o >> 5) & 31, rr = o & 31, n = nbase + 32 * sub + rr;
        if (m0 + t >= M || n >= w.rows) continue;
        const float xsc = a.scales[(size_t)(m0 + t) * a.k_blocks32];  // the token's scale (k_blocks32 = 1)
        float out;
        if constexpr (EXACT) {
            int sum = 0;
#pragma unroll
            for (int v = 0; v < KS; ++v) sum += __float_as_int(sm.part[RT * v + sub][t][rr]);
            out = (float)sum * (w.tensor_scale * xsc);
        } else {
            float sum = 0.0f;
#pragma unroll
            for (int v = 0; v < KS; ++v) sum += sm.part[RT * v + sub][t][rr];
            out = sum * xsc;
        }
        y[(size_t)(m0 + t) * ld + (size_t)n] = out;
    }
}

template <int Q, int RT, int KS>
static void launch_bl_tol_t(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, const char *name) {
    const size_t ntn = (size_t)(w.rows + 32 * RT - 1) / (32 * RT), ntm = (a.m + 31) / 32;
    JK_LAUNCH(name, (bitlinear_tol_kernel<Q, RT, KS>), dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(64 * RT * KS), 0,
              s, w, a, y);
}

// K split over the fewest waves (2, 4 or 8) that leaves each at most kBlTolMaxBlocks blocks (K up
// to 8192);
// 64-row tiles (two row sub-tiles sharing each activation slab) where those give every CU a
// workgroup, 32-row tiles below. (false: K too long for 8 waves; the caller runs the bit-exact
// launch.)
template <int Q>
static bool launch_bitlinear_tol(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y) {
    constexpr int MB = kBlTolMaxBlocks<Q>;
    const int nb = w.nb;
    const bool rt2 = (long)((w.rows + 63) / 64) * (long)((a.m + 31) / 32) >= cu_count();
    if (nb <= 2 * MB) {
        if (rt2) launch_bl_tol_t<Q, 2, 2>(s, w, a, y, "bitlinear_tol_kernel<2x2 waves>");
        else launch_bl_tol_t<Q, 1, 2>(s, w, a, y, "bitlinear_tol_kernel<1x2 waves>");
    } else if (nb <= 4 * MB) {
        if (rt2) launch_bl_tol_t<Q, 2, 4>(s, w, a, y, "bitlinear_tol_kernel<2x4 waves>");
        else launch_bl_tol_t<Q, 1, 4>(s, w, a, y, "bitlinear_tol_kernel<1x4 waves>");
    } else if (nb <= 8 * MB) {
        // (TQ2_0 on 16 waves would spill)
        if constexpr (Q == JK_I2_S) {
            if (rt2) launch_bl_tol_t<Q, 2, 8>(s, w, a, y, "bitlinear_tol_kernel<2x8 waves>");
            else launch_bl_tol_t<Q, 1, 8>(s, w, a, y, "bitlinear_tol_kernel<1x8 waves>");
        } else {
            launch_bl_tol_t<Q, 1, 8>(s, w, a, y, "bitlinear_tol_kernel<1x8 waves>");
        }
    } else {  // (16 waves would spill: 1024 threads leave 128 VGPRs a lane)
        return false;
    }
    return true;
}

constexpr int kBlockSplitkNW = 4;  // (8 waves measured slower on both 128-token BitLinear shapes)

template <int Q, int GB>
static jk_status launch_block_splitk(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    const size_t ntn = (size_t)(r1 - r0 + 31) / 32, ntm = (a.m + 31) / 32;
    JK_LAUNCH("gemm_block_splitk_kernel", (gemm_block_splitk_kernel<Q, GB, kBlockSplitkNW>), dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)),
                       dim3(64 * kBlockSplitkNW), 0, s, w, a, y, r0, r1);
    return check_launch("gemm_block_splitk_kernel");
}

// Tile shape of a launch: the largest tile that still gives every CU two workgroups, down to the
// 32 x 16 single-wave tiles (not for Q6_K). (Four 32 x 32 tiles per CU beat the 32 x 16 tiles
// with the weights cold in HBM: those re-read every weight tile twice as often.)
static int gemm_tile(int quant, long rows, long m) {
    const long ncu = cu_count();
    auto tiles = [&](long tn, long tm) { return (rows + tn - 1) / tn * ((m + tm - 1) / tm); };
    // (the 16-element-group formats do not fit the 128 x 64 tile's register budget without spills)
    if (tiles(128, 64) >= 2 * ncu && quant != JK_Q2_K && quant != JK_Q3_K && quant != JK_Q6_K) return 0;
    if (tiles(64, 64) >= 2 * ncu) return 1;
    if (tiles(32, 32) >= 2 * ncu || quant == JK_Q6_K || quant == JK_Q3_K || quant == JK_Q2_K) return 2;
    return 3;
}

static const char *tile_kernel_name(int tn, int tm, bool tol) {
    if (tol) return tn == 32 ? "gemm_repacked_kernel<32x32, tolerance>" : "gemm_repacked_kernel<tolerance>";
    if (tn == 128) return "gemm_repacked_kernel<128x64>";
    if (tn == 64) return "gemm_repacked_kernel<64x64>";
    return tm == 32 ? "gemm_repacked_kernel<32x32>" : "gemm_repacked_kernel<32x16>";
}

template <int Q, int GB, int TN, int TM, bool TOL = false>
static void launch_tile(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    const size_t ntn = (size_t)(r1 - r0 + TN - 1) / TN, ntm = (a.m + TM - 1) / TM;
    const dim3 grid((unsigned)((ntn + 7) / 8 * 8 * ntm)), block(Tile<TN, TM>::THREADS);
    JK_LAUNCH(tile_kernel_name(TN, TM, TOL), (gemm_repacked_kernel<Q, GB, TN, TM, TOL>), grid, block, 0, s, w, a, y,
              r0, r1);
}

template <int Q, int GB>
static jk_status launch_gemm(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    if constexpr (Q == JK_Q8_0 && GB == 1) {
        // Q8_0 with per-32 activation scales (not BitLinear's one scale per token), whole 128-element
        // chunks, 1.5 to 2 128 x 128 tiles per CU (one round of two resident workgroups a CU) or 6 and
        // more: the global-to-LDS staged tiles (14336 x 4096: 144 against 164 us at 512 tokens, 477
        // against 505 at 2048; at 768-1536 tokens the register-staged 128 x 64 tiles tie or win by 2%)
        const long ncu = cu_count();
        const long t128 = (long)(r1 - r0 + 127) / 128 * (((long)a.m + 127) / 128);
        const bool one_round = 2 * t128 >= 3 * ncu && t128 <= 2 * ncu;
        if ((one_round || t128 >= 6 * ncu) && w.cols % 128 == 0 && a.k_blocks32 * 32 == (size_t)w.cols) {
            const size_t ntn = (size_t)(r1 - r0 + 127) / 128, ntm = (a.m + 127) / 128;
            JK_LAUNCH("gemm_q8_0_exact_dma_128", gemm_q8_0_exact_dma_128, dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)),
                      dim3(256), 0, s, w, a, y, r0, r1);
            return check_launch("gemm_q8_0_exact_dma");
        }
    }
    switch (gemm_tile(Q, r1 - r0, (long)a.m)) {
    case 0:
        if constexpr (GemmFmt<Q>::GK == 32) launch_tile<Q, GB, 128, 64>(s, w, a, y, r0, r1);
        break;
    case 1: launch_tile<Q, GB, 64, 64>(s, w, a, y, r0, r1); break;
    case 2: launch_tile<Q, GB, 32, 32>(s, w, a, y, r0, r1); break;
    default:
        if constexpr (GemmFmt<Q>::GK == 32) {
            const size_t ntn = (size_t)(r1 - r0 + 31) / 32, ntm = (a.m + 15) / 16;
            JK_LAUNCH("gemm16_kernel", (gemm16_kernel<Q, GB>), dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(64), 0, s, w,
                               a, y, r0, r1);
        } else {
            launch_tile<Q, GB, 32, 32>(s, w, a, y, r0, r1);  // not chosen for 16-element groups
        }
        break;
    }
    return check_launch("gemm_repacked_kernel");
}

// Tolerance-mode launch. The bit-exact kernels' results are within the tolerance by definition,
// so the launch takes whichever measured faster: 128 x 128 tolerance tiles with at least 1.5
// tiles per CU, K split over the waves where the tiled launch would fall back to single-wave
// 32-row tiles, the bit-exact launch for the 128 x 64 and 64 x 64 tiles (Q8_0 / Q4_0 / Q4_K
// 14336 x 4096 at 160 to 384 tokens: 6-19% faster than those tiles' tolerance variant, and
// than 128 x 128 tiles at 1.3 per CU), and 32 x 32 tolerance tiles in place of the
// 32 x 16 single-wave ones (VALU scale products).
template <int Q>
static jk_status launch_gemm_tol(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    // The 16-element-group formats: Q6_K and Q3_K combine a step's two groups in integers (128 x 128
    // tiles from 1.5 per CU, K split over the waves of a workgroup below); Q2_K, and Q3_K between 64
    // tokens and the tiles, run the bit-exact kernel.
    if constexpr (GemmFmt<Q>::GK == 16) {
        if constexpr (Q == JK_Q6_K || Q == JK_Q3_K) {
            const long ncu = cu_count();
            const long t128 = (long)(r1 - r0 + 127) / 128 * (((long)a.m + 127) / 128);
            if (2 * t128 >= 3 * ncu && w.cols % 128 == 0) {
                const size_t ntn = (size_t)(r1 - r0 + 127) / 128, ntm = (a.m + 127) / 128;
                JK_LAUNCH("gemm_tol16_kernel", gemm_tol16_kernel<Q>, dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(256), 0, s, w,
                                   a, y, r0, r1);
                return check_launch("gemm_tol16_kernel");
            }
            // below that, K split over the waves of a workgroup: Q6_K at every token count (14336 x 4096
            // at 192 / 256 / 384 tokens 122.9 / 145.9 / 220.0 us against 146.6 / 162.6 / 245.1 us for
            // the bit-exact tiles), Q3_K up to 64 tokens (its heavier unpack lost at 128 tokens: 104.7
            // against 101.3 us)
            if ((Q == JK_Q6_K || a.m <= 64) && w.cols % 128 == 0) {
                const bool xv = a.k_blocks32 % 4 == 0 && (uintptr_t)a.scales % 16 == 0;
                if (xv) launch_splitk_t<Q, 64, true>(s, w, a, y, r0, r1);
                else launch_splitk_t<Q, 64, false>(s, w, a, y, r0, r1);
                return check_launch("gemm_tol_splitk_kernel");
            }
        }
        return launch_gemm<Q, 1>(s, w, a, y, r0, r1);
    } else {
        const long ncu = cu_count();
        const long t128 = (long)(r1 - r0 + 127) / 128 * (((long)a.m + 127) / 128);
        if (2 * t128 >= 3 * ncu && w.cols % 128 == 0) {  // at least 1.5 128 x 128 tiles per CU; whole chunks
            const size_t ntn = (size_t)(r1 - r0 + 127) / 128, ntm = (a.m + 127) / 128;
            if constexpr (Q == JK_Q8_0) {
                // (256-row tiles, one workgroup per CU, measured slower at 512 and 2048 tokens)
                JK_LAUNCH("gemm_q8_0_tol_dma_128", gemm_q8_0_tol_dma_128, dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(256), 0, s, w,
                                   a, y, r0, r1);
                return check_launch("gemm_q8_0_tol_dma");
            }
            JK_LAUNCH("gemm_tol_kernel", gemm_tol_kernel<Q>, dim3((unsigned)((ntn + 7) / 8 * 8 * ntm)), dim3(256), 0, s, w, a, y,
                               r0, r1);
            return check_launch("gemm_tol_kernel");
        }
        // where the tiled launch would fall back to single-wave 32-row tiles (Q8_0 14336 rows:
        // up to 128 tokens), K is split instead
        if (w.cols % 128 == 0 && gemm_tile(Q, r1 - r0, (long)a.m) >= 2) return launch_splitk<Q>(s, w, a, y, r0, r1);
        if (gemm_tile(Q, r1 - r0, (long)a.m) < 2) return launch_gemm<Q, 1>(s, w, a, y, r0, r1);
        launch_tile<Q, 1, 32, 32, true>(s, w, a, y, r0, r1);
        return check_launch("gemm_repacked_kernel");
    }
}

jk_status launch_gemm_repacked_tol(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    if (a.m <= 2) return launch_gemv_repacked(s, w, a, y, r0, r1);
    switch (w.quant) {
    case JK_Q8_0: return launch_gemm_tol<JK_Q8_0>(s, w, a, y, r0, r1);
    case JK_Q4_0: return launch_gemm_tol<JK_Q4_0>(s, w, a, y, r0, r1);
    case JK_Q5_0: return launch_gemm_tol<JK_Q5_0>(s, w, a, y, r0, r1);
    case JK_Q4_K: return launch_gemm_tol<JK_Q4_K>(s, w, a, y, r0, r1);
    case JK_Q5_K: return launch_gemm_tol<JK_Q5_K>(s, w, a, y, r0, r1);
    case JK_Q4_1: return launch_gemm_tol<JK_Q4_1>(s, w, a, y, r0, r1);
    case JK_Q5_1: return launch_gemm_tol<JK_Q5_1>(s, w, a, y, r0, r1);
    case JK_IQ4_NL: return launch_gemm_tol<JK_IQ4_NL>(s, w, a, y, r0, r1);
    case JK_Q2_K: return launch_gemm_tol<JK_Q2_K>(s, w, a, y, r0, r1);
    case JK_Q3_K: return launch_gemm_tol<JK_Q3_K>(s, w, a, y, r0, r1);
    case JK_Q6_K: return launch_gemm_tol<JK_Q6_K>(s, w, a, y, r0, r1);
    case JK_TQ2_0: return launch_gemm_tol<JK_TQ2_0>(s, w, a, y, r0, r1);
    case JK_I2_S: return launch_gemm_tol<JK_I2_S>(s, w, a, y, r0, r1);
    default: return fail(JK_CAPABILITY_MISMATCH, "gemm: unsupported quant %d", w.quant);
    }
}

// bitlinear_i8_rvv (ime.rs:882-938) for m tokens on int8 MFMA: the activation rows act[m][k]
// are read as the GEMM's quantized rows (row stride k) and the per-token scale as a single
// "per-32" scale column (k_blocks32 = 1, every block index clamps to it).
jk_status launch_bitlinear_mfma(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales, int m,
                                float *y) {
    jk_act_q8 a;
    memset(&a, 0, sizeof a);
    a.m = (size_t)m;
    a.k = a.k_padded = (size_t)w.cols;
    a.k_blocks32 = 1;
    a.qs = const_cast<int8_t *>(act);
    a.scales = const_cast<float *>(act_scales);
    // where the tiled launch would fall back to single-wave 32-row tiles (2560 x 6912 and
    // 6912 x 2560 at 128 tokens): one wave per 32 x 32 tile over all of K when those tiles give
    // every CU two waves (6912 x 2560: 864 tiles; TQ2_0 19.3 -> 15.1 us, I2_S 21.6 -> 14.2 us), and
    // otherwise K split over the waves of a workgroup (2560 x 6912: 320 tiles of 27 blocks, where
    // the single-wave chains took 25.0 us against 20.8 us). The wave kernel reads the activation
    // rows with 16-byte loads, so it takes 16-byte aligned ones.
    const bool split = gemm_tile(w.quant, w.rows, m) >= 2;
    const long tiles = (long)(w.rows + 31) / 32 * (long)((m + 31) / 32);
    const bool wave = split && tiles >= 2 * cu_count() && (uintptr_t)act % 16 == 0;
    switch (w.quant) {
    case JK_TQ2_0: return wave    ? launch_bitlinear_wave<JK_TQ2_0>(s, w, a, y)
                          : split ? launch_block_splitk<JK_TQ2_0, 8>(s, w, a, y, 0, w.rows)
                                  : launch_gemm<JK_TQ2_0, 8>(s, w, a, y, 0, w.rows);
    case JK_I2_S: return wave    ? launch_bitlinear_wave<JK_I2_S>(s, w, a, y)
                         : split ? launch_block_splitk<JK_I2_S, 4>(s, w, a, y, 0, w.rows)
                                 : launch_gemm<JK_I2_S, 4>(s, w, a, y, 0, w.rows);
    case JK_Q8_0: return launch_gemm<JK_Q8_0, 1>(s, w, a, y, 0, w.rows);
    default: return fail(JK_CAPABILITY_MISMATCH, "bitlinear: unsupported quant %d", w.quant);
    }
}

// Tolerance mode of the token-batch BitLinear: the K-split kernel above for TQ2_0 / I2_S with
// 16-byte aligned activation rows and K up to 16 waves' register blocks; otherwise (Q8_0,
// unaligned rows, longer K) the bit-exact launch, whose results meet the tolerance by definition.
jk_status launch_bitlinear_mfma_tol(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales,
                                    int m, float *y) {
    if ((w.quant != JK_TQ2_0 && w.quant != JK_I2_S) || (uintptr_t)act % 16 != 0)
        return launch_bitlinear_mfma(s, w, act, act_scales, m, y);
    jk_act_q8 a;
    memset(&a, 0, sizeof a);
    a.m = (size_t)m;
    a.k = a.k_padded = (size_t)w.cols;
    a.k_blocks32 = 1;
    a.qs = const_cast<int8_t *>(act);
    a.scales = const_cast<float *>(act_scales);
    const bool done = w.quant == JK_TQ2_0 ? launch_bitlinear_tol<JK_TQ2_0>(s, w, a, y)
                                          : launch_bitlinear_tol<JK_I2_S>(s, w, a, y);
    if (!done) return launch_bitlinear_mfma(s, w, act, act_scales, m, y);
    return check_launch("bitlinear_tol_kernel");
}

jk_status launch_gemm_repacked(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    if (a.m <= 2) return launch_gemv_repacked(s, w, a, y, r0, r1);
    switch (w.quant) {
    case JK_Q8_0: return launch_gemm<JK_Q8_0, 1>(s, w, a, y, r0, r1);
    case JK_Q4_0: return launch_gemm<JK_Q4_0, 1>(s, w, a, y, r0, r1);
    case JK_Q5_0: return launch_gemm<JK_Q5_0, 1>(s, w, a, y, r0, r1);
    case JK_Q4_K: return launch_gemm<JK_Q4_K, 1>(s, w, a, y, r0, r1);
    case JK_Q5_K: return launch_gemm<JK_Q5_K, 1>(s, w, a, y, r0, r1);
    case JK_Q4_1: return launch_gemm<JK_Q4_1, 1>(s, w, a, y, r0, r1);
    case JK_Q5_1: return launch_gemm<JK_Q5_1, 1>(s, w, a, y, r0, r1);
    case JK_IQ4_NL: return launch_gemm<JK_IQ4_NL, 1>(s, w, a, y, r0, r1);
    case JK_Q2_K: return launch_gemm<JK_Q2_K, 1>(s, w, a, y, r0, r1);
    case JK_Q3_K: return launch_gemm<JK_Q3_K, 1>(s, w, a, y, r0, r1);
    case JK_Q6_K: return launch_gemm<JK_Q6_K, 1>(s, w, a, y, r0, r1);
    case JK_TQ2_0: return launch_gemm<JK_TQ2_0, 1>(s, w, a, y, r0, r1);
    case JK_I2_S: return launch_gemm<JK_I2_S, 1>(s, w, a, y, r0, r1);
    default: return fail(JK_CAPABILITY_MISMATCH, "gemm: unsupported quant %d", w.quant);
    }
}

}  // namespace jk
