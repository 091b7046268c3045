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
// Tiling: a workgroup of 4 waves computes a 128 (weight rows) x 64 (tokens) tile, each
// wave 64 x 32 as two 32x32 MFMA tiles. K advances in chunks of 256 elements (8 steps of
// 32; one super-block of the 256-element formats): while the 8 steps of a chunk are
// evaluated from LDS, the next chunk's weights (unpacked from the plane layout to i8),
// activations and scales are loaded into registers -- each pair of threads reads whole
// 128-byte lines of a row -- and written to LDS after a barrier. LDS rows are padded from
// 256 to 272 bytes so the 16-byte fragment reads of 16 lanes land on distinct banks.
#include "jk_device.hpp"

namespace jk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTN = 128;   // weight rows per workgroup
constexpr int kTM = 64;    // tokens per workgroup
constexpr int kKC = 256;   // K elements per chunk
constexpr int kRowB = 272; // padded LDS bytes per 256-byte row

template <int Q> struct GemmFmt {
    static constexpr int GK = Q == JK_Q6_K ? 16 : 32;  // elements per scale group
    static constexpr bool MINS = Q == JK_Q4_K;
    static constexpr int NG = 128 / GK;                 // scale groups per half chunk
};

struct GemmChunk {
    uint8_t a[kTN * kRowB];  // weights, i8, [row][k]
    uint8_t b[kTM * kRowB];  // activations, i8, [token][k]
    float ws[16][kTN];       // weight scale per scale group of the chunk
    float wm[8][kTN];        // weight min per 32-group (Q4_K)
    float xs[8][kTM];        // activation scale per 32-block
    float xm[8][kTM];        // activation sum per 32-block (Q4_K)
};

// One 16-byte global load without the streaming hint: a weight tile is read once per
// token tile, so its lines are meant to stay in L2 for the neighbouring workgroups.
__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ __forceinline__ const uint8_t *plane_ptr(const WeightDev &w, int c, int r, int b) {
    return w.planes + ((((size_t)c * (size_t)w.rows + (size_t)r) * (size_t)w.nb + (size_t)b) << 4);
}

// Raw bytes of one thread's share of a chunk, exactly as stored in the plane layout, plus
// raw f16 scales. Loading and unpacking are separate so that every global load of a chunk
// is in flight while the previous chunk is evaluated; nothing between the loads depends on
// a loaded value.
//  Q8_0 / Q4_0: a chunk is 8 blocks, 128 contiguous bytes per (plane, row): 8 consecutive
//   lanes read one such line (piece t % 8 = block 8kc + t % 8), load i covers rows
//   32 (i % 4) + t / 8 of plane i / 4. Scales: row t / 2, blocks 8kc + 4 (t % 2) ..
//  K-quants, TQ2_0, I2_S: 16 or 32 bytes per (plane, row) and chunk; thread t takes row
//   t / 2 and the half t % 2 of the chunk's elements (128h .. 128h+127).
template <int Q> struct RawW {
    static constexpr int NV = Q == JK_Q8_0 ? 8 : Q == JK_Q4_0 ? 4 : Q == JK_Q4_K ? 5 : Q == JK_Q6_K ? 7 : 2;
    static constexpr int ND = Q == JK_Q8_0 || Q == JK_Q4_0 ? 4 : 1;
    uint4 v[NV];
    uint32_t d[ND];
};

// Blocks past the row end (a partial last chunk) are read clamped and never used; rows
// past r1 are read clamped to r1 - 1 and never stored.
template <int Q>
__device__ __forceinline__ void chunk_w_load(const WeightDev &w, int n0, int r1, int kc, RawW<Q> &r) {
    const int nb = w.nb, t = threadIdx.x;
    if constexpr (Q == JK_Q8_0 || Q == JK_Q4_0) {
        const int b = min(8 * kc + (t & 7), nb - 1);
#pragma unroll
        for (int i = 0; i < RawW<Q>::NV; ++i) {
            const int n = min(n0 + 32 * (i & 3) + (t >> 3), r1 - 1);
            r.v[i] = ldg16(plane_ptr(w, i >> 2, n, b));
        }
        const int n = min(n0 + (t >> 1), r1 - 1);
        const size_t srow = (size_t)n * (size_t)nb;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.d[j] = w.dplane[srow + (size_t)min(8 * kc + 4 * (t & 1) + j, nb - 1)];
    } else {
        const int n = min(n0 + (t >> 1), r1 - 1), h = t & 1;
        if constexpr (Q == JK_Q4_K) {
            r.v[0] = ldg16(plane_ptr(w, 0, n, kc));  // d, dmin, 12 packed 6-bit scales / mins
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                r.v[1 + 2 * c] = ldg16(plane_ptr(w, 1 + 2 * (2 * h + c), n, kc));
                r.v[2 + 2 * c] = ldg16(plane_ptr(w, 2 + 2 * (2 * h + c), n, kc));
            }
        } else if constexpr (Q == JK_Q6_K) {
#pragma unroll
            for (int c = 0; c < 4; ++c) r.v[c] = ldg16(plane_ptr(w, 4 * h + c, n, kc));      // ql
#pragma unroll
            for (int c = 0; c < 2; ++c) r.v[4 + c] = ldg16(plane_ptr(w, 8 + 2 * h + c, n, kc));  // qh
            r.v[6] = ldg16(plane_ptr(w, 12, n, kc));                                          // i8 scales
            r.d[0] = w.dplane[(size_t)n * (size_t)nb + (size_t)kc];
        } else if constexpr (Q == JK_TQ2_0) {
#pragma unroll
            for (int c = 0; c < 2; ++c) r.v[c] = ldg16(plane_ptr(w, 2 * h + c, n, kc));
            r.d[0] = w.dplane[(size_t)n * (size_t)nb + (size_t)kc];
        } else {  // JK_I2_S: chunk = blocks 2kc, 2kc + 1; half h = block 2kc + h
            const int b = min(2 * kc + h, nb - 1);
#pragma unroll
            for (int c = 0; c < 2; ++c) r.v[c] = ldg16(plane_ptr(w, c, n, b));
        }
    }
}

// The loaded half of the per-row formats as 128 i8 values (q[i]: elements 128h + 16i ..)
// with repack_block_scaled_range_into_i8's values (repack.rs:1724-2103), and the weight
// scale / min of each of its scale groups.
template <int Q>
__device__ __forceinline__ void chunk_w_unpack(const WeightDev &w, const RawW<Q> &r, int h, uint4 (&q)[8],
                                               float (&ws)[8], float (&wm)[4]) {
    if constexpr (Q == JK_Q4_K) {
        // unpack_k4_scales_mins (repack.rs:1158-1170); qs chunk pair (2c, 2c+1) holds
        // elements 64c .. 64c+63 (low nibbles first)
        const uint4 hd = r.v[0];
        const float d = f16_finite(hd.x & 0xFFFFu), dmin = f16_finite(hd.x >> 16);
        const uint32_t sc = h == 0 ? (hd.y & 0x3F3F3F3Fu) : ((hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u));
        const uint32_t mv = h == 0 ? (hd.z & 0x3F3F3F3Fu) : (((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            ws[t] = d * (float)((sc >> (8 * t)) & 255u);
            wm[t] = dmin * (float)((mv >> (8 * t)) & 255u);
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 v0 = r.v[1 + 2 * c], v1 = r.v[2 + 2 * c];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int sh = 4 * hh;
                q[4 * c + 2 * hh] = make_uint4((v0.x >> sh) & 0x0F0F0F0Fu, (v0.y >> sh) & 0x0F0F0F0Fu,
                                               (v0.z >> sh) & 0x0F0F0F0Fu, (v0.w >> sh) & 0x0F0F0F0Fu);
                q[4 * c + 2 * hh + 1] = make_uint4((v1.x >> sh) & 0x0F0F0F0Fu, (v1.y >> sh) & 0x0F0F0F0Fu,
                                                   (v1.z >> sh) & 0x0F0F0F0Fu, (v1.w >> sh) & 0x0F0F0F0Fu);
            }
        }
    } else if constexpr (Q == JK_Q6_K) {
        // dequantize_q6_k_block's element order (quant.rs:594-648): 16-group g of half h
        // (quarter g / 2, is = g % 2) takes ql bytes 16is + 32(quarter & 1) of the half, qh
        // bytes 16is, the low / high nibble and 2-bit field by quarter, scale 8h + g
        const float d = f16_finite(r.d[0]);
        const uint4 scv = r.v[6];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int quarter = g >> 1, is = g & 1, j = 8 * h + g;
            ws[g] = d * (float)(int8_t)(comp(scv, j >> 2) >> (8 * (j & 3)));
            const uint4 lv = r.v[is + 2 * (quarter & 1)], hv = r.v[4 + is];
            const int lsh = quarter < 2 ? 0 : 4, hsh = 2 * quarter;
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t v6 = ((comp(lv, i) >> lsh) & 0x0F0F0F0Fu) | (((comp(hv, i) >> hsh) & 0x03030303u) << 4);
                o[i] = (uint32_t)bytes_sub(v6, 0x20202020u);
            }
            q[g] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else if constexpr (Q == JK_TQ2_0) {
        const float d = f16_finite(r.d[0]);
#pragma unroll
        for (int t = 0; t < 4; ++t) ws[t] = d;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 v = r.v[c];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t wv = comp(v, k);
                q[4 * c + k] = make_uint4((uint32_t)bytes_sub(wv & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((wv >> 2) & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((wv >> 4) & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((wv >> 6) & 0x03030303u, 0x01010101u));
            }
        }
    } else {  // JK_I2_S: group t = 2-bit field t (shift 6 - 2t) of both chunks
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            ws[t] = w.tensor_scale;
            const int sh = 6 - 2 * t;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint4 v = r.v[c];
                q[2 * t + c] = make_uint4((uint32_t)bytes_sub((v.x >> sh) & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((v.y >> sh) & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((v.z >> sh) & 0x03030303u, 0x01010101u),
                                          (uint32_t)bytes_sub((v.w >> sh) & 0x03030303u, 0x01010101u));
            }
        }
    }
}

// Registers of one chunk's staging. Thread t stages weight row t / 2, half t % 2, and
// activation token t / 4, quarter t % 4 (k 64 * (t % 4) ..), with that token's scales
// (and sums) of steps 2 * (t % 4) and 2 * (t % 4) + 1.
template <int Q> struct ChunkRegs {
    RawW<Q> w;
    uint4 xq[4];
    float xs[2], xm[2];
};

// Activations: 64 tokens x 256 bytes, 16 consecutive lanes per token row (load i: token
// 16i + t / 16, piece t % 16); scales (and sums) of token t / 4, steps 2 (t % 4) + {0, 1}.
template <int Q>
__device__ __forceinline__ void chunk_load(ChunkRegs<Q> &r, const WeightDev &w, const jk_act_q8 &a, int n0, int r1,
                                           int m0, int M, int kc) {
    const int t = threadIdx.x;
    chunk_w_load<Q>(w, n0, r1, kc, r.w);
    int k = kKC * kc + 16 * (t & 15);
    if (k >= (int)a.k_padded) k = 0;  // past the row end (partial chunk): in bounds, unused
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = min(m0 + 16 * i + (t >> 4), M - 1);
        r.xq[i] = ldg16(reinterpret_cast<const uint8_t *>(a.qs) + (size_t)m * a.k_padded + k);
    }
    const int m = min(m0 + (t >> 2), M - 1), qq = t & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int b = min(8 * kc + 2 * qq + i, (int)a.k_blocks32 - 1);
        r.xs[i] = a.scales[(size_t)m * a.k_blocks32 + b];
        r.xm[i] = GemmFmt<Q>::MINS ? a.sums[(size_t)m * a.k_blocks32 + b] : 0.0f;
    }
}

template <int Q>
__device__ __forceinline__ void chunk_store(const WeightDev &w, const ChunkRegs<Q> &r, GemmChunk &c) {
    using F = GemmFmt<Q>;
    const int t = threadIdx.x;
    if constexpr (Q == JK_Q8_0 || Q == JK_Q4_0) {
        const int piece = t & 7;
#pragma unroll
        for (int i = 0; i < RawW<Q>::NV; ++i) {
            uint8_t *dst = c.a + (32 * (i & 3) + (t >> 3)) * kRowB + 32 * piece;
            if constexpr (Q == JK_Q8_0) {
                *reinterpret_cast<uint4 *>(dst + 16 * (i >> 2)) = r.w.v[i];
            } else {
                const uint4 v = r.w.v[i];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int sh = 4 * hh;
                    *reinterpret_cast<uint4 *>(dst + 16 * hh) =
                        make_uint4((uint32_t)bytes_sub((v.x >> sh) & 0x0F0F0F0Fu, 0x08080808u),
                                   (uint32_t)bytes_sub((v.y >> sh) & 0x0F0F0F0Fu, 0x08080808u),
                                   (uint32_t)bytes_sub((v.z >> sh) & 0x0F0F0F0Fu, 0x08080808u),
                                   (uint32_t)bytes_sub((v.w >> sh) & 0x0F0F0F0Fu, 0x08080808u));
                }
            }
        }
        const int row = t >> 1, h = t & 1;
#pragma unroll
        for (int j = 0; j < 4; ++j) c.ws[4 * h + j][row] = f16_finite(r.w.d[j]);
    } else {
        const int row = t >> 1, h = t & 1;
        uint4 q[8];
        float ws[8], wm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        chunk_w_unpack<Q>(w, r.w, h, q, ws, wm);
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4 *>(c.a + row * kRowB + 128 * h + 16 * i) = q[i];
#pragma unroll
        for (int g = 0; g < F::NG; ++g) c.ws[F::NG * h + g][row] = ws[g];
        if constexpr (F::MINS)
#pragma unroll
            for (int g = 0; g < 4; ++g) c.wm[4 * h + g][row] = wm[g];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4 *>(c.b + (16 * i + (t >> 4)) * kRowB + 16 * (t & 15)) = r.xq[i];
    const int tok = t >> 2, qq = t & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        c.xs[2 * qq + i][tok] = r.xs[i];
        if constexpr (F::MINS) c.xm[2 * qq + i][tok] = r.xm[i];
    }
}

template <int Q>
__global__ __launch_bounds__(256) void gemm_repacked_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y,
                                                            int r0, int r1) {
    using F = GemmFmt<Q>;
    __shared__ __align__(16) GemmChunk cs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave & 1, wmi = wave >> 1;  // wave tile: rows 64 * wn .., tokens 32 * wmi ..
    const int n0 = r0 + blockIdx.x * kTN, m0 = blockIdx.y * kTM;
    const int M = (int)a.m;
    const int steps = w.cols / 32;
    const int nchunks = (steps + 7) / 8;
    const int hl = lane >> 5, jl = lane & 31;
    const int tok = 32 * wmi + jl;

    float acc[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[nt][v] = 0.0f;

    ChunkRegs<Q> rg;
    chunk_load<Q>(rg, w, a, n0, r1, m0, M, 0);
    chunk_store<Q>(w, rg, cs);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) chunk_load<Q>(rg, w, a, n0, r1, m0, M, kc + 1);
        const int nst = min(8, steps - 8 * kc);
        for (int st = 0; st < nst; ++st) {
            const float xs = cs.xs[st][tok];
            const float xsum = F::MINS ? cs.xm[st][tok] : 0.0f;
#pragma unroll
            for (int gg = 0; gg < 32 / F::GK; ++gg) {
                v16i c[2];
                if constexpr (F::GK == 32) {
                    const v4i bq = *reinterpret_cast<const v4i *>(cs.b + tok * kRowB + 32 * st + 16 * hl);
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const v4i aq =
                            *reinterpret_cast<const v4i *>(cs.a + (64 * wn + 32 * nt + jl) * kRowB + 32 * st + 16 * hl);
                        c[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
                    }
                } else {
                    const long bq = *reinterpret_cast<const long *>(cs.b + tok * kRowB + 32 * st + 16 * gg + 8 * hl);
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const long aq = *reinterpret_cast<const long *>(cs.a + (64 * wn + 32 * nt + jl) * kRowB +
                                                                        32 * st + 16 * gg + 8 * hl);
                        c[nt] = __builtin_amdgcn_mfma_i32_32x32x16_i8(aq, bq, v16i{0}, 0, 0, 0);
                    }
                }
                // C layout: lane holds token column jl, weight rows 8 * (v / 4) + 4 * hl + v % 4
                const int g = (32 / F::GK) * st + gg;
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int rl = 64 * wn + 32 * nt + 8 * q + 4 * hl;
                        const float4 ws4 = *reinterpret_cast<const float4 *>(&cs.ws[g][rl]);
                        float4 wm4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        if constexpr (F::MINS) wm4 = *reinterpret_cast<const float4 *>(&cs.wm[st][rl]);
                        const float wsv[4] = {ws4.x, ws4.y, ws4.z, ws4.w}, wmv[4] = {wm4.x, wm4.y, wm4.z, wm4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float t = (float)c[nt][4 * q + e] * (xs * wsv[e]);
                            if constexpr (F::MINS) acc[nt][4 * q + e] += t - xsum * wmv[e];
                            else acc[nt][4 * q + e] += t;
                        }
                    }
            }
        }
        if (more) {
            __syncthreads();
            chunk_store<Q>(w, rg, cs);
            __syncthreads();
        }
    }

    const int m = m0 + tok;
    if (m < M) {
        const size_t ld = (size_t)(r1 - r0);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int n = n0 + 64 * wn + 32 * nt + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (n < r1) y[(size_t)m * ld + (size_t)(n - r0)] = acc[nt][v];
            }
    }
}

jk_status launch_gemm_repacked(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    const dim3 grid((unsigned)((r1 - r0 + kTN - 1) / kTN), (unsigned)((a.m + kTM - 1) / kTM)), block(256);
    switch (w.quant) {
    case JK_Q8_0: hipLaunchKernelGGL(gemm_repacked_kernel<JK_Q8_0>, grid, block, 0, s, w, a, y, r0, r1); break;
    case JK_Q4_0: hipLaunchKernelGGL(gemm_repacked_kernel<JK_Q4_0>, grid, block, 0, s, w, a, y, r0, r1); break;
    case JK_Q4_K: hipLaunchKernelGGL(gemm_repacked_kernel<JK_Q4_K>, grid, block, 0, s, w, a, y, r0, r1); break;
    case JK_Q6_K: hipLaunchKernelGGL(gemm_repacked_kernel<JK_Q6_K>, grid, block, 0, s, w, a, y, r0, r1); break;
    case JK_TQ2_0: hipLaunchKernelGGL(gemm_repacked_kernel<JK_TQ2_0>, grid, block, 0, s, w, a, y, r0, r1); break;
    case JK_I2_S: hipLaunchKernelGGL(gemm_repacked_kernel<JK_I2_S>, grid, block, 0, s, w, a, y, r0, r1); break;
    default: return fail(JK_CAPABILITY_MISMATCH, "gemm: unsupported quant %d", w.quant);
    }
    return check_launch("gemm_repacked_kernel");
}

}  // namespace jk
