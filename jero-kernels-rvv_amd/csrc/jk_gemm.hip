// jk_gemm.hip -- prefill GEMM on int8 MFMA for the repacked (block-scaled i8) model.
//
// out[m][n] = sum over scale groups g, in order, starting from 0.0:
//     acc += f32(sum_k xq[m][k] * wq[n][k]) * (xs[m][b32(g)] * ws[n][g])  [- xsum * wm]
// (execute_gemm_repacked_rows, repack.rs:2718-3042, accumulate_scaled_tile_scalar
// 3045-3093). One MFMA covers exactly one scale group (32 elements with
// v_mfma_i32_32x32x32_i8, 16 with v_mfma_i32_32x32x16_i8 for Q6_K), so the integer
// partial of every group is exact and the f32 epilogue runs per group in K order:
// each output keeps the reference's arithmetic and order, bit for bit.
//
// Tiling: a 256-lane workgroup computes a 64 (M) x 64 (N) output tile as 2 x 2 waves of
// 32 x 32. Weight fragments are unpacked from the plane layout straight into MFMA
// operand registers; activation scales of a K stage are staged through LDS.
#include "jk_device.hpp"

namespace jk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Scale-group geometry of the repacked layout (BlockScaledTileLayout, repack.rs:1334-1366).
template <int Q> struct GemmFmt {
    static constexpr int GK = Q == JK_Q6_K ? 16 : 32;  // elements per scale group
    static constexpr bool MINS = Q == JK_Q4_K;
};

// B operand of one lane for group g and k-half h: 16 (GK 32) or 8 (GK 16) weights of row n as
// i8, plus the group's weight scale ws and min wm (repack_block_scaled_range_into_i8,
// repack.rs:1724-2103, per format).
template <int Q>
__device__ __forceinline__ void load_b(const WeightDev &w, int n, int g, int h, v4i &bq, long &bq8, float &ws,
                                       float &wm) {
    if constexpr (Q == JK_Q8_0) {
        const uint4 v = ld_chunk(w, h, n, g);
        bq = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        ws = ld_dscale(w, n, g);
    } else if constexpr (Q == JK_Q4_0) {
        const uint4 v = ld_chunk(w, 0, n, g);
        const int sh = 4 * h;
        bq = v4i{bytes_sub((v.x >> sh) & 0x0F0F0F0Fu, 0x08080808u), bytes_sub((v.y >> sh) & 0x0F0F0F0Fu, 0x08080808u),
                 bytes_sub((v.z >> sh) & 0x0F0F0F0Fu, 0x08080808u), bytes_sub((v.w >> sh) & 0x0F0F0F0Fu, 0x08080808u)};
        ws = ld_dscale(w, n, g);
    } else if constexpr (Q == JK_Q4_K) {
        const int b = g >> 3, s = g & 7, c = s >> 1;
        const uint4 hd = ld_chunk(w, 0, n, b);
        const uint4 v = ld_chunk(w, 1 + 2 * c + h, n, b);
        const int sh = 4 * (s & 1);
        bq = v4i{(int)((v.x >> sh) & 0x0F0F0F0Fu), (int)((v.y >> sh) & 0x0F0F0F0Fu), (int)((v.z >> sh) & 0x0F0F0F0Fu),
                 (int)((v.w >> sh) & 0x0F0F0F0Fu)};
        const float d = f16_finite(hd.x & 0xFFFFu), dmin = f16_finite(hd.x >> 16);
        // unpack_k4_scales_mins (repack.rs:1158-1170) for sub-block s
        const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, m_lo = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        const uint32_t scv = s < 4 ? sc_lo : sc_hi, mv = s < 4 ? m_lo : m_hi;
        ws = d * (float)((scv >> (8 * (s & 3))) & 255u);
        wm = dmin * (float)((mv >> (8 * (s & 3))) & 255u);
    } else if constexpr (Q == JK_Q6_K) {
        const int b = g >> 4, j = g & 15;
        const int h6 = j >> 3, quarter = (j & 7) >> 1, is = j & 1;
        const int l0 = 16 * is + 8 * h;  // first of this lane's 8 elements inside the 32-run
        const int lbyte = 64 * h6 + l0 + ((quarter & 1) ? 32 : 0), qbyte = 32 * h6 + l0;
        const uint4 lv = ld_chunk(w, lbyte >> 4, n, b), qv = ld_chunk(w, 8 + (qbyte >> 4), n, b);
        const int li = (lbyte & 15) >> 2, qi = (qbyte & 15) >> 2;
        uint32_t L[2] = {li == 0 ? lv.x : li == 2 ? lv.z : lv.x, li == 0 ? lv.y : li == 2 ? lv.w : lv.y};
        uint32_t H[2] = {qi == 0 ? qv.x : qi == 2 ? qv.z : qv.x, qi == 0 ? qv.y : qi == 2 ? qv.w : qv.y};
        const int lsh = quarter < 2 ? 0 : 4, hsh = 2 * quarter;
        int q2[2];
        for (int i = 0; i < 2; ++i) {
            const uint32_t v6 = ((L[i] >> lsh) & 0x0F0F0F0Fu) | (((H[i] >> hsh) & 0x03030303u) << 4);
            q2[i] = bytes_sub(v6, 0x20202020u);
        }
        bq8 = (long)(((unsigned long)(uint32_t)q2[1] << 32) | (uint32_t)q2[0]);
        const uint4 scv = ld_chunk(w, 12, n, b);
        const uint32_t sd = j < 4 ? scv.x : j < 8 ? scv.y : j < 12 ? scv.z : scv.w;
        ws = ld_dscale(w, n, b) * (float)(int8_t)(sd >> (8 * (j & 3)));
    } else if constexpr (Q == JK_TQ2_0) {
        const int b = g >> 3, s = g & 7, k = 2 * s + h;
        const uint4 v = ld_chunk(w, k >> 2, n, b);
        const uint32_t wv = (k & 3) == 0 ? v.x : (k & 3) == 1 ? v.y : (k & 3) == 2 ? v.z : v.w;
        bq = v4i{bytes_sub(wv & 0x03030303u, 0x01010101u), bytes_sub((wv >> 2) & 0x03030303u, 0x01010101u),
                 bytes_sub((wv >> 4) & 0x03030303u, 0x01010101u), bytes_sub((wv >> 6) & 0x03030303u, 0x01010101u)};
        ws = ld_dscale(w, n, b);
    } else if constexpr (Q == JK_I2_S) {
        const int b = g >> 2, s = g & 3, sh = 6 - 2 * s;
        const uint4 v = ld_chunk(w, h, n, b);
        bq = v4i{bytes_sub((v.x >> sh) & 0x03030303u, 0x01010101u), bytes_sub((v.y >> sh) & 0x03030303u, 0x01010101u),
                 bytes_sub((v.z >> sh) & 0x03030303u, 0x01010101u), bytes_sub((v.w >> sh) & 0x03030303u, 0x01010101u)};
        ws = w.tensor_scale;
    }
}

constexpr int kStageGroups = 8;  // scale groups per LDS stage of activation scales

template <int Q>
__global__ __launch_bounds__(256) void gemm_repacked_kernel(WeightDev w, jk_act_q8 a, float *__restrict__ y,
                                                            int r0, int r1) {
    using F = GemmFmt<Q>;
    __shared__ float s_xs[kStageGroups][64];
    __shared__ float s_xm[F::MINS ? kStageGroups : 1][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm_i = wave & 1, wn_i = wave >> 1;
    const int m_base = blockIdx.y * 64, n_base = r0 + blockIdx.x * 64;
    const int M = (int)a.m;
    const int h = lane >> 5;
    // operand rows of this lane (clamped for loads; masked on store)
    const int am = min(m_base + 32 * wm_i + (lane & 31), M - 1);
    const int bn = min(n_base + 32 * wn_i + (lane & 31), r1 - 1);
    const int ngroups = (w.cols + F::GK - 1) / F::GK;
    float acc[16];
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    const int8_t *arow = a.qs + (size_t)am * a.k_padded;
    for (int g0 = 0; g0 < ngroups; g0 += kStageGroups) {
        __syncthreads();
        // stage xs (and x sums) for 64 rows x kStageGroups groups; element (g, row) at [g][row]
        for (int idx = threadIdx.x; idx < kStageGroups * 64; idx += 256) {
            const int gg = idx >> 6, row = idx & 63;
            const int g = g0 + gg;
            const int mrow = min(m_base + row, M - 1);
            float xs = 0.0f, xm = 0.0f;
            if (g < ngroups) {
                const int b32 = F::GK == 32 ? g : g >> 1;
                xs = a.scales[(size_t)mrow * a.k_blocks32 + b32];
                if constexpr (F::MINS) xm = a.sums[(size_t)mrow * a.k_blocks32 + b32];
            }
            s_xs[gg][row] = xs;
            if constexpr (F::MINS) s_xm[gg][row] = xm;
        }
        __syncthreads();
        const int gend = min(kStageGroups, ngroups - g0);
        for (int gg = 0; gg < gend; ++gg) {
            const int g = g0 + gg;
            v16i c;
            float ws = 0.0f, wmn = 0.0f;
            if constexpr (F::GK == 32) {
                const uint4 av = *reinterpret_cast<const uint4 *>(arow + 32 * g + 16 * h);
                const v4i aq = v4i{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                v4i bq;
                long unused;
                load_b<Q>(w, bn, g, h, bq, unused, ws, wmn);
                c = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq, v16i{0}, 0, 0, 0);
            } else {
                const long aq = *reinterpret_cast<const long *>(arow + 16 * g + 8 * h);
                v4i unused;
                long bq;
                load_b<Q>(w, bn, g, h, unused, bq, ws, wmn);
                c = __builtin_amdgcn_mfma_i32_32x32x16_i8(aq, bq, v16i{0}, 0, 0, 0);
            }
            // C layout: lane holds column n = lane % 32, rows 8 * (i / 4) + 4 * h + i % 4
            for (int i = 0; i < 16; ++i) {
                const int ml = 32 * wm_i + 8 * (i >> 2) + 4 * h + (i & 3);
                const float t = (float)c[i] * (s_xs[gg][ml] * ws);
                if constexpr (F::MINS) acc[i] += t - s_xm[gg][ml] * wmn;
                else acc[i] += t;
            }
        }
    }
    const int n = n_base + 32 * wn_i + (lane & 31);
    if (n < r1) {
        const size_t sub = (size_t)(r1 - r0);
        for (int i = 0; i < 16; ++i) {
            const int m = m_base + 32 * wm_i + 8 * (i >> 2) + 4 * h + (i & 3);
            if (m < M) y[(size_t)m * sub + (size_t)(n - r0)] = acc[i];
        }
    }
}

jk_status launch_gemm_repacked(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1) {
    const dim3 grid((unsigned)((r1 - r0 + 63) / 64), (unsigned)((a.m + 63) / 64)), block(256);
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
