// jk_repack.hip -- GGUF -> plane layout on the device, and row dequantization from it.
#include "jk_device.hpp"

namespace jk {

// 4x4 transpose of the 2-bit fields of one TQ2_0 dword (see jk_internal.hpp).
__device__ __forceinline__ uint32_t tq2_transpose(uint32_t v) {
    uint32_t o = 0;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) {
            uint32_t t = (v >> (8 * j + 2 * i)) & 3u;  // element 4j+i of the GGUF dword
            o |= t << (8 * i + 2 * j);                  // byte i, field j
        }
    return o;
}

__device__ __forceinline__ uint32_t le32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Dword k (0..63) of the TQ2_0 payload that holds the trits of a TQ1_0 block: byte i of
// the payload holds elements 4i..4i+3 as t + 1 in bits 2j. The TQ1_0 trits are the
// base-3 digits of its bytes 2..52 (element 5i + j = digit j of byte 2 + i, least
// significant first) and the lowest digit of byte 53 (element 255), as in
// unpack_tq1_0_block_i8 (ime.rs:595-632).
__device__ uint32_t tq1_as_tq2_dword(const uint8_t *src, int k) {
    uint32_t out = 0;
    for (int e4 = 0; e4 < 16; ++e4) {
        const int e = 16 * k + e4;  // element; bits 2 * e4 of the dword
        unsigned v;
        if (e < 255) {
            v = src[2 + e / 5];
            for (int j = e % 5; j > 0; --j) v /= 3u;
        } else {
            v = src[53];
        }
        out |= (v % 3u) << (2 * e4);
    }
    return out;
}

// One thread per (row, block): cut the GGUF block into its 16-byte chunks, scale and
// word (TQ1_0: re-encoded as the TQ2_0 payload first). The stores are the only writes of
// the planes; the weight handle is read-only after.
// One thread per GGUF block of rows [r0, r0 + nrows); g holds exactly those rows' GGUF bytes.
__global__ __launch_bounds__(256) void repack_kernel(WeightDev w, int gq, const uint8_t *__restrict__ g, int r0,
                                                     int nrows) {
    const size_t li = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (li >= (size_t)nrows * (size_t)w.nb) return;
    const Fmt f = fmt_of(w.quant);    // device layout
    const Fmt fg = fmt_of(gq);        // GGUF block
    const uint8_t *src = g + li * (size_t)fg.bb;
    const int r = r0 + (int)(li / (size_t)w.nb), b = (int)(li % (size_t)w.nb);
    const size_t idx = (size_t)r * (size_t)w.nb + (size_t)b;
    for (int c = 0; c < f.chunks; ++c) {
        uint32_t d4[4];
        for (int k = 0; k < 4; ++k) {
            const int off = f.q_off + 16 * c + 4 * k;
            if (gq == JK_TQ1_0) d4[k] = tq1_as_tq2_dword(src, 4 * c + k);
            else if (off + 4 <= fg.bb) d4[k] = le32(src + off);
            else {  // the last chunk of a Q3_K block: bytes past the block are zero padding
                d4[k] = 0;
                for (int i = 0; off + i < fg.bb; ++i) d4[k] |= (uint32_t)src[off + i] << (8 * i);
            }
            if (f.quant == JK_TQ2_0) d4[k] = tq2_transpose(d4[k]);
        }
        uint4 *dst = const_cast<uint4 *>(chunk_ptr(w, c, r, b));
        *dst = make_uint4(d4[0], d4[1], d4[2], d4[3]);
    }
    if (f.d_off >= 0) {  // TQ1_0 and TQ2_0 both hold d at byte 0
        uint16_t h = (uint16_t)(src[f.d_off] | (src[f.d_off + 1] << 8));
        const_cast<uint16_t *>(w.dplane)[idx] = h;
    }
    for (int i = 0; f.h_off >= 0 && i < f.h_len / 4; ++i)
        const_cast<uint32_t *>(w.hplane)[idx * (size_t)(f.h_len / 4) + i] = le32(src + f.h_off + 4 * i);
}

jk_status launch_repack(hipStream_t s, const WeightDev &w, int gguf_quant, const uint8_t *gguf, int r0, int r1) {
    if (r1 <= r0) return JK_OK;
    const size_t total = (size_t)(r1 - r0) * (size_t)w.nb;
    const unsigned grid = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(repack_kernel, dim3(grid), dim3(256), 0, s, w, gguf_quant, gguf, r0, r1 - r0);
    return check_launch("repack_kernel");
}

__device__ __forceinline__ uint8_t chunk_byte(const uint4 &v, int i) {
    const uint32_t d = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (uint8_t)(d >> (8 * (i & 3)));
}

// Dequantizes block b of row r into out[0..be) with the GGUF block dequantizers' arithmetic:
// dequantize_q4_0_block (quant.rs:550-568), dequantize_q5_0_block (160-164), the Q4_1, Q5_1,
// IQ4_NL, Q2_K and Q3_K block dequantizers (132-356),
// dequantize_q8_0_block (571-588), dequantize_q4_k_m_block (lib.rs:720-766),
// dequantize_q5_k_block (quant.rs:651-706), dequantize_q6_k_block (594-648), the TQ1_0
// and TQ2_0 arms (2359-2378; one device layout) and dequantize_i2_s_block (380-387).
__device__ void dequant_block(const WeightDev &w, int r, int b, float *out) {
    switch (w.quant) {
    case JK_Q4_0: {
        const float d = ld_dscale(w, r, b);
        const uint4 q = ld_chunk(w, 0, r, b);
        for (int i = 0; i < 16; ++i) {
            const uint8_t x = chunk_byte(q, i);
            out[i] = d == 0.0f ? 0.0f : d * (float)((int)(x & 15) - 8);
            out[i + 16] = d == 0.0f ? 0.0f : d * (float)((int)(x >> 4) - 8);
        }
        break;
    }
    case JK_Q5_0: {  // dequantize_q5_0_block (quant.rs:160-164) via unpack_q5_0_block_i8 (139-157)
        const float d = ld_dscale(w, r, b);
        const uint4 q = ld_chunk(w, 0, r, b);
        const uint32_t qh = w.hplane[(size_t)r * (size_t)w.nb + (size_t)b];
        for (int i = 0; i < 16; ++i) {
            const uint8_t x = chunk_byte(q, i);
            const int q0 = (int)((x & 15) | (((qh >> i) & 1u) << 4)) - 16;
            const int q1 = (int)((x >> 4) | (((qh >> (i + 16)) & 1u) << 4)) - 16;
            out[i] = d == 0.0f ? 0.0f : d * (float)q0;
            out[i + 16] = d == 0.0f ? 0.0f : d * (float)q1;
        }
        break;
    }
    case JK_Q4_1:
    case JK_Q5_1: {  // dequantize_q4_1_block / dequantize_q5_1_block (quant.rs:132-136, 190-195):
                     // affine_i8_into_f32 (104-113), both zero -> +0.0, else d * q + m
        const int hl = w.quant == JK_Q4_1 ? 4 : 8;
        const uint32_t dm = ld_word(w, r, b, hl, 0), qh = hl == 8 ? ld_word(w, r, b, hl, 1) : 0u;
        const float d = f16_finite(dm & 0xFFFFu), m = f16_finite(dm >> 16);
        const uint4 q = ld_chunk(w, 0, r, b);
        for (int i = 0; i < 16; ++i) {
            const uint8_t x = chunk_byte(q, i);
            const int q0 = (int)((x & 15) | (((qh >> i) & 1u) << 4));
            const int q1 = (int)((x >> 4) | (((qh >> (i + 16)) & 1u) << 4));
            const bool z = d == 0.0f && m == 0.0f;
            out[i] = z ? 0.0f : d * (float)q0 + m;
            out[i + 16] = z ? 0.0f : d * (float)q1 + m;
        }
        break;
    }
    case JK_IQ4_NL: {  // dequantize_iq4_nl_block (quant.rs:348-356)
        const float d = ld_dscale(w, r, b);
        const uint4 q = ld_chunk(w, 0, r, b);
        for (int i = 0; i < 16; ++i) {
            const uint8_t x = chunk_byte(q, i);
            const int v0 = (int)(int8_t)(iq4nl_lookup(x & 15u) & 255u), v1 = (int)(int8_t)(iq4nl_lookup(x >> 4) & 255u);
            out[i] = d == 0.0f ? 0.0f : d * (float)v0;
            out[i + 16] = d == 0.0f ? 0.0f : d * (float)v1;
        }
        break;
    }
    case JK_Q2_K: {  // dequantize_q2_k_block (quant.rs:238-252) with unpack_q2_k_block_i8 (197-235)
        const uint32_t dd = ld_word(w, r, b, 4, 0);
        const float d = f16_finite(dd & 0xFFFFu), dmin = f16_finite(dd >> 16);
        const uint4 scv = ld_chunk(w, 0, r, b);
        for (int e = 0; e < 256; ++e) {
            const int half = e >> 7, j = (e >> 5) & 3, part = (e >> 4) & 1, l = e & 15;
            const int is = e >> 4;
            const uint8_t sc = chunk_byte(scv, is);
            const float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
            const int qb = 32 * half + 16 * part + l;  // byte of qs (chunks 1..4)
            const int qv = (chunk_byte(ld_chunk(w, 1 + (qb >> 4), r, b), qb & 15) >> (2 * j)) & 3;
            out[e] = dl * (float)qv - ml;
        }
        break;
    }
    case JK_Q3_K: {  // dequantize_q3_k_block (quant.rs:320-331) with unpack_q3_k_block_i8 (254-317)
        const uint4 tail = ld_chunk(w, 6, r, b);  // 12 scale bytes, d, padding
        const float d = f16_finite(tail.w & 0xFFFFu);
        for (int e = 0; e < 256; ++e) {
            const int half = e >> 7, j = (e >> 5) & 3, part = (e >> 4) & 1, l = e & 15;
            const int is = e >> 4;
            const int lo = is < 8 ? (chunk_byte(tail, is) & 15) : (chunk_byte(tail, is - 8) >> 4);
            const int hi = (chunk_byte(tail, 8 + (is & 3)) >> (2 * (is >> 2))) & 3;
            const float dl = d * (float)((lo | (hi << 4)) - 32);
            const int qb = 32 * half + 16 * part + l, hb = 16 * part + l;
            const int v = (chunk_byte(ld_chunk(w, 2 + (qb >> 4), r, b), qb & 15) >> (2 * j)) & 3;
            const int h = (chunk_byte(ld_chunk(w, hb >> 4, r, b), hb & 15) >> (4 * half + j)) & 1;
            out[e] = dl * (float)(v - (h ? 0 : 4));
        }
        break;
    }
    case JK_Q8_0: {
        const float d = ld_dscale(w, r, b);
        for (int c = 0; c < 2; ++c) {
            const uint4 q = ld_chunk(w, c, r, b);
            for (int i = 0; i < 16; ++i) out[16 * c + i] = d == 0.0f ? 0.0f : d * (float)(int8_t)chunk_byte(q, i);
        }
        break;
    }
    case JK_Q4_K: {
        const uint4 h = ld_chunk(w, 0, r, b);
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        uint8_t s[12], sc[8], m[8];
        for (int i = 0; i < 12; ++i) s[i] = chunk_byte(h, 4 + i);
        for (int j = 0; j < 4; ++j) { sc[j] = s[j] & 63; m[j] = s[j + 4] & 63; }
        for (int j = 4; j < 8; ++j) {
            sc[j] = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
            m[j] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
        for (int c = 0; c < 4; ++c) {
            const float d1 = d * (float)sc[2 * c], m1 = dmin * (float)m[2 * c];
            const float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)m[2 * c + 1];
            for (int half = 0; half < 2; ++half) {
                const uint4 q = ld_chunk(w, 1 + 2 * c + half, r, b);
                for (int i = 0; i < 16; ++i) {
                    const uint8_t x = chunk_byte(q, i);
                    const int l = 16 * half + i;
                    out[64 * c + l] = d1 * (float)(x & 15) - m1;
                    out[64 * c + 32 + l] = d2 * (float)(x >> 4) - m2;
                }
            }
        }
        break;
    }
    case JK_Q5_K: {  // dequantize_q5_k_block (quant.rs:651-706)
        const uint4 h = ld_chunk(w, 0, r, b);
        const float d = f16_finite(h.x & 0xFFFFu), dmin = f16_finite(h.x >> 16);
        if (d == 0.0f && dmin == 0.0f) {
            for (int i = 0; i < 256; ++i) out[i] = 0.0f;
            break;
        }
        uint8_t s[12], sc[8], m[8];
        for (int i = 0; i < 12; ++i) s[i] = chunk_byte(h, 4 + i);
        for (int j = 0; j < 4; ++j) { sc[j] = s[j] & 63; m[j] = s[j + 4] & 63; }
        for (int j = 4; j < 8; ++j) {
            sc[j] = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
            m[j] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
        const uint4 qh[2] = {ld_chunk(w, 1, r, b), ld_chunk(w, 2, r, b)};
        for (int c = 0; c < 4; ++c) {
            const float d1 = d * (float)sc[2 * c], m1 = dmin * (float)m[2 * c];
            const float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)m[2 * c + 1];
            for (int half = 0; half < 2; ++half) {
                const uint4 q = ld_chunk(w, 3 + 2 * c + half, r, b);
                for (int i = 0; i < 16; ++i) {
                    const uint8_t x = chunk_byte(q, i), hb = chunk_byte(qh[half], i);
                    const int l = 16 * half + i;
                    out[64 * c + l] = d1 * (float)((x & 15) + ((hb >> (2 * c)) & 1) * 16) - m1;
                    out[64 * c + 32 + l] = d2 * (float)((x >> 4) + ((hb >> (2 * c + 1)) & 1) * 16) - m2;
                }
            }
        }
        break;
    }
    case JK_Q6_K: {
        const float d = ld_dscale(w, r, b);
        if (d == 0.0f) {
            for (int i = 0; i < 256; ++i) out[i] = 0.0f;
            break;
        }
        const uint4 scv = ld_chunk(w, 12, r, b);
        for (int h = 0; h < 2; ++h) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int li = 64 * h + l, hi = 64 * h + l + 32, qi = 32 * h + l;
                const uint8_t L = chunk_byte(ld_chunk(w, li / 16, r, b), li % 16);
                const uint8_t H = chunk_byte(ld_chunk(w, hi / 16, r, b), hi % 16);
                const uint8_t Q = chunk_byte(ld_chunk(w, 8 + qi / 16, r, b), qi % 16);
                const int q1 = (int)((L & 15) | ((Q & 3) << 4)) - 32;
                const int q2 = (int)((H & 15) | (((Q >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((L >> 4) | (((Q >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((H >> 4) | (((Q >> 6) & 3) << 4)) - 32;
                const int sb = 8 * h + is;
                out[128 * h + l] = d * (float)(int8_t)chunk_byte(scv, sb) * (float)q1;
                out[128 * h + l + 32] = d * (float)(int8_t)chunk_byte(scv, sb + 2) * (float)q2;
                out[128 * h + l + 64] = d * (float)(int8_t)chunk_byte(scv, sb + 4) * (float)q3;
                out[128 * h + l + 96] = d * (float)(int8_t)chunk_byte(scv, sb + 6) * (float)q4;
            }
        }
        break;
    }
    case JK_TQ2_0: {
        const float d = ld_dscale(w, r, b);
        for (int c = 0; c < 4; ++c) {
            const uint4 q = ld_chunk(w, c, r, b);
            const uint32_t dw[4] = {q.x, q.y, q.z, q.w};
            for (int k = 0; k < 4; ++k)
                for (int p = 0; p < 16; ++p) {  // element p of the dword: byte p%4, field p/4
                    const int t = (int)((dw[k] >> (8 * (p & 3) + 2 * (p >> 2))) & 3u) - 1;
                    out[64 * c + 16 * k + p] = d == 0.0f ? 0.0f : d * (float)t;
                }
        }
        break;
    }
    case JK_I2_S: {
        const float sc = w.tensor_scale;
        for (int c = 0; c < 2; ++c) {
            const uint4 q = ld_chunk(w, c, r, b);
            for (int i = 0; i < 16; ++i) {
                const uint8_t x = chunk_byte(q, i);
                const int g = 16 * c + i;
                const int t0 = ((x >> 6) & 3) - 1, t1 = ((x >> 4) & 3) - 1, t2 = ((x >> 2) & 3) - 1, t3 = (x & 3) - 1;
                out[g] = sc == 0.0f ? 0.0f : sc * (float)t0;
                out[32 + g] = sc == 0.0f ? 0.0f : sc * (float)t1;
                out[64 + g] = sc == 0.0f ? 0.0f : sc * (float)t2;
                out[96 + g] = sc == 0.0f ? 0.0f : sc * (float)t3;
            }
        }
        break;
    }
    default: break;
    }
}

// convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790) over n output blocks: TQ2_0 block k from I2_S
// blocks 2k and 2k + 1. One thread per output dword: dword j (j < 16) of the 64-byte payload
// holds elements 16j..16j+15, which lie in I2_S block (16j) / 128 at positions p..p+15 (p a
// multiple of 16), i.e. group g = p % 32 .. +15 of field (p / 32); the thread assembles them
// from the 16 source bytes g.. with the field's shift. Thread 16 of each block writes d.
__global__ __launch_bounds__(256) void i2s_to_tq2_kernel(const uint8_t *__restrict__ i2s, size_t n,
                                                         uint16_t d_bits, uint8_t *__restrict__ tq2) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t k = t / 17;
    const int j = (int)(t % 17);
    if (k >= n) return;
    uint8_t *dst = tq2 + k * 66;
    if (j == 16) {
        dst[0] = (uint8_t)(d_bits & 0xFF);
        dst[1] = (uint8_t)(d_bits >> 8);
        return;
    }
    const int e0 = 16 * j;                      // first element of the dword
    const uint8_t *blk = i2s + (2 * k + (size_t)(e0 / 128)) * 32;
    const int pos = e0 % 128, field = pos / 32, g0 = pos % 32;
    const int shift = 6 - 2 * field;            // unpack_i2_s_block_i8: t[32f + g] = (b[g] >> (6 - 2f)) & 3
    for (int i = 0; i < 4; ++i) {
        uint32_t byte = 0;
        for (int q = 0; q < 4; ++q) byte |= (((uint32_t)blk[g0 + 4 * i + q] >> shift) & 3u) << (2 * q);
        dst[2 + 4 * j + i] = (uint8_t)byte;     // the stored field is t + 1 = the I2_S field
    }
}

jk_status launch_i2s_to_tq2(hipStream_t s, const uint8_t *i2s, size_t n, uint16_t d_bits, uint8_t *tq2) {
    const size_t threads = n * 17;
    hipLaunchKernelGGL(i2s_to_tq2_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, i2s, n, d_bits, tq2);
    return check_launch("i2s_to_tq2_kernel");
}

__global__ __launch_bounds__(256) void dequant_rows_kernel(WeightDev w, int r0, int r1, float *__restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(r1 - r0) * (size_t)w.nb;
    if (idx >= total) return;
    const int r = r0 + (int)(idx / (size_t)w.nb), b = (int)(idx % (size_t)w.nb);
    const Fmt f = fmt_of(w.quant);
    // (straight into the output row: a per-thread staging array of a block's values lived in scratch)
    dequant_block(w, r, b, out + (size_t)(r - r0) * (size_t)w.cols + (size_t)b * f.be);
}

jk_status launch_dequant_rows(hipStream_t s, const WeightDev &w, int r0, int r1, float *out) {
    const size_t total = (size_t)(r1 - r0) * (size_t)w.nb;
    hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, w, r0, r1, out);
    return check_launch("dequant_rows_kernel");
}

}  // namespace jk
