/*
 * jk_oracle.c -- CPU restatement of the jero-kernels-rvv portable scalar fallback
 * for the quantized-matmul path. TEST INFRASTRUCTURE ONLY: the oracle of the parity
 * tests and the timed CPU baseline; never part of the product library.
 *
 * Citations are file:line in the reference crate (src/...). Build with
 * -ffp-contract=off so that every `a * b + c` of the reference rounds twice.
 */
#include "jk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Format tables: quant.rs:19-91, ime.rs:27-37, lib.rs:128-132                */
/* ------------------------------------------------------------------------- */
size_t or_block_elements(int q) {
    switch (q) {
    case OR_Q4_0: case OR_Q8_0: case OR_Q5_0: case OR_Q4_1: case OR_Q5_1: case OR_IQ4_NL: return 32;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_TQ1_0: case OR_TQ2_0: case OR_Q2_K: case OR_Q3_K: return 256;
    case OR_I2_S: return 128;
    default: return 0;
    }
}

size_t or_block_bytes(int q) {
    switch (q) {
    case OR_Q4_0: return 18;
    case OR_Q4_1: return 20;
    case OR_Q5_0: return 22;
    case OR_Q5_1: return 24;
    case OR_IQ4_NL: return 18;
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_TQ1_0: return 54;
    case OR_Q6_K: return 210;
    case OR_TQ2_0: return 66;
    case OR_I2_S: return 32;
    default: return 0;
    }
}

/* I2_S carries a 32-byte tensor-wide scale trailer (quant.rs:89-91). */
size_t or_scale_trailer_bytes(int q) { return q == OR_I2_S ? 32 : 0; }

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Rust `sum: f32 = iter.sum()` folds from -0.0; `let mut acc = 0.0` starts at +0.0. */
static float neg_zero(void) { return -0.0f; }

/* Rust `x.round().clamp(lo, hi) as i8`: NaN clamps to NaN and `NaN as i8` is 0. */
static int8_t rust_round_clamp_i8(float v, float lo, float hi) {
    float r = roundf(v);
    if (isnan(r)) return 0;
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------- */
/* f16 decode: lib.rs:676-717                                                 */
/* ------------------------------------------------------------------------- */
float or_f16_to_f32_ieee(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, mant = bits & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (mant == 0) {
            out = sign << 31;
        } else {
            uint32_t m = mant, e = 127u - 14u;
            while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
            m &= 0x3FFu;
            out = (sign << 31) | (e << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        out = mant == 0 ? ((sign << 31) | 0x7F800000u) : ((sign << 31) | 0x7FC00000u | (mant << 13));
    } else {
        out = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

float or_f16_to_f32_finite(uint16_t bits) {
    float v = or_f16_to_f32_ieee(bits);
    return isfinite(v) ? v : 0.0f;
}

/* ------------------------------------------------------------------------- */
/* Block dequantization                                                       */
/* ------------------------------------------------------------------------- */

/* quant.rs:550-568 */
void or_dequantize_q4_0_block(const uint8_t *blk, float *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    if (d == 0.0f) { for (int i = 0; i < 32; i++) out[i] = 0.0f; return; }
    for (int i = 0; i < 16; i++) {
        uint8_t b = blk[2 + i];
        out[i] = d * (float)((int)(b & 0x0F) - 8);
        out[i + 16] = d * (float)((int)((b >> 4) & 0x0F) - 8);
    }
}

/* quant.rs:571-588 */
void or_dequantize_q8_0_block(const uint8_t *blk, float *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    if (d == 0.0f) { for (int i = 0; i < 32; i++) out[i] = 0.0f; return; }
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)blk[2 + i];
}

/* quant_q8.rs:1818-1830 (same table as lib.rs:736-745 and repack.rs:1158-1170) */
static void unpack_k4_scales_mins(const uint8_t *s, uint8_t sc[8], uint8_t m[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 0x3F;
        m[j] = s[j + 4] & 0x3F;
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        m[j] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* lib.rs:720-766 (no zero-scale short cut; d1*q - m1 rounds twice) */
void or_dequantize_q4_k_block(const uint8_t *blk, float *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    float dmin = or_f16_to_f32_finite(rd16(blk + 2));
    uint8_t sc[8], m[8];
    unpack_k4_scales_mins(blk + 4, sc, m);
    const uint8_t *qs = blk + 16;
    for (int c = 0; c < 4; c++) {
        float d1 = d * (float)sc[2 * c], m1 = dmin * (float)m[2 * c];
        float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)m[2 * c + 1];
        for (int l = 0; l < 32; l++) out[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0x0F) - m1;
        for (int l = 0; l < 32; l++) out[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
    }
}

/* quant.rs:594-648: out = (d * sc) * q evaluated left to right */
void or_dequantize_q6_k_block(const uint8_t *blk, float *out) {
    float d = or_f16_to_f32_finite(rd16(blk + 208));
    if (d == 0.0f) { for (int i = 0; i < 256; i++) out[i] = 0.0f; return; }
    const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
    for (int h = 0; h < 2; h++) {
        int n = 128 * h;
        const uint8_t *L = ql + 64 * h, *H = qh + 32 * h;
        const int8_t *S = (const int8_t *)(sc + 8 * h);
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((L[l] & 0x0F) | ((H[l] & 3) << 4)) - 32;
            int q2 = (int)((L[l + 32] & 0x0F) | (((H[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((L[l] >> 4) | (((H[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((L[l + 32] >> 4) | (((H[l] >> 6) & 3) << 4)) - 32;
            out[n + l] = d * (float)S[is] * (float)q1;
            out[n + l + 32] = d * (float)S[is + 2] * (float)q2;
            out[n + l + 64] = d * (float)S[is + 4] * (float)q3;
            out[n + l + 96] = d * (float)S[is + 6] * (float)q4;
        }
    }
}

/* quant.rs:139-157: q = (nibble | 16 * bit) - 16 with the 32 high bits in a little-endian
 * u32 at bytes 2..6 (bit j for element j, bit j + 16 for element j + 16). */
float or_unpack_q5_0_block_i8(const uint8_t *blk, int8_t *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
    for (int j = 0; j < 16; j++) {
        uint8_t b = blk[6 + j];
        int h0 = (int)((qh >> j) & 1u) << 4, h1 = (int)((qh >> (j + 16)) & 1u) << 4;
        out[j] = (int8_t)(((b & 0x0F) | h0) - 16);
        out[j + 16] = (int8_t)((((b >> 4) & 0x0F) | h1) - 16);
    }
    return d;
}

static void scale_i8_into_f32(float scale, const int8_t *q, float *out, int n);

/* quant.rs:160-164 */
void or_dequantize_q5_0_block(const uint8_t *blk, float *out) {
    int8_t q[32];
    float d = or_unpack_q5_0_block_i8(blk, q);
    scale_i8_into_f32(d, q, out, 32);
}

/* quant.rs:651-706: both scales zero -> all +0.0; else d1 * q - m1 per element (q up to 31) */
void or_dequantize_q5_k_block(const uint8_t *blk, float *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    float dmin = or_f16_to_f32_finite(rd16(blk + 2));
    if (d == 0.0f && dmin == 0.0f) { for (int i = 0; i < 256; i++) out[i] = 0.0f; return; }
    uint8_t sc[8], m[8];
    unpack_k4_scales_mins(blk + 4, sc, m);
    const uint8_t *qh = blk + 16, *qs = blk + 48;
    for (int c = 0; c < 4; c++) {
        float d1 = d * (float)sc[2 * c], m1 = dmin * (float)m[2 * c];
        float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)m[2 * c + 1];
        uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
        for (int l = 0; l < 32; l++) {
            uint8_t q1 = (uint8_t)((qs[32 * c + l] & 0x0F) + ((qh[l] & u1) ? 16 : 0));
            out[64 * c + l] = d1 * (float)q1 - m1;
        }
        for (int l = 0; l < 32; l++) {
            uint8_t q2 = (uint8_t)((qs[32 * c + l] >> 4) + ((qh[l] & u2) ? 16 : 0));
            out[64 * c + 32 + l] = d2 * (float)q2 - m2;
        }
    }
}

/* ime.rs:595-632 (the crate's TQ1_0 layout): d at bytes 0..2, then bytes 2..53 each carry
 * five base-3 digits, least significant first (element 5i + j = digit j of byte 2 + i),
 * and byte 53 carries element 255 as its lowest digit; trit t maps to t - 1. */
float or_unpack_tq1_0_block_i8(const uint8_t *blk, int8_t *out) {
    float s = or_f16_to_f32_finite(rd16(blk));
    for (int i = 0; i < 51; i++) {
        unsigned b = blk[2 + i];
        for (int j = 0; j < 5; j++) {
            out[5 * i + j] = (int8_t)((int)(b % 3u) - 1);
            b /= 3u;
        }
    }
    out[255] = (int8_t)((int)(blk[53] % 3u) - 1);
    return s;
}

/* quant.rs:117-129: quants are the nibbles (0..15), (d, m) returned */
static void unpack_q4_1_block_i8(const uint8_t *blk, int8_t *out, float *d, float *m) {
    *d = or_f16_to_f32_finite(rd16(blk));
    *m = or_f16_to_f32_finite(rd16(blk + 2));
    for (int i = 0; i < 16; i++) {
        out[i] = (int8_t)(blk[4 + i] & 0x0F);
        out[i + 16] = (int8_t)((blk[4 + i] >> 4) & 0x0F);
    }
}

/* quant.rs:168-187: quants 0..31 with the fifth bit from the u32 at bytes 4..8 */
static void unpack_q5_1_block_i8(const uint8_t *blk, int8_t *out, float *d, float *m) {
    *d = or_f16_to_f32_finite(rd16(blk));
    *m = or_f16_to_f32_finite(rd16(blk + 2));
    uint32_t qh = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) | ((uint32_t)blk[7] << 24);
    for (int j = 0; j < 16; j++) {
        uint8_t b = blk[8 + j];
        out[j] = (int8_t)((b & 0x0F) | (((qh >> j) & 1u) << 4));
        out[j + 16] = (int8_t)(((b >> 4) & 0x0F) | (((qh >> (j + 16)) & 1u) << 4));
    }
}

/* affine_i8_into_f32 (quant.rs:104-113): both zero -> +0.0, else d * q + m */
static void affine_i8_into_f32(float d, float m, const int8_t *q, float *out, int n) {
    if (d == 0.0f && m == 0.0f) { for (int i = 0; i < n; i++) out[i] = 0.0f; return; }
    for (int i = 0; i < n; i++) out[i] = d * (float)q[i] + m;
}

/* quant.rs:132-136 */
void or_dequantize_q4_1_block(const uint8_t *blk, float *out) {
    int8_t q[32];
    float d, m;
    unpack_q4_1_block_i8(blk, q, &d, &m);
    affine_i8_into_f32(d, m, q, out, 32);
}

/* quant.rs:190-195 */
void or_dequantize_q5_1_block(const uint8_t *blk, float *out) {
    int8_t q[32];
    float d, m;
    unpack_q5_1_block_i8(blk, q, &d, &m);
    affine_i8_into_f32(d, m, q, out, 32);
}

/* quant.rs:197-235: scales[16] at 0, qs[64] at 16, d at 80, dmin at 82. Sub-block is
 * (16 elements) has scale d * (sc & 15) and min dmin * (sc >> 4); its quants are the 2-bit
 * field 2j of qs[32 half + 16 (is % 2) + l] for is = 8 half + 2j + (is % 2). */
void or_unpack_q2_k_block_i8(const uint8_t *blk, int8_t *q, float *scales, float *mins) {
    const uint8_t *sc = blk, *qs = blk + 16;
    float d = or_f16_to_f32_finite(rd16(blk + 80)), dmin = or_f16_to_f32_finite(rd16(blk + 82));
    int is = 0;
    for (int half = 0; half < 2; half++)
        for (int j = 0; j < 4; j++)
            for (int part = 0; part < 2; part++, is++) {
                scales[is] = d * (float)(sc[is] & 0x0F);
                mins[is] = dmin * (float)(sc[is] >> 4);
                for (int l = 0; l < 16; l++)
                    q[128 * half + 32 * j + 16 * part + l] = (int8_t)((qs[32 * half + 16 * part + l] >> (2 * j)) & 3);
            }
}

/* quant.rs:238-252: dl * q - ml per 16-element sub-block */
void or_dequantize_q2_k_block(const uint8_t *blk, float *out) {
    int8_t q[256];
    float sc[16], mn[16];
    or_unpack_q2_k_block_i8(blk, q, sc, mn);
    for (int sb = 0; sb < 16; sb++)
        for (int l = 0; l < 16; l++) out[16 * sb + l] = sc[sb] * (float)q[16 * sb + l] - mn[sb];
}

/* quant.rs:254-317: hmask[32] at 0, qs[64] at 32, 12 packed 6-bit scales at 96, d at 108.
 * The 16 scales (6 bits, biased by 32) are the low nibbles of bytes 0..8 (scales 0..7) or
 * the high nibbles (8..15), with bits 4..5 from byte 8 + (is % 4) at shift 2 (is / 4). Quant
 * of element 128 half + 32 j + 16 part + l: 2-bit field 2j of qs[32 half + 16 part + l], minus
 * 4 when bit (4 half + j) of hmask[16 part + l] is clear. */
void or_unpack_q3_k_block_i8(const uint8_t *blk, int8_t *q, float *scales) {
    const uint8_t *hm = blk, *qs = blk + 32, *raw = blk + 96;
    float d = or_f16_to_f32_finite(rd16(blk + 108));
    for (int is = 0; is < 16; is++) {
        int lo = is < 8 ? (raw[is] & 0x0F) : (raw[is - 8] >> 4);
        int hi = (raw[8 + (is & 3)] >> (2 * (is >> 2))) & 3;
        scales[is] = d * (float)((int8_t)(lo | (hi << 4)) - 32);
    }
    for (int half = 0; half < 2; half++)
        for (int j = 0; j < 4; j++)
            for (int part = 0; part < 2; part++)
                for (int l = 0; l < 16; l++) {
                    int v = (qs[32 * half + 16 * part + l] >> (2 * j)) & 3;
                    int hb = (hm[16 * part + l] >> (4 * half + j)) & 1;
                    q[128 * half + 32 * j + 16 * part + l] = (int8_t)(v - (hb ? 0 : 4));
                }
}

/* quant.rs:320-331: dl * q */
void or_dequantize_q3_k_block(const uint8_t *blk, float *out) {
    int8_t q[256];
    float sc[16];
    or_unpack_q3_k_block_i8(blk, q, sc);
    for (int sb = 0; sb < 16; sb++)
        for (int l = 0; l < 16; l++) out[16 * sb + l] = sc[sb] * (float)q[16 * sb + l];
}

/* KVALUES_IQ4NL (quant.rs:76-78) */
static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* quant.rs:333-345 */
float or_unpack_iq4_nl_block_i8(const uint8_t *blk, int8_t *out) {
    float d = or_f16_to_f32_finite(rd16(blk));
    for (int j = 0; j < 16; j++) {
        out[j] = kvalues_iq4nl[blk[2 + j] & 0x0F];
        out[j + 16] = kvalues_iq4nl[blk[2 + j] >> 4];
    }
    return d;
}

/* quant.rs:348-356 */
void or_dequantize_iq4_nl_block(const uint8_t *blk, float *out) {
    int8_t q[32];
    float d = or_unpack_iq4_nl_block_i8(blk, q);
    scale_i8_into_f32(d, q, out, 32);
}

/* ime.rs:636-658: crate layout, d first, element 4i+j = bits 2j of qs[i] */
float or_unpack_tq2_0_block_i8(const uint8_t *blk, int8_t *out) {
    float s = or_f16_to_f32_finite(rd16(blk));
    for (int i = 0; i < 64; i++) {
        uint8_t b = blk[2 + i];
        out[4 * i] = (int8_t)((b & 3) - 1);
        out[4 * i + 1] = (int8_t)(((b >> 2) & 3) - 1);
        out[4 * i + 2] = (int8_t)(((b >> 4) & 3) - 1);
        out[4 * i + 3] = (int8_t)(((b >> 6) & 3) - 1);
    }
    return s;
}

/* quant.rs:370-377 */
void or_unpack_i2_s_block_i8(const uint8_t *blk, int8_t *out) {
    for (int g = 0; g < 32; g++) {
        uint8_t b = blk[g];
        out[g] = (int8_t)(((b >> 6) & 3) - 1);
        out[32 + g] = (int8_t)(((b >> 4) & 3) - 1);
        out[64 + g] = (int8_t)(((b >> 2) & 3) - 1);
        out[96 + g] = (int8_t)((b & 3) - 1);
    }
}

/* convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790): the 256 trits of two I2_S blocks (blk0 then
 * blk1, each in unpack_i2_s_block_i8 order) re-packed as a crate-layout TQ2_0 block: the f16
 * scale bits first, then byte i = (t[4i] + 1) | (t[4i+1] + 1) << 2 | (t[4i+2] + 1) << 4 |
 * (t[4i+3] + 1) << 6. */
void or_convert_i2_s_blocks_to_tq2_0(const uint8_t *blk0, const uint8_t *blk1, uint16_t scale_f16_bits,
                                     uint8_t *out) {
    int8_t t[256];
    or_unpack_i2_s_block_i8(blk0, t);
    or_unpack_i2_s_block_i8(blk1, t + 128);
    out[0] = (uint8_t)(scale_f16_bits & 0xFF);
    out[1] = (uint8_t)(scale_f16_bits >> 8);
    for (int i = 0; i < 64; i++) {
        const uint8_t q0 = (uint8_t)(t[4 * i] + 1) & 3, q1 = (uint8_t)(t[4 * i + 1] + 1) & 3;
        const uint8_t q2 = (uint8_t)(t[4 * i + 2] + 1) & 3, q3 = (uint8_t)(t[4 * i + 3] + 1) & 3;
        out[2 + i] = (uint8_t)(q0 | (q1 << 2) | (q2 << 4) | (q3 << 6));
    }
}

/* quant.rs:94-102 (scale_i8_into_f32) */
static void scale_i8_into_f32(float scale, const int8_t *q, float *out, int n) {
    if (scale == 0.0f) { for (int i = 0; i < n; i++) out[i] = 0.0f; return; }
    for (int i = 0; i < n; i++) out[i] = scale * (float)q[i];
}

/* quant.rs:380-387 */
void or_dequantize_i2_s_block(const uint8_t *blk, float scale, float *out) {
    int8_t q[128];
    or_unpack_i2_s_block_i8(blk, q);
    scale_i8_into_f32(scale, q, out, 128);
}

/* quant.rs:360-366 */
float or_read_i2_s_trailer_scale(const uint8_t *t, size_t len) {
    if (len < 4) return 0.0f;
    float v;
    memcpy(&v, t, 4);
    return isfinite(v) ? v : 0.0f;
}

/* One block of any path format to f32 (quant.rs:2272-2392 dispatch arms). */
static void dequant_block_any(int q, const uint8_t *blk, float i2s_scale, float *out) {
    switch (q) {
    case OR_Q4_0: or_dequantize_q4_0_block(blk, out); break;
    case OR_Q8_0: or_dequantize_q8_0_block(blk, out); break;
    case OR_Q4_K: or_dequantize_q4_k_block(blk, out); break;
    case OR_Q6_K: or_dequantize_q6_k_block(blk, out); break;
    case OR_Q5_0: or_dequantize_q5_0_block(blk, out); break; /* quant.rs:2306-2310 */
    case OR_Q4_1: or_dequantize_q4_1_block(blk, out); break; /* quant.rs:2301-2305 */
    case OR_Q5_1: or_dequantize_q5_1_block(blk, out); break; /* quant.rs:2311-2315 */
    case OR_Q2_K: or_dequantize_q2_k_block(blk, out); break; /* quant.rs:2321-2325 */
    case OR_Q3_K: or_dequantize_q3_k_block(blk, out); break; /* quant.rs:2326-2330 */
    case OR_IQ4_NL: or_dequantize_iq4_nl_block(blk, out); break; /* quant.rs:2345-2358 */
    case OR_Q5_K: or_dequantize_q5_k_block(blk, out); break; /* quant.rs:2335-2339 */
    case OR_TQ1_0: { /* quant.rs:2359-2368 */
        int8_t t[256];
        float d = or_unpack_tq1_0_block_i8(blk, t);
        scale_i8_into_f32(d, t, out, 256);
        break;
    }
    case OR_TQ2_0: { /* quant.rs:2369-2378 */
        int8_t t[256];
        float d = or_unpack_tq2_0_block_i8(blk, t);
        scale_i8_into_f32(d, t, out, 256);
        break;
    }
    case OR_I2_S: or_dequantize_i2_s_block(blk, i2s_scale, out); break;
    default: break;
    }
}

static int known_quant(int q) { return or_block_elements(q) != 0; }

/* quant.rs:2403-2483 */
int or_dequantize_row_bytes(int quant, const uint8_t *row, size_t row_len, size_t n_cols,
                            float *out, size_t out_len) {
    if (n_cols == 0 || out_len != n_cols) return OR_TENSOR_BOUNDS;
    if (!known_quant(quant)) return OR_CAPABILITY_MISMATCH;
    size_t be = or_block_elements(quant), bb = or_block_bytes(quant);
    if (n_cols % be) return OR_TENSOR_BOUNDS;
    size_t packed = (n_cols / be) * bb;
    if (row_len != packed + or_scale_trailer_bytes(quant)) return OR_TENSOR_BOUNDS;
    float s = quant == OR_I2_S ? or_read_i2_s_trailer_scale(row + packed, row_len - packed) : 1.0f;
    for (size_t b = 0; b < n_cols / be; b++) dequant_block_any(quant, row + b * bb, s, out + b * be);
    return OR_OK;
}

static size_t num_elements(const or_tensor_view *w) {
    size_t n = 1;
    for (size_t i = 0; i < w->ndim; i++) n *= w->shape[i];
    return w->ndim ? n : 0;
}

/* quant.rs:2492-2568 with validate_token_row_geometry quant.rs:1749-1808 */
int or_dequantize_tensor_row(const or_tensor_view *w, size_t row, float *out, size_t out_len) {
    if (!known_quant(w->quant)) return OR_CAPABILITY_MISMATCH;
    size_t cols = out_len;
    if (cols == 0) return OR_TENSOR_BOUNDS;
    size_t total = num_elements(w);
    if (total == 0 || total % cols) return OR_TENSOR_BOUNDS;
    size_t nrows = total / cols;
    if (w->ndim == 2 && !((w->shape[0] == cols && w->shape[1] == nrows) ||
                          (w->shape[1] == cols && w->shape[0] == nrows)))
        return OR_TENSOR_BOUNDS;
    if (row >= nrows) return OR_TENSOR_BOUNDS;
    size_t be = or_block_elements(w->quant), bb = or_block_bytes(w->quant);
    if (cols % be) return OR_TENSOR_BOUNDS;
    size_t row_bytes = (cols / be) * bb, payload = nrows * row_bytes;
    if (w->byte_len < payload + or_scale_trailer_bytes(w->quant)) return OR_TENSOR_BOUNDS;
    float s = w->quant == OR_I2_S ? or_read_i2_s_trailer_scale(w->bytes + payload, w->byte_len - payload)
                                  : 1.0f;
    const uint8_t *r = w->bytes + row * row_bytes;
    for (size_t b = 0; b < cols / be; b++) dequant_block_any(w->quant, r + b * bb, s, out + b * be);
    return OR_OK;
}

/* ------------------------------------------------------------------------- */
/* Activation quantization                                                    */
/* ------------------------------------------------------------------------- */

/* quant_q8.rs:102-108 */
static int8_t round_scaled_to_i8(float v, float inv) {
    if (!isfinite(v)) return 0;
    return rust_round_clamp_i8(v * inv, -127.0f, 127.0f);
}

/* quant_q8.rs:203-219; amax is a fold of f32::max over |finite x| from 0.0 */
static void quantize_block_q8_0(const float *x, or_block_q8_0 *b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++)
        if (isfinite(x[i])) amax = fmaxf(amax, fabsf(x[i]));
    if (amax == 0.0f || !isfinite(amax)) { memset(b, 0, sizeof *b); return; }
    float inv = 127.0f / amax;
    b->d = amax / 127.0f;
    for (int i = 0; i < 32; i++) b->qs[i] = round_scaled_to_i8(x[i], inv);
}

/* quant_q8.rs:111-149 (validate_activation_input / _quant_slice) */
int or_quantize_row_q8_0(const float *x, size_t n, or_block_q8_0 *out, size_t out_len) {
    if (n == 0 || n % 32) return OR_TENSOR_BOUNDS;
    if (out_len != n / 32) return OR_TENSOR_BOUNDS;
    for (size_t b = 0; b < n / 32; b++) quantize_block_q8_0(x + 32 * b, out + b);
    return OR_OK;
}

/* quant_q8.rs:447-475 */
static void quantize_block_q8_k(const float *x, or_block_q8k *b) {
    float amax = 0.0f;
    for (int i = 0; i < 256; i++)
        if (isfinite(x[i])) amax = fmaxf(amax, fabsf(x[i]));
    if (amax == 0.0f || !isfinite(amax)) { memset(b, 0, sizeof *b); return; }
    float inv = 127.0f / amax;
    b->d = amax / 127.0f;
    for (int s = 0; s < 16; s++) {
        int16_t sum = 0;
        for (int i = 0; i < 16; i++) {
            int8_t q = round_scaled_to_i8(x[16 * s + i], inv);
            b->qs[16 * s + i] = q;
            sum = (int16_t)(sum + q);
        }
        b->bsums[s] = sum;
    }
}

/* quant_q8.rs:576-594 */
int or_quantize_row_q8_k(const float *x, size_t n, or_block_q8k *out, size_t out_len) {
    if (n == 0 || n % 256) return OR_TENSOR_BOUNDS;
    if (out_len != n / 256) return OR_TENSOR_BOUNDS;
    for (size_t b = 0; b < n / 256; b++) quantize_block_q8_k(x + 256 * b, out + b);
    return OR_OK;
}

/* repack.rs:175-204: sequential f32 sum from +0.0; zero threshold absmax < 1e-30 */
static void quantize_block32(const float *src, int8_t *q, float *scale, float *sum_out) {
    float clean[32], absmax = 0.0f, sum = 0.0f;
    for (int i = 0; i < 32; i++) {
        float v = isfinite(src[i]) ? src[i] : 0.0f;
        clean[i] = v;
        sum += v;
        float a = fabsf(v);
        if (a > absmax) absmax = a;
    }
    *sum_out = sum;
    if (absmax < 1e-30f) {
        memset(q, 0, 32);
        *scale = 0.0f;
        return;
    }
    float inv = 127.0f / absmax;
    *scale = absmax / 127.0f;
    for (int i = 0; i < 32; i++) q[i] = rust_round_clamp_i8(clean[i] * inv, -127.0f, 127.0f);
}

size_t or_act_q8_bytes(size_t m, size_t k) {
    size_t kp = (k + 31) / 32 * 32, kb = kp / 32, kc = kp / 16, sb = (k + 255) / 256;
    return m * kp + 4 * m * (kb + kb + kc + sb);
}

/* QuantizedActQ8::quantize_into, repack.rs:542-650 (logical row-major form) */
int or_quantize_act_q8(const float *act, size_t m, size_t k, void *storage, size_t storage_len,
                       or_act_q8 *o) {
    if (m == 0 || k == 0) return OR_TENSOR_BOUNDS;
    if (storage_len < or_act_q8_bytes(m, k)) return OR_TENSOR_BOUNDS;
    o->m = m; o->k = k;
    o->k_padded = (k + 31) / 32 * 32;
    o->k_blocks32 = o->k_padded / 32;
    o->k_chunks = o->k_padded / 16;
    o->sb256 = (k + 255) / 256;
    float *f = (float *)storage;
    o->scales = f; f += m * o->k_blocks32;
    o->sums = f; f += m * o->k_blocks32;
    o->sums16 = f; f += m * o->k_chunks;
    o->super256 = f; f += m * o->sb256;
    o->qs = (int8_t *)f;
    float *row_f32 = malloc(o->k_padded * sizeof(float));
    if (!row_f32) return OR_TENSOR_BOUNDS;
    for (size_t r = 0; r < m; r++) {
        const float *src = act + r * k;
        for (size_t i = 0; i < o->k_padded; i++)
            row_f32[i] = i < k ? (isfinite(src[i]) ? src[i] : 0.0f) : 0.0f;
        for (size_t i = 0; i < o->sb256; i++) o->super256[r * o->sb256 + i] = 0.0f;
        /* quantize_row_f32_to_q8_32_scalar, repack.rs:376-400: zero-padded tail */
        for (size_t b = 0; b < o->k_blocks32; b++) {
            float buf[32];
            for (int i = 0; i < 32; i++) {
                size_t idx = 32 * b + i;
                buf[i] = idx < k ? src[idx] : 0.0f;
            }
            float sc, sm;
            quantize_block32(buf, o->qs + r * o->k_padded + 32 * b, &sc, &sm);
            o->scales[r * o->k_blocks32 + b] = sc;
            o->sums[r * o->k_blocks32 + b] = sm;
            size_t sbi = (32 * b) / 256;
            if (sbi < o->sb256 && sc > o->super256[r * o->sb256 + sbi]) o->super256[r * o->sb256 + sbi] = sc;
        }
        /* x_sums_16: `.iter().copied().sum()` over the sanitized f32 row (repack.rs:644-645) */
        for (size_t c = 0; c < o->k_chunks; c++) {
            float s = neg_zero();
            for (int i = 0; i < 16; i++) s += row_f32[16 * c + i];
            o->sums16[r * o->k_chunks + c] = s;
        }
    }
    free(row_f32);
    return OR_OK;
}

/* Shared tail of lib.rs:1072-1098 on already-normalized values. */
static float absmax_quantize_tail(int8_t *out, const float *xn, size_t len) {
    float max_val = 0.0f;
    for (size_t i = 0; i < len; i++) {
        float a = fabsf(xn[i]);
        if (a > max_val) max_val = a;
    }
    if (isnan(max_val) || max_val < 1e-12f) {
        memset(out, 0, len);
        return 1.0f / 127.0f;
    }
    float scale = max_val / 127.0f;
    for (size_t i = 0; i < len; i++) out[i] = rust_round_clamp_i8(xn[i] / scale, -128.0f, 127.0f);
    return scale;
}

/* lib.rs:1042-1101 */
int or_subln_quantize_absmax_i8(int8_t *out, const float *in, const float *w, size_t len,
                                float eps, float *scale_out) {
    if (len == 0) return OR_TENSOR_BOUNDS;
    float sum_sq = 0.0f; /* dot_product_f32_scalar, lib.rs:770-778 */
    for (size_t i = 0; i < len; i++) sum_sq += in[i] * in[i];
    float mean_sq = sum_sq / (float)len;
    float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    float *xn = malloc(len * sizeof(float));
    if (!xn) return OR_TENSOR_BOUNDS;
    for (size_t i = 0; i < len; i++) xn[i] = in[i] * inv_rms * w[i];
    *scale_out = absmax_quantize_tail(out, xn, len);
    free(xn);
    return OR_OK;
}

/* Per-token absmax quantizer without the RMSNorm step: lib.rs:1072-1098 applied to
 * x_norm = input (identical to the subln recipe whenever inv_rms == 1 and w == 1). */
int or_quantize_absmax_i8(int8_t *out, const float *in, size_t len, float *scale_out) {
    if (len == 0) return OR_TENSOR_BOUNDS;
    *scale_out = absmax_quantize_tail(out, in, len);
    return OR_OK;
}

/* ------------------------------------------------------------------------- */
/* Validators                                                                 */
/* ------------------------------------------------------------------------- */

/* Orientation rule shared by validate_quant_matvec_dimensions (quant.rs:1810-1894),
 * validate_q4_0/q8_0/q6_k_dimensions (quant.rs:762-892, 1315-1394) and
 * validate_q4_k_m_dimensions (lib.rs:1195-1260): [rows, cols] or GGUF [cols, rows]. */
static int orient(const or_tensor_view *w, int quant, size_t out_len, size_t in_len,
                  size_t *rows, size_t *cols) {
    if (w->quant != quant) return OR_TENSOR_BOUNDS;
    if (w->ndim == 0) return OR_TENSOR_BOUNDS;
    size_t be = or_block_elements(quant);
    if (w->ndim == 2) {
        size_t d0 = w->shape[0], d1 = w->shape[1];
        if (out_len == d0 && in_len == d1 && d1 % be == 0) { *rows = d0; *cols = d1; }
        else if (out_len == d1 && in_len == d0 && d0 % be == 0) { *rows = d1; *cols = d0; }
        else return OR_TENSOR_BOUNDS;
    } else {
        size_t total = num_elements(w);
        if (in_len == 0 || out_len == 0 || in_len % be || out_len * in_len != total) return OR_TENSOR_BOUNDS;
        *rows = out_len; *cols = in_len;
    }
    /* Byte-length check (quant.rs:1881-1891). The Q8_0 / Q6_K / Q4_K validators leave it
     * to the slice bound, which panics; here every format fails closed instead. */
    if (*cols == 0 || *rows == 0) return OR_TENSOR_BOUNDS;
    size_t need = (*rows * *cols / be) * or_block_bytes(quant) + or_scale_trailer_bytes(quant);
    if (w->byte_len < need) return OR_TENSOR_BOUNDS;
    return OR_OK;
}

/* ------------------------------------------------------------------------- */
/* quant_q8 integer block dots                                                */
/* ------------------------------------------------------------------------- */

/* quant_q8.rs:672-684 */
static float dot_q4_0_q8_0_block(const uint8_t *w, const or_block_q8_0 *x) {
    float dw = or_f16_to_f32_finite(rd16(w));
    if (dw == 0.0f || x->d == 0.0f) return 0.0f;
    int32_t sumi = 0;
    for (int i = 0; i < 16; i++) {
        uint8_t b = w[2 + i];
        sumi += ((int)(b & 0x0F) - 8) * x->qs[i] + ((int)((b >> 4) & 0x0F) - 8) * x->qs[i + 16];
    }
    return (float)sumi * (dw * x->d);
}

/* quant_q8.rs:707-717 */
static float dot_q8_0_q8_0_block(const uint8_t *w, const or_block_q8_0 *x) {
    float dw = or_f16_to_f32_finite(rd16(w));
    if (dw == 0.0f || x->d == 0.0f) return 0.0f;
    int32_t sumi = 0;
    for (int i = 0; i < 32; i++) sumi += (int8_t)w[2 + i] * x->qs[i];
    return (float)sumi * (dw * x->d);
}

/* quant_q8.rs:1834-1862 */
static float dot_q4_k_q8_k_block(const uint8_t *w, const or_block_q8k *x) {
    float d = or_f16_to_f32_finite(rd16(w)), dmin = or_f16_to_f32_finite(rd16(w + 2));
    if ((d == 0.0f && dmin == 0.0f) || x->d == 0.0f) return 0.0f;
    uint8_t sc[8], m[8];
    unpack_k4_scales_mins(w + 4, sc, m);
    const uint8_t *qs = w + 16;
    int32_t sumi = 0, sum_mins = 0;
    for (int c = 0; c < 4; c++) {
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) {
            uint8_t b = qs[32 * c + l];
            lo += (b & 0x0F) * x->qs[64 * c + l];
            hi += (b >> 4) * x->qs[64 * c + 32 + l];
        }
        sumi += sc[2 * c] * lo + sc[2 * c + 1] * hi;
        int32_t bl = x->bsums[4 * c] + x->bsums[4 * c + 1];
        int32_t bh = x->bsums[4 * c + 2] + x->bsums[4 * c + 3];
        sum_mins += m[2 * c] * bl + m[2 * c + 1] * bh;
    }
    return (d * x->d) * (float)sumi - (dmin * x->d) * (float)sum_mins;
}

/* quant_q8.rs:1903-1942 */
static float dot_q6_k_q8_k_block(const uint8_t *w, const or_block_q8k *x) {
    float d = or_f16_to_f32_finite(rd16(w + 208));
    if (d == 0.0f || x->d == 0.0f) return 0.0f;
    const uint8_t *ql = w, *qh = w + 128;
    const int8_t *sc = (const int8_t *)(w + 192);
    int32_t sumi = 0;
    for (int h = 0; h < 2; h++) {
        int n = 128 * h;
        for (int is = 0; is < 2; is++) {
            int32_t s1 = 0, s2 = 0, s3 = 0, s4 = 0;
            for (int l = 16 * is; l < 16 * is + 16; l++) {
                uint8_t bl = ql[64 * h + l], bh = ql[64 * h + l + 32], hb = qh[32 * h + l];
                int q1 = (int)((bl & 0x0F) | ((hb & 3) << 4)) - 32;
                int q2 = (int)((bh & 0x0F) | (((hb >> 2) & 3) << 4)) - 32;
                int q3 = (int)((bl >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                int q4 = (int)((bh >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                s1 += q1 * x->qs[n + l];
                s2 += q2 * x->qs[n + l + 32];
                s3 += q3 * x->qs[n + l + 64];
                s4 += q4 * x->qs[n + l + 96];
            }
            sumi += sc[8 * h + is] * s1 + sc[8 * h + is + 2] * s2 + sc[8 * h + is + 4] * s3 +
                    sc[8 * h + is + 6] * s4;
        }
    }
    return (d * x->d) * (float)sumi;
}

/* quant_q8.rs:1992-2003 with dot_i8_scalar ime.rs:490-496 */
static float dot_tq2_0_q8_k_block(const uint8_t *w, const or_block_q8k *x) {
    if (x->d == 0.0f) return 0.0f;
    int8_t t[256];
    float dw = or_unpack_tq2_0_block_i8(w, t);
    if (dw == 0.0f) return 0.0f;
    int32_t dot = 0;
    for (int i = 0; i < 256; i++) dot += t[i] * x->qs[i];
    return (float)dot * (dw * x->d);
}

typedef float (*blockdot_fn)(const uint8_t *, const void *);

/* quant_q8.rs:688-703 */
static float dot_q5_0_q8_0_block(const uint8_t *w, const or_block_q8_0 *x) {
    float dw = or_f16_to_f32_finite(rd16(w));
    if (dw == 0.0f || x->d == 0.0f) return 0.0f;
    int8_t q[32];
    or_unpack_q5_0_block_i8(w, q);
    int32_t sumi = 0;
    for (int j = 0; j < 16; j++) sumi += q[j] * x->qs[j] + q[j + 16] * x->qs[j + 16];
    return (float)sumi * (dw * x->d);
}

/* quant_q8.rs:1866-1899: the Q4_K recipe with a fifth bit (+16) from qh */
static float dot_q5_k_q8_k_block(const uint8_t *w, const or_block_q8k *x) {
    float d = or_f16_to_f32_finite(rd16(w)), dmin = or_f16_to_f32_finite(rd16(w + 2));
    if ((d == 0.0f && dmin == 0.0f) || x->d == 0.0f) return 0.0f;
    uint8_t sc[8], m[8];
    unpack_k4_scales_mins(w + 4, sc, m);
    const uint8_t *qh = w + 16, *qs = w + 48;
    int32_t sumi = 0, sum_mins = 0;
    for (int c = 0; c < 4; c++) {
        uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) {
            uint8_t b = qs[32 * c + l];
            int32_t h1 = (qh[l] & u1) ? 16 : 0, h2 = (qh[l] & u2) ? 16 : 0;
            lo += ((int32_t)(b & 0x0F) | h1) * x->qs[64 * c + l];
            hi += ((int32_t)(b >> 4) | h2) * x->qs[64 * c + 32 + l];
        }
        sumi += (int32_t)sc[2 * c] * lo + (int32_t)sc[2 * c + 1] * hi;
        int32_t bl = (int32_t)x->bsums[4 * c] + x->bsums[4 * c + 1];
        int32_t bh = (int32_t)x->bsums[4 * c + 2] + x->bsums[4 * c + 3];
        sum_mins += (int32_t)m[2 * c] * bl + (int32_t)m[2 * c + 1] * bh;
    }
    return (d * x->d) * (float)sumi - (dmin * x->d) * (float)sum_mins;
}

/* quant_q8.rs:1977-1988 with unpack_tq1_0_lut (1966-1975), whose table holds the same
 * base-3 digits as unpack_tq1_0_block_i8 */
static float dot_tq1_0_q8_k_block(const uint8_t *w, const or_block_q8k *x) {
    if (x->d == 0.0f) return 0.0f;
    int8_t t[256];
    float dw = or_unpack_tq1_0_block_i8(w, t);
    if (dw == 0.0f) return 0.0f;
    int32_t dot = 0;
    for (int i = 0; i < 256; i++) dot += t[i] * x->qs[i];
    return (float)dot * (dw * x->d);
}

static float bd_q4_0(const uint8_t *w, const void *x) { return dot_q4_0_q8_0_block(w, x); }
static float bd_q8_0(const uint8_t *w, const void *x) { return dot_q8_0_q8_0_block(w, x); }
static float bd_q4_k(const uint8_t *w, const void *x) { return dot_q4_k_q8_k_block(w, x); }
static float bd_q6_k(const uint8_t *w, const void *x) { return dot_q6_k_q8_k_block(w, x); }
static float bd_tq2_0(const uint8_t *w, const void *x) { return dot_tq2_0_q8_k_block(w, x); }
static float bd_q5_0(const uint8_t *w, const void *x) { return dot_q5_0_q8_0_block(w, x); }
static float bd_q5_k(const uint8_t *w, const void *x) { return dot_q5_k_q8_k_block(w, x); }
static float bd_tq1_0(const uint8_t *w, const void *x) { return dot_tq1_0_q8_k_block(w, x); }

static blockdot_fn blockdot_for(int q, size_t *xsz) {
    switch (q) {
    case OR_Q4_0: *xsz = sizeof(or_block_q8_0); return bd_q4_0;
    case OR_Q8_0: *xsz = sizeof(or_block_q8_0); return bd_q8_0;
    case OR_Q4_K: *xsz = sizeof(or_block_q8k); return bd_q4_k;
    case OR_Q6_K: *xsz = sizeof(or_block_q8k); return bd_q6_k;
    case OR_TQ2_0: *xsz = sizeof(or_block_q8k); return bd_tq2_0;
    case OR_Q5_0: *xsz = sizeof(or_block_q8_0); return bd_q5_0;
    case OR_Q5_K: *xsz = sizeof(or_block_q8k); return bd_q5_k;
    case OR_TQ1_0: *xsz = sizeof(or_block_q8k); return bd_tq1_0;
    default: return 0;
    }
}

/* Row drivers dot_*_row (quant_q8.rs:1217-1238, 1290-1311, 2815-2830, 2860-2873, 2902-2915,
 * 2944-2950, 2987-2993):
 * `.map(block_dot).sum()` -> fold from -0.0 in block order. */
static float row_sum_neg0(blockdot_fn f, const uint8_t *w, size_t bb, const uint8_t *x, size_t xsz,
                          size_t nb) {
    float acc = neg_zero();
    for (size_t b = 0; b < nb; b++) acc += f(w + b * bb, x + b * xsz);
    return acc;
}

/* validate_q8_block_row_bytes, quant_q8.rs:644-664 */
static int vec_dot_rowblocks(int q, const uint8_t *w, size_t w_len, const void *x, size_t nx,
                             float *out) {
    size_t xsz, bb = or_block_bytes(q);
    blockdot_fn f = blockdot_for(q, &xsz);
    if (nx == 0 || w_len != nx * bb) return OR_TENSOR_BOUNDS;
    *out = row_sum_neg0(f, w, bb, x, xsz, nx);
    return OR_OK;
}

/* quant_q8.rs:1463 */
int or_vec_dot_q4_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q4_0, w, w_len, x, nx, out);
}
/* quant_q8.rs:1493 */
int or_vec_dot_q8_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q8_0, w, w_len, x, nx, out);
}
/* quant_q8.rs:3019 */
int or_vec_dot_q4_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q4_K, w, w_len, x, nx, out);
}
/* quant_q8.rs:3056 */
int or_vec_dot_q6_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q6_K, w, w_len, x, nx, out);
}
/* quant_q8.rs:3086 */
int or_vec_dot_tq2_0_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_TQ2_0, w, w_len, x, nx, out);
}
/* vec_dot_q5_0_q8_0_blocks (quant_q8.rs:1478) */
int or_vec_dot_q5_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q5_0, w, w_len, x, nx, out);
}
/* quant_q8.rs:3041 */
int or_vec_dot_q5_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_Q5_K, w, w_len, x, nx, out);
}
/* quant_q8.rs:3071 */
int or_vec_dot_tq1_0_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx, float *out) {
    return vec_dot_rowblocks(OR_TQ1_0, w, w_len, x, nx, out);
}

/* run_4row_chunked_gemv (quant_q8.rs:1510-1560) with accumulate = false:
 * rows below (rows / 4) * 4 use the 4-row kernels (acc = [0.0; 4], += per block),
 * the tail rows use the 1-row `.sum()` driver. */
int or_gemv_rows(int quant, float *out, const uint8_t *w, size_t rows, size_t cols, const void *x,
                 size_t r0, size_t r1) {
    size_t xsz, bb = or_block_bytes(quant), nb = cols / or_block_elements(quant);
    blockdot_fn f = blockdot_for(quant, &xsz);
    if (!f) return OR_CAPABILITY_MISMATCH;
    size_t rows4 = rows / 4 * 4, stride = nb * bb;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t *wr = w + r * stride;
        if (r < rows4) {
            float acc = 0.0f;
            for (size_t b = 0; b < nb; b++) acc += f(wr + b * bb, (const uint8_t *)x + b * xsz);
            out[r - r0] = acc;
        } else {
            out[r - r0] = row_sum_neg0(f, wr, bb, x, xsz, nb);
        }
    }
    return OR_OK;
}

/* gemv_* entry points: cols = x_blocks.len() * block_elements, then the format's
 * validator and check_q8_block_len (quant_q8.rs:1562-1578). */
static int gemv_entry(int quant, float *out, size_t out_len, const or_tensor_view *w,
                      const void *x, size_t nx) {
    size_t rows, cols;
    int st = orient(w, quant, out_len, nx * or_block_elements(quant), &rows, &cols);
    if (st) return st;
    if (nx != cols / or_block_elements(quant)) return OR_TENSOR_BOUNDS;
    return or_gemv_rows(quant, out, w->bytes, rows, cols, x, 0, rows);
}

/* quant_q8.rs:1586-1605 */
int or_gemv_q4_0_q8_0(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8_0 *x, size_t nx) {
    return gemv_entry(OR_Q4_0, out, out_len, w, x, nx);
}
/* quant_q8.rs:1670-1689 */
int or_gemv_q8_0_q8_0(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8_0 *x, size_t nx) {
    return gemv_entry(OR_Q8_0, out, out_len, w, x, nx);
}
/* quant_q8.rs:3101-3123 */
int or_gemv_q4_k_q8_k(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8k *x, size_t nx) {
    return gemv_entry(OR_Q4_K, out, out_len, w, x, nx);
}
/* quant_q8.rs:3189-3211 */
int or_gemv_q6_k_q8_k(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8k *x, size_t nx) {
    return gemv_entry(OR_Q6_K, out, out_len, w, x, nx);
}
/* quant_q8.rs:3250-3273 */
int or_gemv_tq2_0_q8_k(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8k *x, size_t nx) {
    return gemv_entry(OR_TQ2_0, out, out_len, w, x, nx);
}
/* quant_q8.rs:1628-1650 */
int or_gemv_q5_0_q8_0(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8_0 *x, size_t nx) {
    return gemv_entry(OR_Q5_0, out, out_len, w, x, nx);
}
/* quant_q8.rs:3160-3182 */
int or_gemv_q5_k_q8_k(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8k *x, size_t nx) {
    return gemv_entry(OR_Q5_K, out, out_len, w, x, nx);
}
/* quant_q8.rs:3219-3242 */
int or_gemv_tq1_0_q8_k(float *out, size_t out_len, const or_tensor_view *w, const or_block_q8k *x, size_t nx) {
    return gemv_entry(OR_TQ1_0, out, out_len, w, x, nx);
}

/* ------------------------------------------------------------------------- */
/* f32-activation matvec: dequantize block, dot_product_f32_scalar, row sum   */
/* ------------------------------------------------------------------------- */

/* vec_dot_q4_0_scalar quant.rs:1401-1436, vec_dot_q8_0_scalar 899-934,
 * vec_dot_q6_k_scalar 1012-1047, vec_dot_q4_k_m_scalar lib.rs:1268-1303,
 * vec_dot_i2_s quant.rs:2199-2240 (zero trailer scale -> row 0.0). */
static int vec_dot_f32_entry(int quant, float *out, size_t out_len, const or_tensor_view *w,
                             const float *in, size_t in_len) {
    size_t rows, cols;
    int st = orient(w, quant, out_len, in_len, &rows, &cols);
    if (st) return st;
    size_t be = or_block_elements(quant), bb = or_block_bytes(quant), nb = cols / be;
    float s = 1.0f;
    if (quant == OR_I2_S) {
        size_t payload = rows * nb * bb;
        s = or_read_i2_s_trailer_scale(w->bytes + payload, w->byte_len - payload);
    }
    float buf[256];
    for (size_t r = 0; r < rows; r++) {
        if (quant == OR_I2_S && s == 0.0f) { out[r] = 0.0f; continue; }
        float row_sum = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            dequant_block_any(quant, w->bytes + (r * nb + b) * bb, s, buf);
            float sum = 0.0f; /* lib.rs:770-778 */
            for (size_t i = 0; i < be; i++) sum += buf[i] * in[b * be + i];
            row_sum += sum;
        }
        out[r] = row_sum;
    }
    return OR_OK;
}

int or_vec_dot_q4_0(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q4_0, out, out_len, w, in, in_len);
}
int or_vec_dot_q8_0(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q8_0, out, out_len, w, in, in_len);
}
int or_vec_dot_q6_k(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q6_K, out, out_len, w, in, in_len);
}
int or_vec_dot_q4_k_m(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q4_K, out, out_len, w, in, in_len);
}
int or_vec_dot_i2_s(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_I2_S, out, out_len, w, in, in_len);
}
/* vec_dot_q5_0 (quant.rs:2036-2054) -> vec_dot_generic_block (1995-2029) */
int or_vec_dot_q5_0(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q5_0, out, out_len, w, in, in_len);
}
/* vec_dot_q4_1 (quant.rs:2062), vec_dot_q5_1 (2081), vec_dot_q2_k (2100), vec_dot_q3_k (2119),
 * vec_dot_iq4_nl (2138): vec_dot_generic_block (1995-2029) over the block dequantizer */
int or_vec_dot_q4_1(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q4_1, out, out_len, w, in, in_len);
}
int or_vec_dot_q5_1(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q5_1, out, out_len, w, in, in_len);
}
int or_vec_dot_q2_k(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q2_K, out, out_len, w, in, in_len);
}
int or_vec_dot_q3_k(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q3_K, out, out_len, w, in, in_len);
}
int or_vec_dot_iq4_nl(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_IQ4_NL, out, out_len, w, in, in_len);
}
/* vec_dot_q5_k (quant.rs:1238-1251) -> vec_dot_q5_k_scalar (1181-1219) */
int or_vec_dot_q5_k(float *out, size_t out_len, const or_tensor_view *w, const float *in, size_t in_len) {
    return vec_dot_f32_entry(OR_Q5_K, out, out_len, w, in, in_len);
}

/* ------------------------------------------------------------------------- */
/* Repacked block-scaled i8 weights and GEMM                                  */
/* ------------------------------------------------------------------------- */

/* validate_matrix_view (repack.rs:1208-1281) + validate_matrix_shape (1172-1206). */
static int validate_matrix_view(const or_tensor_view *w, size_t rows, size_t cols) {
    if (rows == 0 || cols == 0) return OR_TENSOR_BOUNDS;
    size_t be = or_block_elements(w->quant);
    if (cols % be) return OR_TENSOR_BOUNDS;
    if (w->ndim == 1) {
        if (rows * cols != w->shape[0]) return OR_TENSOR_BOUNDS;
    } else if (w->ndim == 2) {
        size_t d0 = w->shape[0], d1 = w->shape[1];
        if (!((d0 == rows && d1 == cols) || (d0 == cols && d1 == rows))) return OR_TENSOR_BOUNDS;
    } else {
        return OR_TENSOR_BOUNDS;
    }
    size_t need = rows * (cols / be) * or_block_bytes(w->quant) + or_scale_trailer_bytes(w->quant);
    if (w->byte_len < need) return OR_TENSOR_BOUNDS;
    return OR_OK;
}

/* BlockScaledTileLayout::from_validated_dims (repack.rs:1334-1366) and the per-format
 * arms of repack_block_scaled_range_into_i8 (repack.rs:1724-2103), written to a
 * logical row-major layout: q[rows][cols], scales/mins[rows][scale_groups]. */
int or_repack_logical(const or_tensor_view *w, size_t rows, size_t cols, int8_t *q,
                      float *scales, float *mins, size_t *sg_out, int *has_mins_out, int *cps_out) {
    if (!known_quant(w->quant)) return OR_CAPABILITY_MISMATCH;
    int st = validate_matrix_view(w, rows, cols);
    if (st) return st;
    int cps = (w->quant == OR_Q6_K || w->quant == OR_Q3_K || w->quant == OR_Q2_K) ? 1 : 2;
    size_t k_padded = (cols + 31) / 32 * 32, sg = k_padded / 16 / cps;
    int has_mins = w->quant == OR_Q4_K || w->quant == OR_Q5_K || w->quant == OR_Q4_1 || w->quant == OR_Q5_1 ||
                   w->quant == OR_Q2_K;
    if (sg_out) *sg_out = sg;
    if (has_mins_out) *has_mins_out = has_mins;
    if (cps_out) *cps_out = cps;
    if (!q) return OR_OK;
    size_t be = or_block_elements(w->quant), bb = or_block_bytes(w->quant), nb = cols / be;
    size_t row_bytes = nb * bb;
    float i2s = 0.0f;
    if (w->quant == OR_I2_S)
        i2s = or_read_i2_s_trailer_scale(w->bytes + rows * row_bytes, w->byte_len - rows * row_bytes);
    memset(q, 0, rows * k_padded);
    for (size_t i = 0; i < rows * sg; i++) scales[i] = 0.0f;
    if (has_mins && mins) for (size_t i = 0; i < rows * sg; i++) mins[i] = 0.0f;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *rr = w->bytes + r * row_bytes;
        int8_t *qr = q + r * k_padded;
        float *sr = scales + r * sg;
        float *mr = has_mins ? mins + r * sg : 0;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = rr + b * bb;
            switch (w->quant) {
            case OR_Q8_0: { /* repack.rs:1766-1781 */
                float d = or_f16_to_f32_finite(rd16(blk));
                sr[b] = d;
                if (d != 0.0f) for (int i = 0; i < 32; i++) qr[32 * b + i] = (int8_t)blk[2 + i];
                break;
            }
            case OR_Q4_0: { /* repack.rs:1782-1813 */
                float d = or_f16_to_f32_finite(rd16(blk));
                sr[b] = d;
                if (d != 0.0f)
                    for (int i = 0; i < 16; i++) {
                        qr[32 * b + i] = (int8_t)((blk[2 + i] & 0x0F) - 8);
                        qr[32 * b + i + 16] = (int8_t)(((blk[2 + i] >> 4) & 0x0F) - 8);
                    }
                break;
            }
            case OR_Q4_K: { /* repack.rs:1912-1955 */
                float d = or_f16_to_f32_finite(rd16(blk)), dmin = or_f16_to_f32_finite(rd16(blk + 2));
                uint8_t sc[8], m[8];
                unpack_k4_scales_mins(blk + 4, sc, m);
                for (int c = 0; c < 4; c++) {
                    size_t g0 = 8 * b + 2 * c;
                    sr[g0] = d * (float)sc[2 * c];
                    mr[g0] = dmin * (float)m[2 * c];
                    sr[g0 + 1] = d * (float)sc[2 * c + 1];
                    mr[g0 + 1] = dmin * (float)m[2 * c + 1];
                    for (int l = 0; l < 32; l++) {
                        qr[256 * b + 64 * c + l] = (int8_t)(blk[16 + 32 * c + l] & 0x0F);
                        qr[256 * b + 64 * c + 32 + l] = (int8_t)(blk[16 + 32 * c + l] >> 4);
                    }
                }
                break;
            }
            case OR_Q4_1: case OR_Q5_1: { /* repack.rs:1814-1829, 1845-1860: quants always written */
                float d, m;
                if (w->quant == OR_Q4_1) unpack_q4_1_block_i8(blk, qr + 32 * b, &d, &m);
                else unpack_q5_1_block_i8(blk, qr + 32 * b, &d, &m);
                sr[b] = d;
                mr[b] = m == 0.0f ? 0.0f : -m;
                break;
            }
            case OR_IQ4_NL: { /* repack.rs:1861-1875 */
                int8_t t[32];
                float d = or_unpack_iq4_nl_block_i8(blk, t);
                sr[b] = d;
                if (d != 0.0f) memcpy(qr + 32 * b, t, 32);
                break;
            }
            case OR_Q2_K: { /* repack.rs:1876-1895 */
                float sc[16], mn[16];
                or_unpack_q2_k_block_i8(blk, qr + 256 * b, sc, mn);
                for (int s = 0; s < 16; s++) { sr[16 * b + s] = sc[s]; mr[16 * b + s] = mn[s]; }
                break;
            }
            case OR_Q3_K: { /* repack.rs:1896-1911 */
                float sc[16];
                or_unpack_q3_k_block_i8(blk, qr + 256 * b, sc);
                for (int s = 0; s < 16; s++) sr[16 * b + s] = sc[s];
                break;
            }
            case OR_Q5_0: { /* repack.rs:1830-1843 */
                int8_t t[32];
                float d = or_unpack_q5_0_block_i8(blk, t);
                sr[b] = d;
                if (d != 0.0f) memcpy(qr + 32 * b, t, 32);
                break;
            }
            case OR_Q5_K: { /* repack.rs:1959-2002 */
                float d = or_f16_to_f32_finite(rd16(blk)), dmin = or_f16_to_f32_finite(rd16(blk + 2));
                uint8_t sc[8], m[8];
                unpack_k4_scales_mins(blk + 4, sc, m);
                const uint8_t *qh = blk + 16, *qs = blk + 48;
                for (int c = 0; c < 4; c++) {
                    size_t g0 = 8 * b + 2 * c;
                    sr[g0] = d * (float)sc[2 * c];
                    mr[g0] = dmin * (float)m[2 * c];
                    sr[g0 + 1] = d * (float)sc[2 * c + 1];
                    mr[g0 + 1] = dmin * (float)m[2 * c + 1];
                    uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
                    for (int l = 0; l < 32; l++) {
                        qr[256 * b + 64 * c + l] = (int8_t)((qs[32 * c + l] & 0x0F) + ((qh[l] & u1) ? 16 : 0));
                        qr[256 * b + 64 * c + 32 + l] = (int8_t)((qs[32 * c + l] >> 4) + ((qh[l] & u2) ? 16 : 0));
                    }
                }
                break;
            }
            case OR_TQ1_0: { /* repack.rs:2046-2060: trits always written */
                float d = or_unpack_tq1_0_block_i8(blk, qr + 256 * b);
                for (int s = 0; s < 8; s++) sr[8 * b + s] = d;
                break;
            }
            case OR_Q6_K: { /* repack.rs:2003-2046 */
                float d = or_f16_to_f32_finite(rd16(blk + 208));
                for (int s = 0; s < 16; s++) sr[16 * b + s] = d * (float)(int8_t)blk[192 + s];
                if (d != 0.0f) {
                    const uint8_t *ql = blk, *qh = blk + 128;
                    for (int h = 0; h < 2; h++)
                        for (int l = 0; l < 32; l++) {
                            uint8_t bl = ql[64 * h + l], bh = ql[64 * h + l + 32], hb = qh[32 * h + l];
                            int8_t *o = qr + 256 * b + 128 * h;
                            o[l] = (int8_t)(((bl & 0x0F) | ((hb & 3) << 4)) - 32);
                            o[l + 32] = (int8_t)(((bh & 0x0F) | (((hb >> 2) & 3) << 4)) - 32);
                            o[l + 64] = (int8_t)(((bl >> 4) | (((hb >> 4) & 3) << 4)) - 32);
                            o[l + 96] = (int8_t)(((bh >> 4) | (((hb >> 6) & 3) << 4)) - 32);
                        }
                }
                break;
            }
            case OR_TQ2_0: { /* repack.rs:2061-2075: trits always written */
                float d = or_unpack_tq2_0_block_i8(blk, qr + 256 * b);
                for (int s = 0; s < 8; s++) sr[8 * b + s] = d;
                break;
            }
            case OR_I2_S: { /* repack.rs:2076-2092 */
                int8_t t[128];
                or_unpack_i2_s_block_i8(blk, t);
                for (int s = 0; s < 4; s++) sr[4 * b + s] = i2s;
                if (i2s != 0.0f) memcpy(qr + 128 * b, t, 128);
                break;
            }
            }
        }
    }
    return OR_OK;
}

/* execute_gemm_repacked_rows (repack.rs:2718-3042) on the scalar arm with
 * tile_dot_scalar_rows (ime.rs:127-148) and accumulate_scaled_tile_scalar
 * (repack.rs:3045-3093), over weights already in the logical repacked form (the reference
 * repacks once at load time, RepackedWeight::repack, repack.rs:2255): tokens [m0, m1) x rows
 * [r0, r1), acc starts at 0.0 and adds one term per scale group in order. out is
 * [m1 - m0][r1 - r0]. */
int or_gemm_logical_rows(float *out, const int8_t *q, const float *sc, const float *mn, size_t cols, size_t sg,
                         int cps, const or_act_q8 *act, size_t m0, size_t m1, size_t r0, size_t r1) {
    if (act->k != cols || m0 > m1 || m1 > act->m || r0 > r1) return OR_TENSOR_BOUNDS;
    size_t kp = (cols + 31) / 32 * 32, sub = r1 - r0;
    size_t gl = 16 * (size_t)cps;
    for (size_t i = m0; i < m1; i++) {
        const int8_t *xq = act->qs + i * act->k_padded;
        for (size_t r = r0; r < r1; r++) {
            const int8_t *wq = q + r * kp;
            float acc = 0.0f;
            for (size_t g = 0; g < sg; g++) {
                int32_t c = 0;
                for (size_t k = g * gl; k < (g + 1) * gl; k++) c += xq[k] * wq[k];
                size_t b32 = cps == 2 ? g : g / 2;
                float xs = act->scales[i * act->k_blocks32 + b32];
                float ws = sc[r * sg + g];
                if (mn) {
                    float xsm = cps == 2 ? act->sums[i * act->k_blocks32 + b32] : act->sums16[i * act->k_chunks + g];
                    acc += (float)c * (xs * ws) - xsm * mn[r * sg + g];
                } else {
                    acc += (float)c * (xs * ws);
                }
            }
            out[(i - m0) * sub + (r - r0)] = acc;
        }
    }
    return OR_OK;
}

/* The same product from the GGUF bytes: repack (or_repack_logical) then or_gemm_logical_rows
 * over every token. */
int or_gemm_repacked(float *out, size_t out_len, const or_tensor_view *w, size_t rows, size_t cols,
                     const or_act_q8 *act, size_t r0, size_t r1) {
    size_t sg;
    int has_mins, cps;
    int st = or_repack_logical(w, rows, cols, 0, 0, 0, &sg, &has_mins, &cps);
    if (st) return st;
    if (act->k != cols) return OR_TENSOR_BOUNDS;
    if (r0 > r1 || r1 > rows) return OR_TENSOR_BOUNDS;
    size_t m = act->m, sub = r1 - r0;
    if (out_len != m * sub) return OR_TENSOR_BOUNDS;
    if (sub == 0) return OR_OK;
    size_t kp = (cols + 31) / 32 * 32;
    int8_t *q = malloc(rows * kp);
    float *sc = malloc(rows * sg * sizeof(float));
    float *mn = has_mins ? malloc(rows * sg * sizeof(float)) : 0;
    if (!q || !sc || (has_mins && !mn)) { free(q); free(sc); free(mn); return OR_TENSOR_BOUNDS; }
    or_repack_logical(w, rows, cols, q, sc, mn, 0, 0, 0);
    st = or_gemm_logical_rows(out, q, sc, mn, cols, sg, cps, act, 0, m, r0, r1);
    free(q); free(sc); free(mn);
    return st;
}

/* ------------------------------------------------------------------------- */
/* PackedNibbleMatrix GEMM (the compact 4-bit path, repack.rs:4216-5397)      */
/* ------------------------------------------------------------------------- */

enum { NIB_TILE_N = 8, NIB_TILE_M = 8, NIB_TILE_K = 16 }; /* ime.rs:40-48 */

/* PackedNibbleMatrix (repack.rs:4216-4229): tiles[nt][b32] of 128 bytes (bytes 0..63 hold
 * columns 0..15, 64..127 columns 16..31; within each half, 16-byte segment `pair` holds row
 * 2*pair in the low nibbles and row 2*pair+1 in the high nibbles), plus the per-format
 * metadata of PackedNibbleMeta (repack.rs:4185-4210). */
typedef struct {
    size_t rows, cols, k_blocks32, n_tiles;
    int quant;
    uint8_t *tiles;
    uint16_t *scales_f16, *mins_f16; /* [nt][b32][j] (Q4_0, IQ4_NL; Q4_1 both) */
    uint8_t *headers;                /* [nt][sb][j][16] raw Q4_K headers */
} nibble_matrix;

static void nibble_free(nibble_matrix *nm) {
    free(nm->tiles); free(nm->scales_f16); free(nm->mins_f16); free(nm->headers);
}

/* pack_pair_split_nibbles_into_tile, scalar arm (repack.rs:4297-4305): column k of the even
 * and odd rows' 16 bytes (low nibbles = columns 0..15, high nibbles = columns 16..31). */
static void nibble_pack_pair(const uint8_t *e, const uint8_t *o, uint8_t *tile, int pair) {
    for (int k = 0; k < 16; k++) {
        tile[pair * 16 + k] = (uint8_t)((e[k] & 0x0F) | ((o[k] & 0x0F) << 4));
        tile[64 + pair * 16 + k] = (uint8_t)((e[k] >> 4) | (o[k] & 0xF0));
    }
}

/* pack_q4k_pair_chunk32_into_tiles, scalar arm (repack.rs:4379-4394): the 32 qs bytes of a
 * Q4_K 64-element chunk; low nibbles go to tile lo (b32 = 2c), high nibbles to tile hi. */
static void nibble_pack_q4k_chunk(const uint8_t *e, const uint8_t *o, uint8_t *lo, uint8_t *hi, int pair) {
    for (int k = 0; k < 16; k++) {
        lo[pair * 16 + k] = (uint8_t)((e[k] & 0x0F) | ((o[k] & 0x0F) << 4));
        hi[pair * 16 + k] = (uint8_t)((e[k] >> 4) | (o[k] & 0xF0));
        lo[64 + pair * 16 + k] = (uint8_t)((e[16 + k] & 0x0F) | ((o[16 + k] & 0x0F) << 4));
        hi[64 + pair * 16 + k] = (uint8_t)((e[16 + k] >> 4) | (o[16 + k] & 0xF0));
    }
}

/* PackedNibbleMatrix::from_tensor (repack.rs:4788-4865) via repack_nibble_into_tile_range over
 * every tile (repack.rs:4414-4644). Q4_0 / IQ4_NL blocks whose scale decodes to 0 keep a zero
 * scale and zero nibbles. */
static int nibble_pack(const or_tensor_view *w, size_t rows, size_t cols, nibble_matrix *nm) {
    memset(nm, 0, sizeof *nm);
    int q = w->quant;
    if (q != OR_Q4_0 && q != OR_Q4_K && q != OR_Q4_1 && q != OR_IQ4_NL) return OR_CAPABILITY_MISMATCH;
    int st = validate_matrix_view(w, rows, cols);
    if (st) return st;
    size_t bb = or_block_bytes(q), row_bytes = cols / or_block_elements(q) * bb;
    nm->rows = rows; nm->cols = cols; nm->quant = q;
    nm->k_blocks32 = cols / 32;
    nm->n_tiles = (rows + NIB_TILE_N - 1) / NIB_TILE_N;
    size_t kb = nm->k_blocks32, nt_n = nm->n_tiles, n_sblks = cols / 256;
    nm->tiles = calloc(nt_n * kb, 128);
    if (q == OR_Q4_K) nm->headers = calloc(nt_n * n_sblks * NIB_TILE_N, 16);
    else nm->scales_f16 = calloc(nt_n * kb * NIB_TILE_N, 2);
    if (q == OR_Q4_1) nm->mins_f16 = calloc(nt_n * kb * NIB_TILE_N, 2);
    if (!nm->tiles || (q == OR_Q4_K ? !nm->headers : !nm->scales_f16) || (q == OR_Q4_1 && !nm->mins_f16)) {
        nibble_free(nm);
        return OR_TENSOR_BOUNDS;
    }
    static const uint8_t zero[32] = {0};
    for (size_t nt = 0; nt < nt_n; nt++) {
        uint8_t *ts = nm->tiles + nt * kb * 128;
        for (int pair = 0; pair < 4; pair++) {
            size_t re = nt * NIB_TILE_N + 2 * (size_t)pair;
            if (re >= rows) break;
            int has_odd = re + 1 < rows;
            const uint8_t *er = w->bytes + re * row_bytes, *orr = has_odd ? er + row_bytes : 0;
            if (q == OR_Q4_0 || q == OR_IQ4_NL) {
                for (size_t b = 0; b < kb; b++) {
                    const uint8_t *be = er + b * 18;
                    uint16_t eb = rd16(be);
                    int ez = or_f16_to_f32_finite(eb) == 0.0f;
                    nm->scales_f16[(nt * kb + b) * NIB_TILE_N + 2 * pair] = ez ? 0 : eb;
                    int oz = 1;
                    const uint8_t *no = zero;
                    if (has_odd) {
                        const uint8_t *bo = orr + b * 18;
                        uint16_t ob = rd16(bo);
                        oz = or_f16_to_f32_finite(ob) == 0.0f;
                        nm->scales_f16[(nt * kb + b) * NIB_TILE_N + 2 * pair + 1] = oz ? 0 : ob;
                        if (!oz) no = bo + 2;
                    }
                    const uint8_t *ne = ez ? zero : be + 2;
                    if (!ez || !oz) nibble_pack_pair(ne, no, ts + b * 128, pair);
                }
            } else if (q == OR_Q4_1) {
                for (size_t b = 0; b < kb; b++) {
                    const uint8_t *be = er + b * 20;
                    size_t ie = (nt * kb + b) * NIB_TILE_N + 2 * pair;
                    nm->scales_f16[ie] = rd16(be);
                    nm->mins_f16[ie] = rd16(be + 2);
                    const uint8_t *no = zero;
                    if (has_odd) {
                        const uint8_t *bo = orr + b * 20;
                        nm->scales_f16[ie + 1] = rd16(bo);
                        nm->mins_f16[ie + 1] = rd16(bo + 2);
                        no = bo + 4;
                    }
                    nibble_pack_pair(be + 4, no, ts + b * 128, pair);
                }
            } else { /* Q4_K */
                for (size_t sb = 0; sb < n_sblks; sb++) {
                    const uint8_t *be = er + sb * 144, *bo = has_odd ? orr + sb * 144 : 0;
                    memcpy(nm->headers + ((nt * n_sblks + sb) * NIB_TILE_N + 2 * pair) * 16, be, 16);
                    if (bo) memcpy(nm->headers + ((nt * n_sblks + sb) * NIB_TILE_N + 2 * pair + 1) * 16, bo, 16);
                    for (int c = 0; c < 4; c++) {
                        size_t blo = sb * 8 + 2 * (size_t)c;
                        nibble_pack_q4k_chunk(be + 16 + 32 * c, bo ? bo + 16 + 32 * c : zero, ts + blo * 128,
                                              ts + (blo + 1) * 128, pair);
                    }
                }
            }
        }
    }
    return OR_OK;
}

/* PackedNibbleMatrix::decode_tile_scales (repack.rs:5044-5090): per (b32, j) scale and min of
 * tile nt; returns whether the format has mins. */
static int nibble_decode_tile_scales(const nibble_matrix *nm, size_t nt, float *sc, float *mn) {
    size_t len = nm->k_blocks32 * NIB_TILE_N, base = nt * len;
    if (nm->quant == OR_Q4_0 || nm->quant == OR_IQ4_NL) {
        for (size_t i = 0; i < len; i++) sc[i] = or_f16_to_f32_finite(nm->scales_f16[base + i]);
        return 0;
    }
    if (nm->quant == OR_Q4_1) {
        for (size_t i = 0; i < len; i++) {
            sc[i] = or_f16_to_f32_finite(nm->scales_f16[base + i]);
            float m = or_f16_to_f32_finite(nm->mins_f16[base + i]);
            mn[i] = m == 0.0f ? 0.0f : -m;
        }
        return 1;
    }
    size_t n_sblks = nm->k_blocks32 / 8;
    for (size_t sb = 0; sb < n_sblks; sb++)
        for (int j = 0; j < NIB_TILE_N; j++) {
            const uint8_t *h = nm->headers + ((nt * n_sblks + sb) * NIB_TILE_N + (size_t)j) * 16;
            float d = or_f16_to_f32_finite(rd16(h)), dmin = or_f16_to_f32_finite(rd16(h + 2));
            uint8_t s8[8], m8[8];
            unpack_k4_scales_mins(h + 4, s8, m8);
            for (int is = 0; is < 8; is++) {
                size_t idx = (sb * 8 + (size_t)is) * NIB_TILE_N + (size_t)j;
                sc[idx] = d * (float)s8[is];
                mn[idx] = dmin * (float)m8[is];
            }
        }
    return 1;
}

/* unpack_nibble_tile_to_chunks (repack.rs:5093-5130): ch[0] = columns 0..15, ch[1] = columns
 * 16..31, each [row j][16]; Q4_0 subtracts 8, IQ4_NL looks up KVALUES_IQ4NL, Q4_1 / Q4_K keep
 * the nibble. */
static void nibble_unpack(const uint8_t *t, int quant, int8_t ch[2][128]) {
    for (int pair = 0; pair < 4; pair++)
        for (int k = 0; k < 16; k++) {
            uint8_t b0 = t[pair * 16 + k], b1 = t[64 + pair * 16 + k];
            int v[4] = {b0 & 0x0F, b0 >> 4, b1 & 0x0F, b1 >> 4};
            for (int i = 0; i < 4; i++) v[i] = quant == OR_Q4_0 ? v[i] - 8 : quant == OR_IQ4_NL ? kvalues_iq4nl[v[i]] : v[i];
            ch[0][(2 * pair) * NIB_TILE_K + k] = (int8_t)v[0];
            ch[0][(2 * pair + 1) * NIB_TILE_K + k] = (int8_t)v[1];
            ch[1][(2 * pair) * NIB_TILE_K + k] = (int8_t)v[2];
            ch[1][(2 * pair + 1) * NIB_TILE_K + k] = (int8_t)v[3];
        }
}

/* execute_nibble_gemm_rows (repack.rs:5181-5397), the host (non-RISC-V) arm: per 8-row tile and
 * 8-token tile, acc starts at 0.0; per 32-element block, the i8 tile dot of the activation chunks
 * with the unpacked nibble chunks (tile_dot_scalar_rows, ime.rs:127-148) is folded in by
 * accumulate_scaled_tile_scalar with two chunks per scale (repack.rs:3045-3093). The activation
 * tiles are read through the logical qs[m][k_padded] (the same elements). */
int or_nibble_gemm_rows(float *out, size_t out_len, const or_tensor_view *w, size_t rows, size_t cols,
                        const or_act_q8 *act, size_t r0, size_t r1) {
    nibble_matrix nm;
    int st = nibble_pack(w, rows, cols, &nm);
    if (st) return st;
    st = OR_TENSOR_BOUNDS;
    size_t m = act->m, sub = r1 - r0, kb = nm.k_blocks32;
    float *sc = malloc(kb * NIB_TILE_N * sizeof(float)), *mn = malloc(kb * NIB_TILE_N * sizeof(float));
    if (act->k != cols || r0 > r1 || r1 > rows || out_len != m * sub || !sc || !mn) goto done;
    st = OR_OK;
    if (sub == 0) goto done;
    for (size_t nt = r0 / NIB_TILE_N; nt <= (r1 - 1) / NIB_TILE_N; nt++) {
        size_t j0 = r0 > nt * NIB_TILE_N ? r0 - nt * NIB_TILE_N : 0;
        size_t j1 = r1 - nt * NIB_TILE_N < NIB_TILE_N ? r1 - nt * NIB_TILE_N : NIB_TILE_N;
        int has_mins = nibble_decode_tile_scales(&nm, nt, sc, mn);
        for (size_t mt = 0; mt * NIB_TILE_M < m; mt++) {
            size_t active = m - mt * NIB_TILE_M < NIB_TILE_M ? m - mt * NIB_TILE_M : NIB_TILE_M;
            float acc[NIB_TILE_M * NIB_TILE_N] = {0};
            for (size_t b = 0; b < kb; b++) {
                int8_t ch[2][128];
                nibble_unpack(nm.tiles + (nt * kb + b) * 128, nm.quant, ch);
                for (size_t i = 0; i < active; i++) {
                    size_t gm = mt * NIB_TILE_M + i;
                    const int8_t *xq = act->qs + gm * act->k_padded + 32 * b;
                    float xs = act->scales[gm * act->k_blocks32 + b];
                    float xsm = has_mins ? act->sums[gm * act->k_blocks32 + b] : 0.0f;
                    for (size_t j = j0; j < j1; j++) {
                        int32_t c = 0;
                        for (int h = 0; h < 2; h++)
                            for (int k = 0; k < NIB_TILE_K; k++)
                                c += (int32_t)xq[16 * h + k] * (int32_t)ch[h][j * NIB_TILE_K + (size_t)k];
                        float ws = sc[b * NIB_TILE_N + j];
                        if (has_mins) acc[i * NIB_TILE_N + j] += (float)c * (xs * ws) - xsm * mn[b * NIB_TILE_N + j];
                        else acc[i * NIB_TILE_N + j] += (float)c * (xs * ws);
                    }
                }
            }
            for (size_t i = 0; i < active; i++)
                for (size_t j = j0; j < j1; j++)
                    out[(mt * NIB_TILE_M + i) * sub + (nt * NIB_TILE_N + j - r0)] = acc[i * NIB_TILE_N + j];
        }
    }
done:
    free(sc); free(mn);
    nibble_free(&nm);
    return st;
}

/* ------------------------------------------------------------------------- */
/* BitLinear: bitlinear_i8_rvv (ime.rs:882-938)                               */
/* ------------------------------------------------------------------------- */

/* validate_bitlinear_dimensions (ime.rs:660-763) */
int or_bitlinear_i8(float *out, size_t out_len, const or_tensor_view *w, const int8_t *act,
                    size_t act_len, float act_scale) {
    int q = w->quant;
    if (q != OR_TQ1_0 && q != OR_TQ2_0 && q != OR_Q8_0 && q != OR_I2_S) return OR_TENSOR_BOUNDS;
    if (w->ndim == 0) return OR_TENSOR_BOUNDS;
    size_t be = or_block_elements(q), bb = or_block_bytes(q);
    if (w->ndim == 2) {
        size_t d0 = w->shape[0], d1 = w->shape[1];
        if (!((out_len == d0 && act_len == d1 && d1 % be == 0) ||
              (out_len == d1 && act_len == d0 && d0 % be == 0)))
            return OR_TENSOR_BOUNDS;
    } else {
        size_t total = num_elements(w);
        if (act_len == 0 || out_len == 0 || act_len % be || out_len * act_len != total) return OR_TENSOR_BOUNDS;
    }
    size_t rows = out_len, cols = act_len, nb = cols / be;
    if (w->byte_len < (rows * cols / be) * bb + or_scale_trailer_bytes(q)) return OR_TENSOR_BOUNDS;
    float i2s = 0.0f;
    if (q == OR_I2_S)
        i2s = or_read_i2_s_trailer_scale(w->bytes + rows * nb * bb, w->byte_len - rows * nb * bb);
    int8_t wb[256];
    for (size_t r = 0; r < rows; r++) {
        float row_sum = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = w->bytes + (r * nb + b) * bb;
            float bs; /* unpack_bitlinear_block_i8, ime.rs:792-871 */
            if (q == OR_TQ1_0) bs = or_unpack_tq1_0_block_i8(blk, wb);
            else if (q == OR_TQ2_0) bs = or_unpack_tq2_0_block_i8(blk, wb);
            else if (q == OR_Q8_0) {
                bs = or_f16_to_f32_finite(rd16(blk));
                for (int i = 0; i < 32; i++) wb[i] = (int8_t)blk[2 + i];
            } else {
                or_unpack_i2_s_block_i8(blk, wb);
                bs = i2s;
            }
            int32_t dot = 0;
            for (size_t i = 0; i < be; i++) dot += wb[i] * act[b * be + i];
            row_sum += (float)dot * (bs * act_scale);
        }
        out[r] = row_sum;
    }
    return OR_OK;
}

/* ------------------------------------------------------------------------- */
/* The step after the path: gated activations and argmax                      */
/* ------------------------------------------------------------------------- */

/* swiglu_f32_scalar (swiglu.rs:98-121): silu = 0 below -20, g above 20, else
 * g / (1 + exp(-g)); out = silu * up. Rust's f32::exp is the platform libm expf. */
int or_swiglu_f32(float *out, const float *gate, const float *up, size_t n) {
    if (n == 0) return OR_TENSOR_BOUNDS;
    for (size_t i = 0; i < n; i++) {
        float g = gate[i], silu;
        if (g < -20.0f) silu = 0.0f;
        else if (g > 20.0f) silu = g;
        else silu = g / (1.0f + expf(-g));
        out[i] = silu * up[i];
    }
    return OR_OK;
}

/* relu_squared_gate_scalar (lib.rs:1140-1147): relu = g > 0 ? g : 0; out = relu * relu * up */
int or_relu_squared_gate_f32(float *out, const float *gate, const float *up, size_t n) {
    if (n == 0) return OR_TENSOR_BOUNDS;
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float relu = g > 0.0f ? g : 0.0f;
        out[i] = relu * relu * up[i];
    }
    return OR_OK;
}

/* argmax_f32_scalar (lib.rs:555-568): lowest index of the largest non-NaN value (values
 * that compare equal, +0.0 and -0.0 included, keep the first); -1 for empty or all-NaN. */
long or_argmax_f32(const float *x, size_t n) {
    long best = -1;
    float best_val = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        if (isnan(v)) continue;
        if (best < 0 || v > best_val) { best_val = v; best = (long)i; }
    }
    return best;
}


/* ------------------------------------------------------------------------- */
/* int8 primitives (ime.rs)                                                   */
/* ------------------------------------------------------------------------- */

/* dot_i8_scalar (ime.rs:490-496): a.iter().zip(b).map(i32 product).sum() */
int32_t or_dot_i8(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len) {
    size_t n = a_len < b_len ? a_len : b_len;
    int32_t s = 0;
    for (size_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

/* gemm_i8_vector (ime.rs:563-583): for n in n_range, for row in 0..m, one dot per output */
void or_gemm_i8_vector(int32_t *c, const int8_t *a, size_t m, const int8_t *b, size_t n0, size_t n1, size_t k) {
    for (size_t n = n0; n < n1; n++)
        for (size_t row = 0; row < m; row++)
            c[row * (n1 - n0) + (n - n0)] = or_dot_i8(a + row * k, k, b + n * k, k);
}

/* pack_tiles (ime.rs:81-94): [row_tile][k_chunk][8][16], missing rows zero */
int or_pack_tiles(int8_t *out, size_t out_len, const int8_t *src, size_t src_len, size_t rows, size_t k) {
    if (k % 16 != 0 || src_len != rows * k) return OR_TENSOR_BOUNDS;
    size_t kc = k / 16;
    if (out_len != (rows + 7) / 8 * kc * 128) return OR_TENSOR_BOUNDS;
    memset(out, 0, out_len);
    for (size_t row = 0; row < rows; row++) {
        size_t tile = row / 8, r = row % 8;
        for (size_t chunk = 0; chunk < kc; chunk++)
            memcpy(out + (tile * kc + chunk) * 128 + r * 16, src + row * k + chunk * 16, 16);
    }
    return OR_OK;
}

/* tile_dot_scalar_rows (ime.rs:127-148): c[i * 8 + j] += a[i][k] * b[j][k] per chunk, rows i < active_m */
void or_tile_dot_scalar_rows(int32_t *c, const int8_t *a, const int8_t *b, size_t k_chunks, size_t active_m) {
    memset(c, 0, 64 * sizeof(int32_t));
    size_t mb = active_m < 8 ? active_m : 8;
    for (size_t chunk = 0; chunk < k_chunks; chunk++) {
        const int8_t *at = a + chunk * 128, *bt = b + chunk * 128;
        for (size_t i = 0; i < mb; i++)
            for (size_t j = 0; j < 8; j++)
                for (size_t kk = 0; kk < 16; kk++) c[i * 8 + j] += (int32_t)at[i * 16 + kk] * (int32_t)bt[j * 16 + kk];
    }
}

/* gemm_i8_ime (ime.rs:449-486), the non-RISC-V arm: tile_dot_scalar (ime.rs:152-156) per pair */
void or_gemm_i8_ime(int32_t *c, const int8_t *a_packed, size_t m_tiles, const int8_t *b_packed, size_t nt0,
                    size_t nt1, size_t k_chunks) {
    size_t stride = k_chunks * 128;
    for (size_t nt = nt0; nt < nt1; nt++)
        for (size_t mt = 0; mt < m_tiles; mt++)
            or_tile_dot_scalar_rows(c + (mt * (nt1 - nt0) + (nt - nt0)) * 64, a_packed + mt * stride,
                                    b_packed + nt * stride, k_chunks, 8);
}
