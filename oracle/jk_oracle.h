/*
 * jk_oracle.h -- CPU restatement of the jero-kernels-rvv portable scalar fallback
 * for the quantized-matmul path (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL, Q2_K, Q3_K, Q4_K,
 * Q5_K, Q6_K, TQ1_0, TQ2_0, I2_S).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle the HIP product library
 * (libjk.so) is compared with, and the timed CPU baseline of bench.py. It is
 * never linked into, loaded by, or called from the product path.
 *
 * Every function follows one reference function; the citation (file:line,
 * relative to the reference crate root) is on its definition in jk_oracle.c.
 * Floating-point order follows the reference exactly: products and sums are
 * rounded separately (build with -ffp-contract=off), sums run in the same
 * sequence, and Rust's `Iterator<f32>::sum` is modelled as a fold that starts
 * at -0.0 (its neutral element) while explicit `let mut acc = 0.0` loops start
 * at +0.0.
 */
#ifndef JK_ORACLE_H
#define JK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the two K3Error kinds the reference returns on this path. */
enum { OR_OK = 0, OR_TENSOR_BOUNDS = 1, OR_CAPABILITY_MISMATCH = 2 };

/* GGML type ids (the reference's QuantType variants on this path). */
enum {
    OR_Q4_0 = 2,
    OR_Q4_1 = 3,
    OR_Q5_0 = 6,
    OR_Q5_1 = 7,
    OR_Q8_0 = 8,
    OR_Q2_K = 10,
    OR_Q3_K = 11,
    OR_Q4_K = 12, /* QuantType::Q4_K_M */
    OR_Q5_K = 13,
    OR_Q6_K = 14,
    OR_IQ4_NL = 20,
    OR_TQ1_0 = 34,
    OR_TQ2_0 = 35,
    OR_I2_S = 36
};

/* BlockQ8_0 (quant_q8.rs:37-44): f32 scale + 32 x i8, 36 bytes, repr(C). */
typedef struct {
    float d;
    int8_t qs[32];
} or_block_q8_0;

/* BlockQ8K (quant_q8.rs:62-72): f32 scale + 256 x i8 + 16 x i16 sums, 292 bytes. */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} or_block_q8k;

/* The fields of jero_core::TensorView that the path reads. */
typedef struct {
    int quant;
    const size_t *shape;
    size_t ndim;
    const uint8_t *bytes;
    size_t byte_len;
} or_tensor_view;

/* Logical contents of QuantizedActQ8 (repack.rs:462-486) in row-major form. */
typedef struct {
    size_t m, k, k_padded, k_blocks32, k_chunks, sb256;
    int8_t *qs;     /* [m][k_padded] */
    float *scales;  /* [m][k_blocks32]  (x_scales) */
    float *sums;    /* [m][k_blocks32]  (x_sums) */
    float *sums16;  /* [m][k_chunks]    (x_sums_16) */
    float *super256;/* [m][sb256]       (super_scales_256) */
} or_act_q8;

/* ---- format tables ---- */
size_t or_block_elements(int quant);
size_t or_block_bytes(int quant);
size_t or_scale_trailer_bytes(int quant);

/* ---- f16 ---- */
float or_f16_to_f32_ieee(uint16_t bits);
float or_f16_to_f32_finite(uint16_t bits);

/* ---- block dequant / unpack ---- */
void or_dequantize_q4_0_block(const uint8_t *blk, float *out);
void or_dequantize_q8_0_block(const uint8_t *blk, float *out);
void or_dequantize_q4_k_block(const uint8_t *blk, float *out);
void or_dequantize_q6_k_block(const uint8_t *blk, float *out);
float or_unpack_q5_0_block_i8(const uint8_t *blk, int8_t *out);
void or_dequantize_q5_0_block(const uint8_t *blk, float *out);
void or_dequantize_q5_k_block(const uint8_t *blk, float *out);
float or_unpack_tq1_0_block_i8(const uint8_t *blk, int8_t *out);
void or_dequantize_q4_1_block(const uint8_t *blk, float *out);
void or_dequantize_q5_1_block(const uint8_t *blk, float *out);
void or_unpack_q2_k_block_i8(const uint8_t *blk, int8_t *q, float *scales, float *mins);
void or_dequantize_q2_k_block(const uint8_t *blk, float *out);
void or_unpack_q3_k_block_i8(const uint8_t *blk, int8_t *q, float *scales);
void or_dequantize_q3_k_block(const uint8_t *blk, float *out);
float or_unpack_iq4_nl_block_i8(const uint8_t *blk, int8_t *out);
void or_dequantize_iq4_nl_block(const uint8_t *blk, float *out);
float or_unpack_tq2_0_block_i8(const uint8_t *blk, int8_t *out);
void or_unpack_i2_s_block_i8(const uint8_t *blk, int8_t *out);
void or_convert_i2_s_blocks_to_tq2_0(const uint8_t *blk0, const uint8_t *blk1, uint16_t scale_f16_bits,
                                     uint8_t *out);
void or_dequantize_i2_s_block(const uint8_t *blk, float scale, float *out);
float or_read_i2_s_trailer_scale(const uint8_t *trailer, size_t len);
int or_dequantize_row_bytes(int quant, const uint8_t *row, size_t row_len, size_t n_cols,
                            float *out, size_t out_len);
int or_dequantize_tensor_row(const or_tensor_view *w, size_t row, float *out, size_t out_len);

/* ---- activation quantization ---- */
int or_quantize_row_q8_0(const float *x, size_t n, or_block_q8_0 *out, size_t out_len);
int or_quantize_row_q8_k(const float *x, size_t n, or_block_q8k *out, size_t out_len);
size_t or_act_q8_bytes(size_t m, size_t k);
int or_quantize_act_q8(const float *act, size_t m, size_t k, void *storage, size_t storage_len,
                       or_act_q8 *out);
int or_subln_quantize_absmax_i8(int8_t *out, const float *in, const float *norm_w, size_t len,
                                float eps, float *scale_out);
int or_quantize_absmax_i8(int8_t *out, const float *in, size_t len, float *scale_out);

/* ---- quant_q8 integer path ---- */
int or_vec_dot_q4_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx,
                         float *out);
int or_vec_dot_q8_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx,
                         float *out);
int or_vec_dot_q4_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx,
                         float *out);
int or_vec_dot_q6_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx,
                         float *out);
int or_vec_dot_tq2_0_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx,
                          float *out);
int or_vec_dot_q5_0_q8_0(const uint8_t *w, size_t w_len, const or_block_q8_0 *x, size_t nx,
                         float *out);
int or_vec_dot_q5_k_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx,
                         float *out);
int or_vec_dot_tq1_0_q8_k(const uint8_t *w, size_t w_len, const or_block_q8k *x, size_t nx,
                          float *out);
int or_gemv_q4_0_q8_0(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8_0 *x, size_t nx);
int or_gemv_q8_0_q8_0(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8_0 *x, size_t nx);
int or_gemv_q4_k_q8_k(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8k *x, size_t nx);
int or_gemv_q6_k_q8_k(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8k *x, size_t nx);
int or_gemv_tq2_0_q8_k(float *out, size_t out_len, const or_tensor_view *w,
                       const or_block_q8k *x, size_t nx);
int or_gemv_q5_0_q8_0(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8_0 *x, size_t nx);
int or_gemv_q5_k_q8_k(float *out, size_t out_len, const or_tensor_view *w,
                      const or_block_q8k *x, size_t nx);
int or_gemv_tq1_0_q8_k(float *out, size_t out_len, const or_tensor_view *w,
                       const or_block_q8k *x, size_t nx);
/* Same computation restricted to output rows [r0, r1) (row-partitioned CPU baseline). */
int or_gemv_rows(int quant, float *out, const uint8_t *w, size_t rows, size_t cols,
                 const void *x, size_t r0, size_t r1);

/* ---- f32-activation matvec (scalar dequant + f32 dot) ---- */
int or_vec_dot_q4_0(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q8_0(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q6_k(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q4_k_m(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                      size_t in_len);
int or_vec_dot_i2_s(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q5_0(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q5_k(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q4_1(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q5_1(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q2_k(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_q3_k(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                    size_t in_len);
int or_vec_dot_iq4_nl(float *out, size_t out_len, const or_tensor_view *w, const float *in,
                      size_t in_len);

/* ---- repacked (block-scaled i8) GEMM ---- */
int or_repack_logical(const or_tensor_view *w, size_t rows, size_t cols, int8_t *q,
                      float *scales, float *mins, size_t *scale_groups_out,
                      int *has_mins_out, int *chunks_per_scale_out);
int or_gemm_repacked(float *out, size_t out_len, const or_tensor_view *w, size_t rows,
                     size_t cols, const or_act_q8 *act, size_t r0, size_t r1);
/* The product over weights already repacked by or_repack_logical (q [rows][kp], scales and
 * mins [rows][sg]; mins NULL for formats without): tokens [m0, m1) x rows [r0, r1) into out
 * [m1 - m0][r1 - r0]. */
int or_gemm_logical_rows(float *out, const int8_t *q, const float *sc, const float *mn, size_t cols, size_t sg,
                         int cps, const or_act_q8 *act, size_t m0, size_t m1, size_t r0, size_t r1);
/* PackedNibbleMatrix::gemm_rows (repack.rs:5181-5397): the compact 4-bit path for Q4_0, Q4_1,
 * IQ4_NL and Q4_K (packing, tile-scale decode and the host arm's tile dot and accumulation). */
int or_nibble_gemm_rows(float *out, size_t out_len, const or_tensor_view *w, size_t rows, size_t cols,
                        const or_act_q8 *act, size_t r0, size_t r1);

/* ---- gated activations, argmax ---- */
int or_swiglu_f32(float *out, const float *gate, const float *up, size_t n);
int or_relu_squared_gate_f32(float *out, const float *gate, const float *up, size_t n);
long or_argmax_f32(const float *x, size_t n);

/* ---- BitLinear ---- */
int or_bitlinear_i8(float *out, size_t out_len, const or_tensor_view *w, const int8_t *act,
                    size_t act_len, float act_scale);

/* ---- int8 primitives (ime.rs) ---- */
/* dot_i8_scalar (ime.rs:490-496): the sum over the min(a_len, b_len) pairs of the zip. */
int32_t or_dot_i8(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len);
/* gemm_i8_vector (ime.rs:563-583) with the sink storing c[row][n - n0]. */
void or_gemm_i8_vector(int32_t *c, const int8_t *a, size_t m, const int8_t *b, size_t n0, size_t n1, size_t k);
/* pack_tiles (ime.rs:81-94): OR_TENSOR_BOUNDS where the reference asserts (k % 16, lengths). */
int or_pack_tiles(int8_t *out, size_t out_len, const int8_t *src, size_t src_len, size_t rows, size_t k);
/* tile_dot_scalar_rows (ime.rs:127-148) */
void or_tile_dot_scalar_rows(int32_t *c, const int8_t *a, const int8_t *b, size_t k_chunks, size_t active_m);
/* gemm_i8_ime (ime.rs:449-486) off the RISC-V target: tile_dot_scalar per tile pair, the sink
 * storing tile (mt, nt) at c[(mt * (nt1 - nt0) + nt - nt0) * 64]. */
void or_gemm_i8_ime(int32_t *c, const int8_t *a_packed, size_t m_tiles, const int8_t *b_packed, size_t nt0,
                    size_t nt1, size_t k_chunks);

#ifdef __cplusplus
}
#endif
#endif
