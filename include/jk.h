/*
 * jk.h -- C ABI of the MI355X (gfx950) quantized-matmul library `libjk.so`.
 *
 * Drop-in replacement for the quant / quant_q8 / repack / BitLinear hot path of
 * jero-kernels-rvv. Every entry point below names the reference interface it
 * replaces (file:line relative to the reference crate root). Signatures are
 * plain C: pointers and sizes, no C++ or torch types.
 *
 * Two tiers:
 *  - device tier (jk_*):   weights live on the GPU in a jk_weight handle, activations
 *                          and outputs are device pointers, work is enqueued on a
 *                          stream (hipStream_t, NULL = default stream) and returns
 *                          without synchronizing;
 *  - host tier (jk_host_*): synchronous, host-memory mirrors of the reference's
 *                          signatures (copy in, launch, copy out, synchronize).
 *
 * Errors: every call validates its arguments before touching any memory and returns
 * a jk_status. JK_TENSOR_BOUNDS and JK_CAPABILITY_MISMATCH mirror
 * K3Error::TensorBoundsError / K3Error::CapabilityMismatch; jk_last_error() returns a
 * thread-local description of the most recent failure on the calling thread.
 * Outputs are fully overwritten, never accumulated into.
 *
 * Numerics: activation quantization and block dequantization are bit-exact with the
 * reference's portable scalar fallback; dot products, GEMV, GEMM and BitLinear are
 * evaluated with the reference's per-block arithmetic and its block-order f32
 * accumulation, so they are bit-exact as well. The *_tol entry points (GEMM, BitLinear,
 * f32 vec_dot) are opt-in alternatives held to 1e-5 of the output-row L2 norm instead, and
 * the int8 primitives are exact integer sums.
 */
#ifndef JK_H
#define JK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JK_ABI_VERSION 4

typedef enum jk_status {
    JK_OK = 0,
    JK_TENSOR_BOUNDS = 1,       /* K3Error::TensorBoundsError */
    JK_CAPABILITY_MISMATCH = 2, /* K3Error::CapabilityMismatch */
    JK_DEVICE_ERROR = 3         /* HIP runtime failure (no reference counterpart) */
} jk_status;

/* GGML type ids of the jero_core::QuantType variants on this path. */
typedef enum jk_quant {
    JK_Q4_0 = 2,
    JK_Q4_1 = 3,
    JK_Q5_0 = 6,
    JK_Q5_1 = 7,
    JK_Q8_0 = 8,
    JK_Q2_K = 10,
    JK_Q3_K = 11,
    JK_Q4_K = 12, /* QuantType::Q4_K_M */
    JK_Q5_K = 13,
    JK_Q6_K = 14,
    JK_IQ4_NL = 20,
    JK_TQ1_0 = 34,
    JK_TQ2_0 = 35,
    JK_I2_S = 36
} jk_quant;

/* BlockQ8_0 (quant_q8.rs:37-44): #[repr(C)] { d: f32, qs: [i8; 32] }, 36 bytes. */
typedef struct jk_block_q8_0 {
    float d;
    int8_t qs[32];
} jk_block_q8_0;

/* BlockQ8K (quant_q8.rs:62-72): #[repr(C)] { d: f32, qs: [i8; 256], bsums: [i16; 16] }, 292 bytes. */
typedef struct jk_block_q8k {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} jk_block_q8k;

/* The fields of jero_core::TensorView the path reads (name, quant, shape, bytes, offset). */
typedef struct jk_tensor_view {
    const char *name;
    int32_t quant; /* jk_quant */
    const size_t *shape;
    size_t ndim;
    const void *bytes; /* host memory */
    size_t byte_len;
    size_t offset; /* TensorView::offset: the tensor's byte offset in its file (reported in errors only) */
} jk_tensor_view;

/* QuantizedActQ8 (repack.rs:462-486) on the device, as logical row-major arrays carved
 * from one caller-owned device buffer by jk_act_q8_bind. */
typedef struct jk_act_q8 {
    size_t m, k, k_padded, k_blocks32, k_chunks, sb256;
    int8_t *qs;      /* [m][k_padded]   quantized values (repack.rs:474 tiles, untiled) */
    float *scales;   /* [m][k_blocks32] x_scales */
    float *sums;     /* [m][k_blocks32] x_sums (sequential f32 sums) */
    float *sums16;   /* [m][k_chunks]   x_sums_16 */
    float *super256; /* [m][sb256]      super_scales_256 */
} jk_act_q8;

typedef void *jk_stream; /* hipStream_t; NULL is the default stream */
typedef struct jk_weight jk_weight;

typedef struct jk_weight_info {
    int32_t quant;
    size_t rows, cols;
    size_t device_bytes; /* bytes of the device layout (GGUF bytes; 66 per 54-byte TQ1_0 block) */
    size_t gguf_bytes;   /* bytes of the GGUF payload it was built from */
} jk_weight_info;

/* K3Error's payload for the most recent failure on the calling thread. For JK_TENSOR_BOUNDS the
 * fields are TensorBoundsError's (quant.rs:403-411, repack.rs:2725-2778): tensor_name, offset,
 * byte_len, buffer_len and reason, with the values the reference puts there for the same check
 * (0 where it reports none); for the other kinds only tensor_name and reason are set. The strings
 * stay valid until the next failing call on the same thread. status is JK_OK when nothing failed. */
typedef struct jk_error_info {
    jk_status status;
    const char *tensor_name;
    size_t offset, byte_len, buffer_len;
    const char *reason;
} jk_error_info;

/* ---------------------------------------------------------------- runtime */
const char *jk_last_error(void);
jk_status jk_last_error_info(jk_error_info *out);
int jk_abi_version(void);
/* Selects the device for this thread's subsequent calls. */
jk_status jk_init(int device);
jk_status jk_stream_create(jk_stream *out);
jk_status jk_stream_destroy(jk_stream s);
jk_status jk_stream_sync(jk_stream s);
/* Plain device memory for callers that bring no allocator of their own. */
jk_status jk_device_alloc(size_t bytes, void **out);
jk_status jk_device_free(void *p);
jk_status jk_copy_to_device(jk_stream s, void *dst, const void *src, size_t bytes);
jk_status jk_copy_to_host(jk_stream s, void *dst, const void *src, size_t bytes);

/* ---------------------------------------------------------------- weights */
/* RepackedWeight::from_tensor (repack.rs:2288-2300) / RepackedWeight::repack when
 * rows == cols == 0 (repack.rs:2255-2285): copies the GGUF payload to the device and
 * rewrites it there into the plane layout (same byte count as GGUF, except TQ1_0, whose
 * trits are stored 2 bits each, and Q3_K, padded from 110 to 112 bytes). Formats: Q4_0, Q4_1,
 * Q5_0, Q5_1, Q8_0, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, TQ1_0, TQ2_0, I2_S (the formats of
 * BlockScaledTileLayout::for_tensor, repack.rs:1308-1333, and so of PackedNibbleMatrix,
 * repack.rs:4788); others are a CapabilityMismatch. Validation follows validate_matrix_view
 * (repack.rs:1208-1281). The handle is immutable and may be used from any thread and
 * stream once the upload stream has completed. */
jk_status jk_weight_upload(jk_stream s, const jk_tensor_view *w, size_t rows, size_t cols,
                           jk_weight **out);
jk_status jk_weight_free(jk_weight *w);
jk_status jk_weight_get_info(const jk_weight *w, jk_weight_info *out);

/* BlockScaledTileLayout (repack.rs:1286-1449): the tile-grid geometry of a weight, as
 * RepackedWeight::block_scaled_layout (repack.rs:2372) / BlockScaledTileLayout::for_tensor
 * (repack.rs:1308) compute it. The reference's buffer lengths are reported for callers that
 * size work by them; device_bytes is what jk_weight_create allocates (the plane layout). */
typedef struct jk_weight_layout {
    int32_t quant;
    size_t rows, cols, row_bytes, k_padded;
    size_t n_tiles;          /* rows.div_ceil(8) */
    size_t k_chunks;         /* k_padded / 16 */
    size_t chunks_per_scale; /* 1 for Q6_K / Q3_K / Q2_K, else 2 */
    size_t scale_groups;     /* k_chunks / chunks_per_scale */
    int32_t has_mins;        /* Q4_K, Q5_K, Q4_1, Q5_1, Q2_K */
    size_t total_tiles, total_scales, total_mins;
    size_t device_bytes, gguf_bytes;
    float tensor_scale; /* I2_S: the trailer's per-tensor scale (read_i2_s_trailer_scale), else 0 */
} jk_weight_layout;
/* Same formats and validation as jk_weight_upload with explicit rows, cols (no orientation
 * inference, as for_tensor). */
jk_status jk_weight_layout_for(const jk_tensor_view *w, size_t rows, size_t cols, jk_weight_layout *out);
/* The allocation half of RepackedWeight::from_tile_buffers (repack.rs:2386-2450): a device
 * handle for layout whose planes are zero (all-zero blocks) until tile ranges are written. */
jk_status jk_weight_create(jk_stream s, const jk_weight_layout *layout, jk_weight **out);
/* repack_into_tile_range (repack.rs:1579-1650): repacks the 8-row tiles [tile_begin, tile_end)
 * of w's GGUF bytes (the whole tensor view, as in the reference; only those rows are copied)
 * into the handle on the device. The view must be the one the layout was computed from (same
 * format and dimensions; for I2_S the same trailer scale). Returns once the host bytes are no
 * longer read. Calls for disjoint tile ranges may run concurrently from several host threads
 * (each on its own stream); an empty range is a no-op. */
jk_status jk_weight_upload_tile_range(jk_stream s, jk_weight *w, const jk_tensor_view *view, size_t tile_begin,
                                      size_t tile_end);
/* The same from GGUF bytes already in device memory: gguf holds exactly the rows of tiles
 * [tile_begin, tile_end) (row_bytes each; the last tile may be partial). Allocates nothing
 * and does not synchronize: gguf must stay valid until the stream reaches the repack. */
jk_status jk_weight_repack_tile_range(jk_stream s, jk_weight *w, const void *gguf, size_t gguf_len,
                                      size_t tile_begin, size_t tile_end);
/* The validation half of from_tile_buffers: fails (TensorBounds) unless every tile has been
 * written, then makes the handle usable by the compute entry points (which refuse an unsealed
 * handle) and immutable (further tile writes are refused). The tile bookkeeping is host-side:
 * work on another stream must wait for the streams that wrote the tiles (an event, or a
 * synchronize), as after jk_weight_create's own stream. */
jk_status jk_weight_seal(jk_weight *w);

/* ------------------------------------------------------------------ GGUF */
/* GGUF v2 / v3 files, memory-mapped and bounds-checked. The reference reads its weights as
 * jero_core::TensorView byte slices of such a file (dims [ne0, ne1] = [cols, rows]); no
 * reference function corresponds to the reader itself. ggml type ids are the jk_quant values. */
typedef struct jk_gguf jk_gguf;
typedef struct jk_gguf_file_info {
    uint32_t version;
    size_t n_tensors, n_kv;
    size_t alignment;   /* general.alignment, default 32 */
    size_t data_offset; /* file offset of the tensor data section */
    size_t file_bytes;
} jk_gguf_file_info;
typedef struct jk_gguf_tensor {
    const char *name; /* valid until jk_gguf_close */
    uint32_t ggml_type;
    uint32_t n_dims;
    uint64_t ne[4];      /* ne[0] is the contiguous (column) dimension */
    size_t offset;       /* file offset of the data */
    size_t nbytes;       /* 0 when the type's size is not known to this library */
    const void *data;    /* the mapped bytes (NULL when nbytes is 0); valid until jk_gguf_close */
} jk_gguf_tensor;
jk_status jk_gguf_open(const char *path, jk_gguf **out);
jk_status jk_gguf_close(jk_gguf *g);
jk_status jk_gguf_get_file_info(const jk_gguf *g, jk_gguf_file_info *out);
jk_status jk_gguf_tensor_info(const jk_gguf *g, size_t index, jk_gguf_tensor *out);
jk_status jk_gguf_find(const jk_gguf *g, const char *name, size_t *index);
/* RepackedWeight::from_tensor of a 2D tensor of the file, assembled as from_tile_buffers from
 * tile ranges (repack.rs:1579, 2386): rows are streamed in chunks of about chunk_bytes (0: 32
 * MiB) through two pinned host buffers, copied out of the mapping by several host threads while
 * the previous chunk is transferred and repacked on stream s. The result is the handle
 * jk_weight_upload makes of the same bytes; returns once it is complete and sealed. The
 * streaming buffers (2 x chunk pinned host + 2 x chunk device) stay with the file handle for
 * the next load until jk_gguf_close; loads through one file handle are serialized. */
jk_status jk_gguf_load_weight(jk_stream s, const jk_gguf *g, size_t index, size_t chunk_bytes, jk_weight **out);
/* dequantize_tensor_row (quant.rs:2492-2568) over output rows [row_begin, row_end):
 * out[(row - row_begin) * cols + col], bit-exact with the GGUF block dequantizers.
 * RepackedWeight::dequantize_row (repack.rs:2529-2598) agrees up to the sign of zero. */
jk_status jk_weight_dequantize_rows(jk_stream s, const jk_weight *w, size_t row_begin,
                                    size_t row_end, float *out, size_t out_len);

/* ------------------------------------------------- activation quantization */
/* quantize_row_q8_0 (quant_q8.rs:395) over n = out_blocks * 32 values (any number of
 * rows laid end to end). */
jk_status jk_quantize_row_q8_0(jk_stream s, const float *x, size_t n, jk_block_q8_0 *out,
                               size_t out_blocks);
/* quantize_row_q8_k (quant_q8.rs:576-594). */
jk_status jk_quantize_row_q8_k(jk_stream s, const float *x, size_t n, jk_block_q8k *out,
                               size_t out_blocks);
/* Device bytes that jk_act_q8_bind needs for an [m, k] batch. */
size_t jk_act_q8_bytes(size_t m, size_t k);
jk_status jk_act_q8_bind(void *storage, size_t storage_len, size_t m, size_t k, jk_act_q8 *out);
/* QuantizedActQ8::quantize_into (repack.rs:542-650). */
jk_status jk_quantize_act_q8(jk_stream s, const float *x, size_t m, size_t k, const jk_act_q8 *act);
/* subln_quantize_absmax_i8 (lib.rs:1042-1101) applied to each of m rows:
 * q[m][k], scales[m]. */
jk_status jk_subln_quantize_absmax_i8(jk_stream s, const float *x, const float *norm_w,
                                      size_t m, size_t k, float eps, int8_t *q, float *scales);
/* The same per-token absmax recipe (lib.rs:1072-1098) without the RMSNorm step. */
jk_status jk_quantize_absmax_i8(jk_stream s, const float *x, size_t m, size_t k, int8_t *q,
                                float *scales);

/* ---------------------------------------------- quant_q8 integer GEMV (M=1) */
/* gemv_q4_0_q8_0 (quant_q8.rs:1586-1605), gemv_q5_0_q8_0 (1628-1650), gemv_q8_0_q8_0
 * (1670-1689), gemv_q4_k_q8_k (3101-3123), gemv_q5_k_q8_k (3160-3182), gemv_q6_k_q8_k
 * (3189-3211), gemv_tq1_0_q8_k (3219-3242), gemv_tq2_0_q8_k (3250-3273): y[rows] from the
 * weight handle and nx pre-quantized activation blocks. */
jk_status jk_gemv_q4_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_q8_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_q4_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_q6_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_tq2_0_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx,
                             float *y, size_t y_len);
jk_status jk_gemv_q5_0_q8_0(jk_stream s, const jk_weight *w, const jk_block_q8_0 *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_q5_k_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx,
                            float *y, size_t y_len);
jk_status jk_gemv_tq1_0_q8_k(jk_stream s, const jk_weight *w, const jk_block_q8k *x, size_t nx,
                             float *y, size_t y_len);
/* Row-sliced form of the eight above (format taken from the handle): writes
 * y[row - row_begin] for rows [row_begin, row_end), identical to the full call. */
jk_status jk_gemv_q8_rows(jk_stream s, const jk_weight *w, const void *x, size_t nx, float *y,
                          size_t row_begin, size_t row_end);

/* Grouped quant_q8 GEMV: one launch evaluates several independent products of one
 * weight format (e.g. a layer's Q/K/V projections, or gate and up). Each job is a
 * gemv_* call of the eight above over rows [row_begin, row_end) of its weight, writing
 * y[row - row_begin]; its activation is either caller blocks (x_q8: BlockQ8_0 for
 * Q4_0/Q5_0/Q8_0, BlockQ8K for the 256-element formats) or f32 values (x_f32) that the launch
 * quantizes with quantize_row_q8_0 / quantize_row_q8_k (quant_q8.rs:395, 576) -- results
 * are identical either way. Jobs of different formats are split into separate launches.
 * No single reference function corresponds: this is the reference's per-matrix sequence
 * (quantize_row_q8_k, then gemv_q4_k_q8_k per matrix) batched into one launch. */
typedef struct jk_gemv_job {
    const jk_weight *w;
    const void *x_q8;
    const float *x_f32;
    float *y;
    size_t row_begin, row_end;
} jk_gemv_job;
jk_status jk_gemv_q8_batch(jk_stream s, const jk_gemv_job *jobs, size_t njobs);
/* quantize_row_q8_0 / quantize_row_q8_k (quant_q8.rs:395, 576) of x followed by the
 * matching gemv_* (quant_q8.rs:1586-3273) in one launch: y[rows] from f32 x[cols]. */
jk_status jk_gemv_q8_f32(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y, size_t y_len);

/* ------------------------------------------ f32-activation matvec (vec_dot) */
/* vec_dot_q4_0 (quant.rs:1458), vec_dot_q4_1 (2062), vec_dot_q5_0 (2036), vec_dot_q5_1
 * (2081), vec_dot_q8_0 (1069), vec_dot_iq4_nl (2138), vec_dot_q2_k (2100), vec_dot_q3_k
 * (2119), VectorKernel::vec_dot_q4_k_m (lib.rs:157, scalar impl 1268-1303), vec_dot_q5_k
 * (quant.rs:1238), vec_dot_q6_k (1089), vec_dot_i2_s (2199-2240): dequantize each block
 * and dot it with f32 x. TQ1_0 / TQ2_0 have none (CapabilityMismatch). */
jk_status jk_vec_dot_f32(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y,
                         size_t y_len);
/* The same products in tolerance mode: the same arguments, validation and errors as
 * jk_vec_dot_f32, with each block's element products added over four fused multiply-add
 * accumulators instead of the reference's one product and one add per element in element
 * order; every output within 1e-5 of its row's L2 norm of the reference's result. No
 * reference function has this rounding: it is jk_vec_dot_f32's alternative. */
jk_status jk_vec_dot_f32_tol(jk_stream s, const jk_weight *w, const float *x, size_t n, float *y,
                             size_t y_len);

/* ----------------------------------------------------- repacked GEMV / GEMM */
/* Every format of jk_weight_upload. PackedNibbleMatrix::gemm / gemm_rows / gemv
 * (repack.rs:4945-4985) compute the same products for its formats (Q4_0, Q4_1, IQ4_NL,
 * Q4_K) and map to these calls on a handle from jk_weight_upload.
 * gemm_repacked_rows (repack.rs:4087-4094) / RepackedWeight::gemm_rows (2661-2668):
 * y[m][row - row_begin] for rows [row_begin, row_end), y_len = m * (row_end - row_begin).
 * gemv_repacked_rows (repack.rs:4014-4061) is the m == 1 case. */
jk_status jk_gemm_repacked(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y,
                           size_t y_len, size_t row_begin, size_t row_end);
/* gemm_repacked_rows (repack.rs:4087-4094) in tolerance mode: the same arguments, validation and
 * errors as jk_gemm_repacked, with each scale group's exact integer partial applied by one fused
 * multiply-add (acc = fma(partial, xs * ws, acc); formats with mins add -(xsum * wm) as one more
 * rounded step) instead of the reference's separately rounded product and sum. Every output is
 * within 1e-5 of its token's output-row L2 norm of the bit-exact result (the tolerance the port
 * is held to for f32 products). From 1.5 128 x 128 tiles per CU on (14336 rows: 448 tokens), the
 * 32-element-group formats run larger tiles with fewer VALU operations per scale group, about
 * 1.2x the throughput of jk_gemm_repacked; Q8_0 there applies each group as
 * fma(B + partial, ws * xs, acc - B * ws * xs) with B = 1.5 * 2^23 (the second product accumulated on
 * the matrix core), so a scale product |ws * xs| above 2^104 can overflow to infinity where the
 * bit-exact call stays finite. Q6_K and Q3_K combine a step's two 16-element groups in integers;
 * Q2_K, and launches where the bit-exact tiles measured faster, run the bit-exact kernels (whose
 * results meet the bar by definition). No reference function has this rounding: it is the
 * bit-exact call's alternative. */
jk_status jk_gemm_repacked_tol(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y,
                               size_t y_len, size_t row_begin, size_t row_end);
/* gemv_repacked_view_rows (repack.rs:4045-4061): requires act->m == 1. */
jk_status jk_gemv_repacked(jk_stream s, const jk_weight *w, const jk_act_q8 *act, float *y,
                           size_t y_len, size_t row_begin, size_t row_end);

/* --------------------------------- the step after the products (epilogues) */
/* Gated activations of a feed-forward block: out = act(gate) * up elementwise. */
typedef enum jk_act {
    JK_ACT_SWIGLU = 1, /* swiglu_f32 (swiglu.rs:62-121): gate / (1 + exp(-gate)) * up, 0 below -20, gate above 20 */
    JK_ACT_RELU2 = 2   /* relu_squared_gate_f32 (lib.rs:1111-1147): max(gate, 0)^2 * up */
} jk_act;
/* swiglu_f32 (swiglu.rs:62), relu_squared_gate_f32 (lib.rs:1111) over n device values. SwiGLU
 * uses the device's single-precision exp: results agree with the reference within the
 * reference's own tolerance for its vector path (max(1e-6, 1e-5 |y|)); ReLU^2 is bit-exact. */
jk_status jk_swiglu_f32(jk_stream s, const float *gate, const float *up, size_t n, float *out);
jk_status jk_relu_squared_gate_f32(jk_stream s, const float *gate, const float *up, size_t n, float *out);
/* The activation fused into the next product's activation quantizer: quantize_row_q8_k
 * (quant_q8.rs:576) / QuantizedActQ8::quantize_into (repack.rs:542) of act(gate, up), without
 * writing the intermediate. Identical to jk_swiglu_f32 / jk_relu_squared_gate_f32 followed by
 * jk_quantize_row_q8_k / jk_quantize_act_q8 (no reference counterpart for the fusion itself). */
jk_status jk_quantize_row_q8_k_gated(jk_stream s, int act, const float *gate, const float *up, size_t n,
                                     jk_block_q8k *out, size_t out_blocks);
jk_status jk_quantize_act_q8_gated(jk_stream s, int act, const float *gate, const float *up, size_t m, size_t k,
                                   const jk_act_q8 *act_q8);
/* argmax_f32 (lib.rs:662, scalar recipe 555-568): *index = the lowest index of the largest
 * non-NaN value, -1 when x is empty or all NaN (Option::None). The device workspace holds one
 * 8-byte partial result per workgroup: at least jk_argmax_workspace_bytes(n) bytes, 8-byte
 * aligned, needing no initialization (each call overwrites what it reads). Calls that share a
 * workspace must not overlap (same stream, or synchronized). */
size_t jk_argmax_workspace_bytes(size_t n);
jk_status jk_argmax_f32(jk_stream s, const float *x, size_t n, int32_t *index, void *workspace,
                        size_t workspace_bytes);
/* A quant_q8 GEMV (as jk_gemv_q8_f32 with x_f32, or the format's jk_gemv_* with caller blocks
 * x_q8 of x_len blocks) with argmax_f32 of its output fused into the GEMV's store phase: each
 * workgroup reduces the rows it wrote and one small launch after it reduces the workgroups, so
 * *index = argmax of y, computed from the same bits; y may be NULL when only the index is wanted
 * (a greedy lm_head step). Exactly one of x_q8 / x_f32 is set; x_len counts its blocks or
 * values. The workspace is as for jk_argmax_f32 with n = the weight's rows. No single reference
 * function corresponds: gemv_* followed by argmax_f32. */
jk_status jk_gemv_q8_argmax(jk_stream s, const jk_weight *w, const void *x_q8, const float *x_f32, size_t x_len,
                            float *y, int32_t *index, void *workspace, size_t workspace_bytes);
/* jk_gemv_q8_argmax without a workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc); it has no
 * counterpart in the reference. The argmax slots live in a static array of the library, one
 * copy per GPU (about 2 MiB, held until the process ends), so the weight may have at most
 * 262144 output rows (JK_TENSOR_BOUNDS beyond). The call allocates nothing. Calls on one GPU
 * share that array: calls that overlap on one GPU (other streams, unordered host threads)
 * race and must not be issued; each call overwrites every slot it reads. Results are those of
 * jk_gemv_q8_argmax. */
jk_status jk_gemv_q8_argmax_noalloc(jk_stream s, const jk_weight *w, const void *x_q8, const float *x_f32,
                                    size_t x_len, float *y, int32_t *index);

/* -------------------------------------------------------------- BitLinear */
/* bitlinear_i8_rvv (ime.rs:882-938) applied to m tokens: y[m][rows] from act[m][k]
 * and one f32 scale per token (TQ1_0, TQ2_0, I2_S and Q8_0 weights). */
jk_status jk_bitlinear_i8(jk_stream s, const jk_weight *w, const int8_t *act,
                          const float *act_scales, size_t m, size_t k, float *y, size_t y_len);
/* bitlinear_i8_rvv (ime.rs:882-938) for m tokens in tolerance mode: the same arguments,
 * validation and errors as jk_bitlinear_i8, with the per-block addends summed in any order --
 * every output within 1e-5 of its token's output-row L2 norm of the reference's block-order
 * sum. From 16 tokens on, TQ2_0 / TQ1_0 / I2_S weights with 16-byte aligned activation rows run
 * K split over the waves of a workgroup: I2_S sums the whole row in exact integers and rounds
 * once (f32(sum) * (scale * act_scale)), TQ2_0 adds one fused multiply-add per 256-element
 * block. Other cases run the bit-exact kernels. No reference function has this rounding: it is
 * the bit-exact call's alternative, as jk_gemm_repacked_tol is jk_gemm_repacked's. */
jk_status jk_bitlinear_i8_tol(jk_stream s, const jk_weight *w, const int8_t *act,
                              const float *act_scales, size_t m, size_t k, float *y, size_t y_len);

/* convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790) on the device over a run of block pairs: TQ2_0
 * block k (66 bytes, crate layout: the f16 scale bits, then 64 bytes of 2-bit fields t + 1) holds
 * the 256 trits of I2_S blocks 2k and 2k + 1 (32 bytes each). i2s_blocks must be 2 * tq2_blocks. */
jk_status jk_convert_i2_s_to_tq2_0(jk_stream s, const void *i2s, size_t i2s_blocks, uint16_t scale_f16_bits,
                                   void *tq2, size_t tq2_blocks);

/* ------------------------------------------------------- int8 primitives */
/* Exact i32 results on the int8 matrix cores, equal to the reference's while no sum overflows
 * i32: k (or 16 * k_chunks) is at most 131071, JK_TENSOR_BOUNDS beyond. Device pointers; a slice
 * shorter than its indexing needs (a panic in the reference) is JK_TENSOR_BOUNDS. */
/* gemm_i8_vector (ime.rs:563-583): C = A * B^T for the rows n0..n1 of B. a: m x k row-major
 * (a_len >= m * k), b: row-major rows of k (b_len >= n1 * k); c[row][n - n0], m x (n1 - n0),
 * receives what the reference's sink(row, n, value) gets. Adds m * (n1 - n0) to the vector-dot
 * counter. Any k and alignment; k a multiple of 16 with 16-byte aligned a and b is fastest. */
jk_status jk_gemm_i8(jk_stream s, const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0,
                     size_t n1, size_t k, int32_t *c, size_t c_len);
/* gemm_i8_ime (ime.rs:449-486) on pack_tiles layouts: a_packed holds m_tiles tile rows and
 * b_packed at least nt1, each k_chunks 128-byte tiles of 8 rows x 16 (16-byte aligned); c receives
 * the 8 x 8 tile (mt, nt) of sink(mt, nt, tile) at c[(mt * (nt1 - nt0) + nt - nt0) * 64 ..], row i of A
 * and row j of B at i * 8 + j. Adds m_tiles * (nt1 - nt0) * k_chunks to the matrix tile counter,
 * as the reference adds one 8 x 8 x 16 tile step per chunk. */
jk_status jk_gemm_i8_tiles(jk_stream s, const int8_t *a_packed, size_t a_len, size_t m_tiles, const int8_t *b_packed,
                           size_t b_len, size_t nt0, size_t nt1, size_t k_chunks, int32_t *c, size_t c_len);
/* pack_tiles (ime.rs:81-94): rows x k row-major (src_len == rows * k, k a multiple of 16) into
 * [row_tile][k_chunk][8][16], rows past the last zero-filled; dst_len == tile_count(rows) * (k / 16) * 128. */
jk_status jk_pack_tiles_i8(jk_stream s, const int8_t *src, size_t src_len, size_t rows, size_t k, int8_t *dst,
                           size_t dst_len);
/* dot_i8_vector (ime.rs:548-557): *out = sum of a[i] * b[i] over the min(a_len, b_len) pairs of the
 * two slices (the reference zips them); 0 for none. */
jk_status jk_dot_i8(jk_stream s, const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, int32_t *out);
/* ime_vmadot_count / vector_dot_count (ime.rs:53-66): monotonic per-process counters. The first
 * counts 8 x 8 x 16 tile steps of jk_gemm_i8_tiles; the second the dot products of jk_gemm_i8 and of
 * the BitLinear entry points (one per weight block and token, as bitlinear_i8_rvv counts). Counted
 * when a launch is issued. Either pointer may be NULL. */
void jk_op_counts(uint64_t *matrix_tile_steps, uint64_t *vector_dots);

/* ------------------------------------------- host tier (synchronous mirrors) */
/* The jk_host_* mirrors run on a per-thread stream and per-thread device scratch (grown on
 * demand, kept until jk_host_release_thread). By default every call uploads its weight, as the
 * reference reads a slice's bytes on every call. Residency is opt in: after
 * jk_host_cache_set_limit(bytes > 0) a view is uploaded once, keyed by its byte range, format,
 * shape and a fingerprint of sampled bytes, and later calls with it perform no upload and no
 * allocation (tests/wave4_zero_alloc_gemv.rs:88+ is the reference's zero-allocation contract for
 * these paths). With the cache on, the bytes behind a cached view must not change while it is
 * cached: after changing or freeing them call jk_host_cache_invalidate (or jk_host_cache_clear).
 * jk_host_cache_set_verify(1) removes that obligation at a cost: every hit hashes all of the
 * view's bytes (a few ms for a 33 MB matrix) and, if they changed since the upload, drops the
 * entry and uploads again (counted in stale_reuploads); setting it clears the cache. Entries
 * beyond the byte limit are evicted least recently used. No reference function corresponds to
 * this control surface. */
typedef struct jk_host_stats {
    uint64_t weight_uploads;  /* views uploaded (cache misses, and every call with the cache off) */
    uint64_t cache_hits;      /* calls served by a resident weight */
    uint64_t cache_evictions;
    uint64_t device_allocs;   /* device allocations made by the host tier (uploads and scratch growth) */
    uint64_t cached_weights, cached_bytes, cache_limit;
    uint64_t stale_reuploads; /* verify mode: hits whose bytes had changed, uploaded again */
    uint64_t verify;          /* 1 while jk_host_cache_set_verify(1) is in effect */
} jk_host_stats;
jk_status jk_host_cache_set_limit(size_t bytes);
/* Drops every cached weight whose view overlaps [bytes, bytes + len). */
jk_status jk_host_cache_invalidate(const void *bytes, size_t len);
jk_status jk_host_cache_clear(void);
jk_status jk_host_cache_set_verify(int on);
jk_status jk_host_get_stats(jk_host_stats *out);
/* Frees the calling thread's host-tier stream and scratch. */
jk_status jk_host_release_thread(void);

/* quantize_row_q8_0 (quant_q8.rs:395), quantize_row_q8_k (576). */
jk_status jk_host_quantize_row_q8_0(const float *x, size_t n, jk_block_q8_0 *out, size_t out_len);
jk_status jk_host_quantize_row_q8_k(const float *x, size_t n, jk_block_q8k *out, size_t out_len);
/* vec_dot_q4_0_q8_0 (quant_q8.rs:1463), vec_dot_q8_0_q8_0 (1493), vec_dot_q4_k_q8_k (3019),
 * vec_dot_q6_k_q8_k (3056), vec_dot_tq2_0_q8_k (3086): one row of blocks -> *out. */
jk_status jk_host_vec_dot_q4_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out);
jk_status jk_host_vec_dot_q8_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out);
jk_status jk_host_vec_dot_q4_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out);
jk_status jk_host_vec_dot_q6_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out);
jk_status jk_host_vec_dot_tq2_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out);
/* vec_dot_q5_0_q8_0_blocks (quant_q8.rs:1478), vec_dot_q5_k_q8_k (3041), vec_dot_tq1_0_q8_k (3071). */
jk_status jk_host_vec_dot_q5_0_q8_0(const void *w, size_t w_len, const jk_block_q8_0 *x, size_t nx, float *out);
jk_status jk_host_vec_dot_q5_k_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out);
jk_status jk_host_vec_dot_tq1_0_q8_k(const void *w, size_t w_len, const jk_block_q8k *x, size_t nx, float *out);
/* gemv_q4_0_q8_0 (quant_q8.rs:1586) ... gemv_tq2_0_q8_k (3250) with a TensorView. */
jk_status jk_host_gemv_q4_0_q8_0(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx);
jk_status jk_host_gemv_q8_0_q8_0(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx);
jk_status jk_host_gemv_q4_k_q8_k(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx);
jk_status jk_host_gemv_q6_k_q8_k(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx);
jk_status jk_host_gemv_tq2_0_q8_k(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx);
/* gemv_q5_0_q8_0 (quant_q8.rs:1628), gemv_q5_k_q8_k (3160), gemv_tq1_0_q8_k (3219). */
jk_status jk_host_gemv_q5_0_q8_0(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8_0 *x, size_t nx);
jk_status jk_host_gemv_q5_k_q8_k(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx);
jk_status jk_host_gemv_tq1_0_q8_k(float *out, size_t out_len, const jk_tensor_view *w, const jk_block_q8k *x, size_t nx);
/* vec_dot_q4_0 (quant.rs:1458), vec_dot_q8_0 (1069), vec_dot_q6_k (1089),
 * VectorKernel::vec_dot_q4_k_m (lib.rs:157), vec_dot_i2_s (quant.rs:2199). */
jk_status jk_host_vec_dot_q4_0(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q8_0(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q6_k(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q4_k_m(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_i2_s(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
/* vec_dot_q5_0 (quant.rs:2036), vec_dot_q5_k (1238), vec_dot_q4_1 (2062), vec_dot_q5_1 (2081),
 * vec_dot_q2_k (2100), vec_dot_q3_k (2119), vec_dot_iq4_nl (2138). */
jk_status jk_host_vec_dot_q5_0(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q5_k(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q4_1(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q5_1(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q2_k(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_q3_k(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
jk_status jk_host_vec_dot_iq4_nl(float *out, size_t out_len, const jk_tensor_view *w, const float *in, size_t in_len);
/* dequantize_tensor_row / dequantize_token_row (quant.rs:2492, 2580). */
jk_status jk_host_dequantize_tensor_row(const jk_tensor_view *w, size_t row, float *out, size_t out_len);
/* gemm_repacked_f32_rows (repack.rs:4143-4165): quantizes input [m, cols] with
 * QuantizedActQ8 semantics, then the repacked GEMM; out[m][row_end - row_begin]. */
jk_status jk_host_gemm_repacked_f32(float *out, size_t out_len, const jk_weight *w, const float *input,
                                   size_t m, size_t row_begin, size_t row_end);
/* swiglu_f32 (swiglu.rs:62), relu_squared_gate_f32 (lib.rs:1111), argmax_f32 (lib.rs:662;
 * *index = -1 for None) on host slices. */
jk_status jk_host_swiglu_f32(float *out, size_t out_len, const float *gate, size_t gate_len, const float *up,
                             size_t up_len);
jk_status jk_host_relu_squared_gate_f32(float *out, size_t out_len, const float *gate, size_t gate_len,
                                        const float *up, size_t up_len);
jk_status jk_host_argmax_f32(const float *x, size_t n, int64_t *index);
/* convert_i2_s_blocks_to_tq2_0 (ime.rs:767-790): blk0 and blk1 are 32 bytes, out 66 bytes. */
jk_status jk_host_convert_i2_s_blocks_to_tq2_0(const uint8_t *blk0, const uint8_t *blk1, uint16_t scale_f16_bits,
                                               uint8_t *out);
/* bitlinear_i8_rvv (ime.rs:882-938). */
jk_status jk_host_bitlinear_i8(float *out, size_t out_len, const jk_tensor_view *w, const int8_t *act,
                               size_t act_len, float act_scale);
/* gemm_i8_vector (ime.rs:563-583) and dot_i8_vector (ime.rs:548-557) on host slices: the arguments,
 * checks and results of jk_gemm_i8 / jk_dot_i8 (c[row][n - n0]; the zip of the two slices). */
jk_status jk_host_gemm_i8(const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0,
                          size_t n1, size_t k, int32_t *c, size_t c_len);
jk_status jk_host_dot_i8(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, int32_t *out);

/* ---------------------------------------------------------------- measurement */

/* A plain streaming read of `bytes` (a non-zero multiple of 16, 16-byte aligned) of device
 * memory: coalesced 16-byte non-temporal loads, one-shot 256-thread workgroups of 32 KB each,
 * nothing written (sink is a 4-byte device word that is stored only if the xor of everything
 * read equals a fixed constant). It is the ceiling the GEMV launches are measured against:
 * the same byte count read once on the same launch path. No counterpart in the reference. */
jk_status jk_measure_stream_read(jk_stream s, const void *buf, size_t bytes, uint32_t *sink);

/* Which kernel a call would launch, as a static string in *kernel, found by running the
 * launcher with the launch recorded instead of made (nothing is enqueued; the arguments are
 * validated as the call itself validates them). jk_gemm_plan: jk_gemm_repacked (tolerance 0)
 * or jk_gemm_repacked_tol (1) of `act` against rows [row_begin, row_end) of w (*kernel NULL
 * for an empty range). jk_bitlinear_plan: jk_bitlinear_i8 (tolerance 0) or jk_bitlinear_i8_tol (1)
 * of m tokens whose rows start at act.
 * For tests and benchmarks; no counterpart in the reference. */
jk_status jk_gemm_plan(const jk_weight *w, const jk_act_q8 *act, size_t row_begin, size_t row_end, int tolerance,
                       const char **kernel);
jk_status jk_bitlinear_plan(const jk_weight *w, const int8_t *act, size_t m, int tolerance, const char **kernel);

#ifdef __cplusplus
}
#endif
#endif /* JK_H */
