// jk_internal.hpp -- shared host/device definitions of libjk (gfx950 only).
//
// Device weight layout ("plane layout"). A GGUF block of a row is cut into C
// 16-byte chunks; chunk c of block b of row r lives in plane c at
//     planes + ((c * rows + r) * nb + b) * 16
// and the block's f16 scale, when it is not inside a chunk, lives in the scale
// plane at dplane[r * nb + b]; a 4- or 8-byte field that is neither (high bits,
// d / m pairs) lives in the word plane, hplane[(r * nb + b) * h_len / 4 ..]. Lanes
// that walk consecutive blocks of one row therefore read consecutive 16-byte
// chunks (one coalesced 128-bit load per lane per plane), and the layout holds
// exactly the GGUF bytes (Q3_K: 2 bytes of padding in its last chunk):
//
//   format  block  bytes  chunks (16 B)                         scale  word
//   Q4_0     32     18    qs[0..16)                             d      -
//   Q4_1     32     20    qs[0..16)                             -      d m
//   Q5_0     32     22    qs[0..16)                             d      qh
//   Q5_1     32     24    qs[0..16)                             -      d m qh
//   Q8_0     32     34    qs[0..16), qs[16..32)                 d      -
//   IQ4_NL   32     18    qs[0..16)                             d      -
//   Q2_K    256     84    scales16, qs x4                       -      d dmin
//   Q3_K    256    110    hmask x2, qs x4, [scales12 d 0 0]     -      -
//   Q4_K    256    144    [d dmin scales12], qs[16c..16c+16)    -      -
//   Q5_K    256    176    [d dmin scales12], qh x2, qs x8       -      -
//   Q6_K    256    210    ql x8, qh x4, scales x1               d      -
//   TQ2_0   256     66    qs x4 (2-bit fields transposed 4x4    d      -
//                         inside every dword, see below)
//   I2_S    128     32    bytes[0..16), bytes[16..32)           - (tensor scale)
//
// TQ2_0 transposition: GGUF byte i of a dword holds elements 4i+j in bits 2j.
// The device dword holds element 4j+i in bits 2j of byte i, so that
// (w >> 2j) & 0x03030303 is the four elements of activation dword j.
//
// TQ1_0 (54 bytes: d, then base-3 digits, five per byte) is the one format that is
// re-encoded at upload: its trits are decoded once and stored in the TQ2_0 device
// layout (66 bytes per block), which every kernel then reads as TQ2_0. The two
// formats have the same arithmetic on every entry point (the TQ1_0 and TQ2_0 arms
// of the reference differ only in how the trits are unpacked); decoding five base-3
// digits per byte in the kernels would cost about twice the VALU budget that
// streaming the 54-byte blocks at full HBM bandwidth leaves.
#pragma once

#include <atomic>
#include <mutex>
#include <string>
#include <vector>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/jk.h"

namespace jk {

struct Fmt {
    int quant;
    int be;      // elements per block
    int bb;      // GGUF bytes per block
    int chunks;  // 16-byte chunks per block in the planes
    int d_off;   // byte offset of the f16 scale inside the GGUF block, -1 if none
    int q_off;   // byte offset of chunk 0 inside the GGUF block
    int h_off;   // byte offset of the word-plane field inside the GGUF block, -1 if none
    int h_len;   // bytes of the word-plane field (4 or 8)
};

// Device layout of each GGUF format (TQ1_0: the GGUF block geometry; its device
// layout is TQ2_0's, see dev_quant).
__host__ __device__ constexpr Fmt fmt_of(int q) {
    return q == JK_Q4_0    ? Fmt{JK_Q4_0, 32, 18, 1, 0, 2, -1, 0}
           : q == JK_Q4_1   ? Fmt{JK_Q4_1, 32, 20, 1, -1, 4, 0, 4}
           : q == JK_Q5_0   ? Fmt{JK_Q5_0, 32, 22, 1, 0, 6, 2, 4}
           : q == JK_Q5_1   ? Fmt{JK_Q5_1, 32, 24, 1, -1, 8, 0, 8}
           : q == JK_Q8_0   ? Fmt{JK_Q8_0, 32, 34, 2, 0, 2, -1, 0}
           : q == JK_IQ4_NL ? Fmt{JK_IQ4_NL, 32, 18, 1, 0, 2, -1, 0}
           : q == JK_Q2_K   ? Fmt{JK_Q2_K, 256, 84, 5, -1, 0, 80, 4}
           : q == JK_Q3_K   ? Fmt{JK_Q3_K, 256, 110, 7, -1, 0, -1, 0}
           : q == JK_Q4_K   ? Fmt{JK_Q4_K, 256, 144, 9, -1, 0, -1, 0}
           : q == JK_Q5_K   ? Fmt{JK_Q5_K, 256, 176, 11, -1, 0, -1, 0}
           : q == JK_Q6_K   ? Fmt{JK_Q6_K, 256, 210, 13, 208, 0, -1, 0}
           : q == JK_TQ1_0  ? Fmt{JK_TQ1_0, 256, 54, 0, 0, 2, -1, 0}
           : q == JK_TQ2_0  ? Fmt{JK_TQ2_0, 256, 66, 4, 0, 2, -1, 0}
           : q == JK_I2_S   ? Fmt{JK_I2_S, 128, 32, 2, -1, 0, -1, 0}
                            : Fmt{0, 0, 0, 0, -1, 0, -1, 0};
}

// Format of the device layout a GGUF format is stored in.
__host__ __device__ constexpr int dev_quant(int q) { return q == JK_TQ1_0 ? JK_TQ2_0 : q; }

inline bool fmt_known(int q) { return fmt_of(q).be != 0; }
// Formats with a quant_q8 GEMV / a BitLinear product / an f32-activation vec_dot in the reference.
inline bool has_q8_gemv(int q) {
    return q == JK_Q4_0 || q == JK_Q5_0 || q == JK_Q8_0 || q == JK_Q4_K || q == JK_Q5_K || q == JK_Q6_K ||
           q == JK_TQ1_0 || q == JK_TQ2_0;
}
inline bool has_bitlinear(int q) { return q == JK_TQ1_0 || q == JK_TQ2_0 || q == JK_I2_S || q == JK_Q8_0; }
inline bool has_vec_dot_f32(int q) { return fmt_known(q) && q != JK_TQ1_0 && q != JK_TQ2_0; }
inline size_t trailer_bytes(int q) { return q == JK_I2_S ? 32 : 0; }

// Plain-old-data view of a weight handle that kernels take by value.
struct WeightDev {
    const uint8_t *planes;
    const uint16_t *dplane;
    const uint32_t *hplane;
    float tensor_scale;
    int quant;
    int rows;
    int cols;
    int nb;
};

// One product of a grouped quant_q8 GEMV launch: y[row - r0] for rows [r0, r1) of w,
// against pre-quantized activation blocks xq or f32 activations xf (quantized in the
// launch). nwg (the job's workgroup count) and upg are filled in by the launcher.
constexpr int kMaxGemvJobs = 8;
struct GemvJob {
    WeightDev w;
    const void *xq;
    const float *xf;
    float *y;                       // may be null when am_slots is set (argmax only)
    unsigned long long *am_slots;   // argmax of the job's outputs: one key per workgroup, or null
    int32_t *am_index;              // where the reduction of the slots writes the index
    int r0, r1;  // output rows [r0, r1)
    int nwg;     // workgroups of the job (the columns of its grid row that do work)
    int upg;     // units per workgroup (fast kernel)
};
struct GemvGroup {
    GemvJob job[kMaxGemvJobs];  // job blockIdx.y of a group launch
    int njobs;
    int upw;      // units per wave (upper bound), sizes the per-wave result slots in LDS
    int out_off;  // byte offset of the result slots in dynamic LDS
};

}  // namespace jk

struct jk_weight {
    jk::WeightDev dev = {};  // dev.quant: the device layout (dev_quant of quant)
    std::string name;        // TensorView::name / offset of the tensor it was built from (for errors)
    size_t offset = 0;
    int quant = 0;           // GGUF format of the uploaded tensor
    int device = 0;
    size_t device_bytes = 0;
    size_t gguf_bytes = 0;
    size_t row_bytes = 0;     // GGUF bytes of one row
    void *alloc = nullptr;    // base of the device allocation (planes, then scale plane)
    // Assembly from tile ranges (jk_weight_create .. jk_weight_seal): which 8-row tiles have
    // been written. Compute entry points accept the handle only once it is sealed.
    std::mutex mu;
    std::vector<uint8_t> tile_done;
    std::atomic<bool> ready{false};
};

namespace jk {

// Thread-local error reporting behind jk_last_error() / jk_last_error_info(). fail() takes the
// tensor_name from the message's "name: " prefix; fail_tb() sets TensorBoundsError's fields.
struct Tb {
    const char *name;
    size_t offset, byte_len, buffer_len;
};
jk_status fail(jk_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
jk_status fail_tb(const Tb &t, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// The view's fields as TensorView::name / offset / byte_len / as_bytes().len() report them.
Tb tb_view(const jk_tensor_view *w);
jk_status hip_fail(hipError_t e, const char *what);
void clear_error();

#define JK_HIP(expr)                                          \
    do {                                                      \
        hipError_t e_ = (expr);                               \
        if (e_ != hipSuccess) return ::jk::hip_fail(e_, #expr); \
    } while (0)

#define JK_TRY(expr)                    \
    do {                                \
        jk_status s_ = (expr);          \
        if (s_ != JK_OK) return s_;     \
    } while (0)

// Orientation / byte-length validation shared by the matvec entry points.
jk_status validate_matvec(const jk_tensor_view *w, int quant, size_t out_len, size_t in_len, size_t *rows,
                          size_t *cols);

// Adds to the crate's vector-dot operation counter (vector_dot_count, ime.rs:53-66).
void count_vector_dots(uint64_t n);
// Argument checks of jk_gemm_i8 / jk_dot_i8, shared with their host-tier mirrors.
jk_status gemm_i8_check(const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0, size_t n1,
                        size_t k, const int32_t *c, size_t c_len);
jk_status dot_i8_check(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, const int32_t *out);

// Checks the last kernel launch on the current thread.
jk_status check_launch(const char *what);

// Launch plans: with t_plan.dry set, the GEMM / BitLinear launchers record the kernel they
// would launch (its name) instead of launching it. jk_gemm_plan / jk_bitlinear_plan use this
// to report a shape's kernel, so tests and the bench can check which kernel a call runs.
struct LaunchPlan {
    bool dry = false;
    const char *kernel = nullptr;
};
extern thread_local LaunchPlan t_plan;
#define JK_LAUNCH(NAME, ...)                   \
    do {                                       \
        if (::jk::t_plan.dry)                  \
            ::jk::t_plan.kernel = (NAME);      \
        else                                   \
            hipLaunchKernelGGL(__VA_ARGS__);   \
    } while (0)

// Kernel launchers (device tier internals). All arguments are validated by callers.
// gguf_quant: the GGUF format of the staged payload (w.quant is its device layout).
// Repacks GGUF rows [r0, r1) (gguf: exactly those rows' bytes, in device memory) into w's planes.
jk_status launch_repack(hipStream_t s, const WeightDev &w, int gguf_quant, const uint8_t *gguf, int r0, int r1);
jk_status launch_dequant_rows(hipStream_t s, const WeightDev &w, int r0, int r1, float *out);
// convert_i2_s_blocks_to_tq2_0 over n output blocks (2n I2_S blocks in, 66-byte TQ2_0 blocks out).
jk_status launch_i2s_to_tq2(hipStream_t s, const uint8_t *i2s, size_t n, uint16_t d_bits, uint8_t *tq2);
jk_status launch_quantize_q8_0(hipStream_t s, const float *x, size_t nblocks, jk_block_q8_0 *out);
jk_status launch_quantize_q8_k(hipStream_t s, const float *x, size_t nblocks, jk_block_q8k *out);
jk_status launch_quantize_act_q8(hipStream_t s, const float *x, const jk_act_q8 &a);
// act: 0 none, 1 SwiGLU, 2 ReLU^2 of (x, up) -- the jk_act values.
jk_status launch_quantize_q8_k_gated(hipStream_t s, int act, const float *x, const float *up, size_t nblocks,
                                     jk_block_q8k *out);
jk_status launch_quantize_act_q8_gated(hipStream_t s, int act, const float *x, const float *up, const jk_act_q8 &a);
jk_status launch_gated(hipStream_t s, int act, const float *gate, const float *up, size_t n, float *out);
jk_status launch_argmax(hipStream_t s, const float *x, size_t n, int32_t *index, void *ws);
// Reduces n argmax keys (one per workgroup of a finished launch) to the index.
jk_status launch_argmax_slots(hipStream_t s, const unsigned long long *slots, int n, int32_t *index);
// Workspace bytes for an argmax over n values (standalone) or n output rows (fused GEMV).
size_t argmax_ws_bytes(size_t n);
jk_status launch_absmax_i8(hipStream_t s, const float *x, const float *norm_w, size_t m, size_t k,
                           float eps, int8_t *q, float *scales);
jk_status launch_gemv_q8(hipStream_t s, const WeightDev &w, const void *x, float *y, int r0, int r1);
jk_status launch_gemv_group(hipStream_t s, const GemvJob *jobs, int n);
// Largest K a grouped GEMV job of device format q can take as f32 activations (the launch
// quantizes them into LDS); caller Q8 blocks have no limit.
size_t gemv_f32_max_cols(int q);
// Repacked GEMV for one or two tokens on the GEMV-shaped kernel (jk_gemv_q8.hip): the formats and
// activation sizes it takes, and the launch (bit-identical to the GEMM's m <= 2 route).
bool gemv_repacked_fast_ok(int quant, size_t m, size_t k_padded, size_t k_blocks32);
jk_status launch_gemv_repacked_fast(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1);
// Looks up this device's copy of the no-alloc entry point's static scratch (jk_noalloc.hip).
jk_status noalloc_setup();
// Validated GEMV + fused argmax job over all rows of w (am_slots left null).
jk_status gemv_argmax_job(const char *what, const jk_weight *w, const void *x_q8, const float *x_f32, size_t x_len,
                          float *y, int32_t *index, GemvJob *out);
jk_status launch_vec_dot_f32(hipStream_t s, const WeightDev &w, const float *x, float *y);
// The same products with each block's element products spread over four fused multiply-add
// accumulators: within 1e-5 of each output's row L2 norm.
jk_status launch_vec_dot_f32_tol(hipStream_t s, const WeightDev &w, const float *x, float *y);
// Token count from which jk_bitlinear_i8 uses the MFMA GEMM path.
constexpr int kBitlinearMfmaMinTokens = 16;
jk_status launch_bitlinear_mfma(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales, int m,
                                float *y);
// The same products within 1e-5 of each token's output-row L2 norm, K split over waves.
jk_status launch_bitlinear_mfma_tol(hipStream_t s, const WeightDev &w, const int8_t *act, const float *act_scales,
                                    int m, float *y);
jk_status launch_bitlinear(hipStream_t s, const WeightDev &w, const int8_t *act,
                           const float *act_scales, int m, float *y);
jk_status launch_gemm_repacked(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y,
                               int r0, int r1);
// The same products with each scale group's exact i32 partial (int8 MFMA) rescaled by one fused
// multiply-add instead of the reference's separately rounded product and sum; outputs within 1e-5
// of their token's output-row L2 norm. Launches whose bit-exact tiles measured faster run those.
jk_status launch_gemm_repacked_tol(hipStream_t s, const WeightDev &w, const jk_act_q8 &a, float *y, int r0, int r1);

}  // namespace jk
