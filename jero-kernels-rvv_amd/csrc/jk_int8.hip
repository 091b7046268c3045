// jk_int8.hip -- the crate's plain int8 primitives, in exact i32 on the int8 matrix cores:
//   jk_gemm_i8        C = A * B^T of row-major i8 matrices      (gemm_i8_vector, ime.rs:563-583)
//   jk_gemm_i8_tiles  the same product over 8 x 16 packed tiles (gemm_i8_ime, ime.rs:449-486)
//   jk_pack_tiles_i8  row-major rows into those tiles           (pack_tiles, ime.rs:81-94)
//   jk_dot_i8         one dot product                           (dot_i8_vector, ime.rs:548-557)
//   jk_op_counts      the crate's operation counters            (ime.rs:53-66)
// Integer sums do not depend on their order, so the products run as v_mfma_i32_32x32x32_i8
// tiles and the dot as a workgroup reduction: every result equals the reference's i32 while
// |sum| < 2^31, which k <= 131071 guarantees (|a * b| <= 2^14).
#include <atomic>

#include "jk_device.hpp"

namespace jk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kI8MaxK = 131071;
constexpr int kI8Row = 80;  // LDS bytes per staged row: a 64-byte stage of K plus 16 bytes of padding,
                            // so the 16-byte reads of 16 consecutive rows land on distinct banks

static std::atomic<uint64_t> g_tile_steps{0}, g_vector_dots{0};

void count_vector_dots(uint64_t n) { g_vector_dots.fetch_add(n, std::memory_order_relaxed); }

// Where the 16-byte piece c (elements 16 c .. 16 c + 15) of row r of an operand lives:
//   kRowAligned  row-major rows x k, k a multiple of 16 and the base 16-byte aligned
//   kRowBytes    row-major rows x k, any k and alignment (byte loads; the last piece zero-filled)
//   kTiles       pack_tiles layout: ((r / 8) * kc + c) * 128 + (r % 8) * 16, base 16-byte aligned
enum I8Layout { kRowAligned = 0, kRowBytes = 1, kTiles = 2 };

struct I8Args {
    const int8_t *a, *b;  // b: row 0 is the first row of the requested range
    int32_t *c;
    int m, n;    // rows of A; rows of B in the range (tiles: 8 per tile)
    int k;       // elements per row (kTiles: 16 kc)
    int kc;      // 16-byte pieces per row, ceil(k / 16)
    size_t ldc;  // row-major output: elements per output row
    int ntm, ntn;  // workgroup tiles along A's rows and B's rows
};

// Piece c of row r, or zeros for a row past `rows` or a piece past the row's end.
template <int L>
__device__ __forceinline__ v4i load_piece(const int8_t *base, int rows, int k, int kc, int r, int c) {
    if (r >= rows || c >= kc) return v4i{0, 0, 0, 0};
    if constexpr (L == kRowAligned) {
        return *reinterpret_cast<const v4i *>(base + (size_t)r * k + 16 * c);
    } else if constexpr (L == kTiles) {
        return *reinterpret_cast<const v4i *>(base + ((size_t)(r >> 3) * kc + c) * 128 + (r & 7) * 16);
    } else {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(base + (size_t)r * k + 16 * c);
        const int nv = min(16, k - 16 * c);
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < nv) w[i >> 2] |= (uint32_t)p[i] << (8 * (i & 3));
        return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

// One workgroup: 4 waves in a 2 x 2 grid, each computing WM x WN MFMA tiles of 32 x 32, i.e. a
// 64 WM x 64 WN block of C. K advances in 64-byte stages (two 32-deep MFMA steps): every thread
// loads its share of the next stage's pieces into registers while the current stage is read
// from LDS, then writes them to the other LDS buffer; one barrier per stage orders both.
// Workgroup wg runs on XCD wg % 8; each XCD takes whole columns of tiles along B (the
// workgroups sharing B's rows), so those rows are read into one L2.
template <int L, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_i8_kernel(I8Args g) {
    constexpr int TM = 64 * WM, TN = 64 * WN;
    constexpr int PA = TM * 4 / 256, PB = TN * 4 / 256;  // pieces per thread and stage
    __shared__ __align__(16) int8_t sa[2][TM * kI8Row];
    __shared__ __align__(16) int8_t sb[2][TN * kI8Row];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int jl = lane & 31, hl = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / g.ntm) * 8 + (wg & 7), tm = local % g.ntm;
    if (tn >= g.ntn) return;  // workgroup-uniform, before any barrier
    const int m0 = tm * TM, n0 = tn * TN;
    const int nst = (g.kc + 3) >> 2;  // 64-byte stages

    v4i ra[PA], rb[PB];
    auto gload = [&](int st) {
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int idx = tid + 256 * i;
            ra[i] = load_piece<L>(g.a, g.m, g.k, g.kc, m0 + (idx >> 2), 4 * st + (idx & 3));
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int idx = tid + 256 * i;
            rb[i] = load_piece<L>(g.b, g.n, g.k, g.kc, n0 + (idx >> 2), 4 * st + (idx & 3));
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int idx = tid + 256 * i;
            *reinterpret_cast<v4i *>(&sa[buf][(idx >> 2) * kI8Row + 16 * (idx & 3)]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int idx = tid + 256 * i;
            *reinterpret_cast<v4i *>(&sb[buf][(idx >> 2) * kI8Row + 16 * (idx & 3)]) = rb[i];
        }
    };

    v16i acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = v16i{0};
    gload(0);
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        sstore(buf);
        // the stage's pieces are visible to the workgroup, and every wave has finished reading
        // this buffer two stages ago
        lds_barrier();
        if (st + 1 < nst) gload(st + 1);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v4i xa[WM], xb[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i)
                xa[i] = *reinterpret_cast<const v4i *>(&sa[buf][(32 * (WM * wm + i) + jl) * kI8Row + 32 * s + 16 * hl]);
#pragma unroll
            for (int j = 0; j < WN; ++j)
                xb[j] = *reinterpret_cast<const v4i *>(&sb[buf][(32 * (WN * wn + j) + jl) * kI8Row + 32 * s + 16 * hl]);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], xb[j], acc[i][j], 0, 0, 0);
        }
    }

    // acc[i][j][v] is C[row of A 8 (v / 4) + 4 hl + v % 4][row of B jl] of the 32 x 32 tile (i, j):
    // for each v the 32 lanes of a half-wave store 32 consecutive outputs of one row of C
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + 32 * (WM * wm + i) + 8 * (v >> 2) + 4 * hl + (v & 3);
                const int n = n0 + 32 * (WN * wn + j) + jl;
                if (m < g.m && n < g.n) {
                    if constexpr (L == kTiles)
                        g.c[((size_t)(m >> 3) * (size_t)(g.n >> 3) + (size_t)(n >> 3)) * 64 + (m & 7) * 8 + (n & 7)] =
                            acc[i][j][v];
                    else
                        g.c[(size_t)m * g.ldc + n] = acc[i][j][v];
                }
            }
}

// Large row-major products with K a multiple of 128 (both operands 16-byte aligned): 8 waves per
// workgroup computing a 128 (A rows) x 256 (B rows) tile, each wave 64 x 64 as 2 x 2 MFMA tiles.
// Every 128-byte chunk of K goes from global memory straight into LDS (global_load_lds: lane l
// of a load writes bytes 16 l .. of a 1 KB span), through a ring of three chunk stages (144 KB):
// while chunk kc is evaluated, chunks kc + 1 and kc + 2 stream in. Each wave waits for its own
// loads of a stage (vmcnt) before the barrier that publishes it; that barrier also shows every
// wave done with chunk kc - 1, whose stage then takes chunk kc + 2. In a stage, piece p (16
// bytes) of row r sits at slot p ^ (r & 7), so the 32 rows an MFMA operand read covers fall on
// distinct banks in every group of 8 lanes. Rows past the end re-read the last row (their
// outputs are not stored).
constexpr int kI8Ring = 3;
constexpr int kI8StageBytes = (128 + 256) * 128;  // A: 128 rows, B: 256 rows, 128 bytes each
constexpr int kI8DmaPerWave = 6;                  // 48 spans of 1 KB per stage over 8 waves

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_i8_dma_kernel(I8Args g) {
    __shared__ __align__(16) uint8_t ring[kI8Ring * kI8StageBytes];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int jl = lane & 31, hl = lane >> 5;
    const int wm = wave >> 2, wn = wave & 3;  // the wave's rows: A 64 wm .., B 64 wn ..
    const int wg = (int)blockIdx.x, local = wg >> 3;
    const int tn = (local / g.ntm) * 8 + (wg & 7), tm = local % g.ntm;
    if (tn >= g.ntn) return;  // workgroup-uniform, before any barrier
    const int m0 = tm * 128, n0 = tn * 256;
    const int nch = g.k >> 7;

    // this lane's share of a stage: spans 6 wave + i (A: 0..15, B: 16..47), row 8 (span) + lane / 8
    // of the operand, the piece that belongs in slot lane % 8 (addresses of chunk 0; chunk kc adds 128 kc)
    const int rr = lane >> 3, slot = lane & 7;
    const int8_t *src[kI8DmaPerWave];
#pragma unroll
    for (int i = 0; i < kI8DmaPerWave; ++i) {
        const int span = kI8DmaPerWave * wave + i;
        const int r = 8 * (span < 16 ? span : span - 16) + rr, p = slot ^ (r & 7);
        src[i] = span < 16 ? g.a + (size_t)min(m0 + r, g.m - 1) * (size_t)g.k + 16 * p
                           : g.b + (size_t)min(n0 + r, g.n - 1) * (size_t)g.k + 16 * p;
    }
    auto issue = [&](int kc) {
        const uint8_t *S = ring + (kc % kI8Ring) * kI8StageBytes;
#pragma unroll
        for (int i = 0; i < kI8DmaPerWave; ++i)
            lds_dma16(src[i] + (size_t)kc * 128, (lds_u8_t *)S + 1024 * (kI8DmaPerWave * wave + i));
    };
    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16i{0};
    auto chunk = [&](int kc) {
        const uint8_t *SA = ring + (kc % kI8Ring) * kI8StageBytes, *SB = SA + 128 * 128;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int pc = 2 * st + hl;  // 16-byte piece of the 32-deep step, half hl
            v4i xa[2], xb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = 64 * wm + 32 * i + jl;
                xa[i] = *reinterpret_cast<const v4i *>(SA + r * 128 + ((pc ^ (r & 7)) << 4));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = 64 * wn + 32 * j + jl;
                xb[j] = *reinterpret_cast<const v4i *>(SB + r * 128 + ((pc ^ (r & 7)) << 4));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], xb[j], acc[i][j], 0, 0, 0);
        }
    };
    issue(0);
    if (nch > 1) issue(1);
    for (int kc = 0; kc < nch; ++kc) {
        if (kc + 1 < nch) JK_WAIT_VMCNT(kI8DmaPerWave);  // chunk kc + 1 stays in flight
        else JK_WAIT_VMCNT(0);
        stage_barrier();
        if (kc + 2 < nch) issue(kc + 2);
        chunk(kc);
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                const int n = n0 + 64 * wn + 32 * j + jl;
                if (m < g.m && n < g.n) g.c[(size_t)m * g.ldc + n] = acc[i][j][v];
            }
}

// dot_i8_vector over one workgroup: 16-byte pieces through v_dot4_i32_i8 when both operands are
// 16-byte aligned, bytes otherwise (and for the tail), then a wave and a workgroup sum.
__global__ __launch_bounds__(256) void dot_i8_kernel(const int8_t *__restrict__ a, const int8_t *__restrict__ b, int k,
                                                     int aligned, int32_t *__restrict__ out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int acc = 0, head = 0;
    if (aligned) {
        const int n16 = k >> 4;
        const v4i *a4 = reinterpret_cast<const v4i *>(a), *b4 = reinterpret_cast<const v4i *>(b);
        for (int i = tid; i < n16; i += 256) {
            const v4i x = a4[i], y = b4[i];
            acc = dot4(x[0], y[0], acc);
            acc = dot4(x[1], y[1], acc);
            acc = dot4(x[2], y[2], acc);
            acc = dot4(x[3], y[3], acc);
        }
        head = n16 << 4;
    }
    for (int i = head + tid; i < k; i += 256) acc += (int)a[i] * (int)b[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    __shared__ int part[4];
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (tid == 0) *out = (part[0] + part[1]) + (part[2] + part[3]);
}

// pack_tiles: output piece p = (tile t, chunk c, row r of the tile) at byte 16 p holds elements
// 16 c .. 16 c + 15 of source row 8 t + r, or zeros past the last row.
__global__ __launch_bounds__(256) void pack_tiles_i8_kernel(const int8_t *__restrict__ src, int rows, int k, int kc,
                                                            int aligned, int8_t *__restrict__ dst, size_t pieces) {
    const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= pieces) return;
    const int r = (int)(p & 7);
    const size_t tc = p >> 3;
    const int c = (int)(tc % (size_t)kc);
    const size_t row = (tc / (size_t)kc) * 8 + (size_t)r;
    if (aligned) {
        v4i v = v4i{0, 0, 0, 0};
        if (row < (size_t)rows) v = *reinterpret_cast<const v4i *>(src + row * (size_t)k + 16 * (size_t)c);
        *reinterpret_cast<v4i *>(dst + 16 * p) = v;
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) dst[16 * p + i] = row < (size_t)rows ? src[row * (size_t)k + 16 * (size_t)c + i] : 0;
    }
}

template <int L>
static jk_status launch_gemm_i8(hipStream_t s, I8Args g, const char *what) {
    // 128 x 128 tiles of the product: at least one per CU -> the staged 128 x 256 workgroups where
    // K allows, else register-staged 128 x 128 workgroups when two per CU, 64 x 64 below
    const size_t big = (size_t)((g.m + 127) / 128) * (size_t)((g.n + 127) / 128);
    const bool dma = L == kRowAligned && g.k % 128 == 0 && big >= 256;
    const bool large = !dma && big >= 512;
    const int tm = dma || large ? 128 : 64, tn = dma ? 256 : tm;
    g.ntm = (g.m + tm - 1) / tm;
    g.ntn = (g.n + tn - 1) / tn;
    const size_t grid = (size_t)((g.ntn + 7) / 8) * 8 * (size_t)g.ntm;
    if (grid > 0x7fffffffu) return fail(JK_TENSOR_BOUNDS, "%s: %d x %d rows need too many workgroups", what, g.m, g.n);
    if (dma)
        hipLaunchKernelGGL(gemm_i8_dma_kernel, dim3((unsigned)grid), dim3(512), 0, s, g);
    else if (large)
        hipLaunchKernelGGL((gemm_i8_kernel<L, 2, 2>), dim3((unsigned)grid), dim3(256), 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<L, 1, 1>), dim3((unsigned)grid), dim3(256), 0, s, g);
    return check_launch(what);
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Sizes the kernels index with int: rows of A and of B (tiles: 8 rows each) and the grid.
constexpr size_t kI8MaxRows = (size_t)1 << 28;

}  // namespace jk

namespace jk {

// gemm_i8_vector's slice indexing (ime.rs:563-583) as argument checks: a panic there is
// JK_TENSOR_BOUNDS here, before any copy or launch. Shared by the device and host entry points.
jk_status gemm_i8_check(const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0, size_t n1,
                        size_t k, const int32_t *c, size_t c_len) {
    if (m > kI8MaxRows || n1 > kI8MaxRows)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8: %zu rows of A or n_range end %zu exceed 2^28", m, n1);
    if (k > (size_t)kI8MaxK)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8: k = %zu exceeds %d (an i32 sum of k products of i8 could overflow)", k,
                    kI8MaxK);
    if (n0 > n1) return fail(JK_TENSOR_BOUNDS, "gemm_i8: invalid n_range %zu..%zu", n0, n1);
    if (a_len < m * k || b_len < n1 * k)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8: A holds %zu bytes (needs m * k = %zu), B %zu (needs n_range end * k = %zu)",
                    a_len, m * k, b_len, n1 * k);
    if (c_len != m * (n1 - n0))
        return fail(JK_TENSOR_BOUNDS, "gemm_i8: output length %zu != m (%zu) * n_range (%zu)", c_len, m, n1 - n0);
    if (m == 0 || n1 == n0) return JK_OK;
    if (!c || (k > 0 && (!a || !b))) return fail(JK_TENSOR_BOUNDS, "gemm_i8: null pointer");
    return JK_OK;
}

jk_status dot_i8_check(const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, const int32_t *out) {
    const size_t k = a_len < b_len ? a_len : b_len;  // the pairs of a zip of the two slices
    if (k > (size_t)kI8MaxK)
        return fail(JK_TENSOR_BOUNDS, "dot_i8: %zu pairs exceed %d (an i32 sum of products of i8 could overflow)", k,
                    kI8MaxK);
    if (!out || (k > 0 && (!a || !b))) return fail(JK_TENSOR_BOUNDS, "dot_i8: null pointer");
    return JK_OK;
}

}  // namespace jk

using namespace jk;

extern "C" {

jk_status jk_gemm_i8(jk_stream s, const int8_t *a, size_t a_len, size_t m, const int8_t *b, size_t b_len, size_t n0,
                     size_t n1, size_t k, int32_t *c, size_t c_len) {
    clear_error();
    JK_TRY(gemm_i8_check(a, a_len, m, b, b_len, n0, n1, k, c, c_len));
    if (m == 0 || n1 == n0) return JK_OK;
    I8Args g{};
    g.a = a;
    g.b = b ? b + n0 * k : b;
    g.c = c;
    g.m = (int)m;
    g.n = (int)(n1 - n0);
    g.k = (int)k;
    g.kc = (int)((k + 15) / 16);
    g.ldc = n1 - n0;
    if (k % 16 == 0 && aligned16(g.a) && aligned16(g.b))
        JK_TRY(launch_gemm_i8<kRowAligned>((hipStream_t)s, g, "gemm_i8"));
    else
        JK_TRY(launch_gemm_i8<kRowBytes>((hipStream_t)s, g, "gemm_i8"));
    count_vector_dots((uint64_t)m * (uint64_t)(n1 - n0));
    return JK_OK;
}

jk_status jk_gemm_i8_tiles(jk_stream s, const int8_t *a_packed, size_t a_len, size_t m_tiles, const int8_t *b_packed,
                           size_t b_len, size_t nt0, size_t nt1, size_t k_chunks, int32_t *c, size_t c_len) {
    clear_error();
    if (m_tiles > kI8MaxRows / 8 || nt1 > kI8MaxRows / 8)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: %zu tiles of A or n_tiles end %zu exceed 2^28 rows", m_tiles, nt1);
    if (k_chunks > (size_t)kI8MaxK / 16)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: %zu chunks of 16 exceed k = %d (an i32 sum could overflow)",
                    k_chunks, kI8MaxK);
    if (nt0 > nt1) return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: invalid n_tiles %zu..%zu", nt0, nt1);
    const size_t stride = k_chunks * 128;  // bytes of one packed tile row
    if (a_len < m_tiles * stride || b_len < nt1 * stride)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: A holds %zu bytes (needs %zu), B %zu (needs %zu)", a_len,
                    m_tiles * stride, b_len, nt1 * stride);
    if (c_len != m_tiles * (nt1 - nt0) * 64)
        return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: output length %zu != m_tiles (%zu) * n_tiles (%zu) * 64", c_len,
                    m_tiles, nt1 - nt0);
    if (m_tiles == 0 || nt1 == nt0) return JK_OK;
    if (!c || (k_chunks > 0 && (!a_packed || !b_packed))) return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: null pointer");
    if (!aligned16(a_packed) || !aligned16(b_packed))
        return fail(JK_TENSOR_BOUNDS, "gemm_i8_tiles: packed tiles must be 16-byte aligned (%p, %p)",
                    static_cast<const void *>(a_packed), static_cast<const void *>(b_packed));
    I8Args g{};
    g.a = a_packed;
    g.b = b_packed ? b_packed + nt0 * stride : b_packed;
    g.c = c;
    g.m = (int)(m_tiles * 8);
    g.n = (int)((nt1 - nt0) * 8);
    g.kc = (int)k_chunks;
    g.k = 16 * g.kc;
    g.ldc = 0;
    JK_TRY(launch_gemm_i8<kTiles>((hipStream_t)s, g, "gemm_i8_tiles"));  // k_chunks = 0: tiles of zeros
    g_tile_steps.fetch_add((uint64_t)m_tiles * (uint64_t)(nt1 - nt0) * (uint64_t)k_chunks, std::memory_order_relaxed);
    return JK_OK;
}

jk_status jk_pack_tiles_i8(jk_stream s, const int8_t *src, size_t src_len, size_t rows, size_t k, int8_t *dst,
                           size_t dst_len) {
    clear_error();
    if (k % 16 != 0) return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: k = %zu is not a multiple of 16", k);
    if (rows > kI8MaxRows || k > ((size_t)1 << 30))
        return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: %zu x %zu exceeds the supported size", rows, k);
    if (src_len != rows * k)
        return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: source length %zu != rows * k (%zu)", src_len, rows * k);
    const size_t kc = k / 16, need = (rows + 7) / 8 * kc * 128;
    if (dst_len != need)
        return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: output length %zu != %zu (tile_count(%zu) * %zu chunks * 128)",
                    dst_len, need, rows, kc);
    if (need == 0) return JK_OK;
    if (!src || !dst) return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: null pointer");
    const size_t pieces = need / 16;
    if ((pieces + 255) / 256 > 0x7fffffffu) return fail(JK_TENSOR_BOUNDS, "pack_tiles_i8: %zu bytes is too large", need);
    const int aligned = aligned16(src) && aligned16(dst);
    hipLaunchKernelGGL(pack_tiles_i8_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, (hipStream_t)s, src,
                       (int)rows, (int)k, (int)kc, aligned, dst, pieces);
    return check_launch("pack_tiles_i8");
}

jk_status jk_dot_i8(jk_stream s, const int8_t *a, size_t a_len, const int8_t *b, size_t b_len, int32_t *out) {
    clear_error();
    JK_TRY(dot_i8_check(a, a_len, b, b_len, out));
    const size_t k = a_len < b_len ? a_len : b_len;
    hipLaunchKernelGGL(dot_i8_kernel, dim3(1), dim3(256), 0, (hipStream_t)s, a, b, (int)k,
                       (int)(aligned16(a) && aligned16(b)), out);
    return check_launch("dot_i8");
}

void jk_op_counts(uint64_t *matrix_tile_steps, uint64_t *vector_dots) {
    if (matrix_tile_steps) *matrix_tile_steps = g_tile_steps.load(std::memory_order_relaxed);
    if (vector_dots) *vector_dots = g_vector_dots.load(std::memory_order_relaxed);
}

}  // extern "C"
