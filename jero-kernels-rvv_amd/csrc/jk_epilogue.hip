// jk_epilogue.hip -- the operations that follow the path's products: the gated activations of a
// feed-forward block and the argmax of a logits vector.
#include <algorithm>

#include "jk_device.hpp"

namespace jk {

// swiglu_f32 (swiglu.rs:62-121) / relu_squared_gate_f32 (lib.rs:1111-1147): out = gated(gate, up),
// four elements per thread.
template <int ACT>
__global__ __launch_bounds__(256) void gated_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                    size_t n, float *__restrict__ out) {
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (i0 + k < n) out[i0 + k] = gated<ACT>(gate[i0 + k], up[i0 + k]);
}

jk_status launch_gated(hipStream_t s, int act, const float *gate, const float *up, size_t n, float *out) {
    const dim3 grid((unsigned)((n + 1023) / 1024)), block(256);
    if (act == kActSwiglu) hipLaunchKernelGGL(gated_kernel<kActSwiglu>, grid, block, 0, s, gate, up, n, out);
    else hipLaunchKernelGGL(gated_kernel<kActRelu2>, grid, block, 0, s, gate, up, n, out);
    return check_launch("gated_kernel");
}

// argmax_f32 (lib.rs:662-674, scalar recipe 555-568) over n values in two launches: each
// workgroup stores the largest key of its elements to its slot, then one workgroup reduces the
// slots and writes the index (lowest index of the largest non-NaN value, -1 for none).
constexpr int kArgmaxThreads = 256, kArgmaxMaxWgs = 1024, kArgmaxPerThread = 4;
constexpr int kSlotThreads = 1024;

// Each thread takes kArgmaxPerThread elements per pass, their loads issued together.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(const float *__restrict__ x, size_t n,
                                                                        unsigned long long *slots) {
    __shared__ unsigned long long s_keys[kArgmaxThreads / 64];
    unsigned long long key = 0ull;
    const size_t stride = (size_t)gridDim.x * kArgmaxThreads;
    for (size_t base = (size_t)blockIdx.x * kArgmaxThreads + threadIdx.x; base < n;
         base += stride * kArgmaxPerThread) {
        float v[kArgmaxPerThread];
#pragma unroll
        for (int k = 0; k < kArgmaxPerThread; ++k) {
            const size_t i = base + (size_t)k * stride;
            v[k] = i < n ? x[i] : __builtin_nanf("");
        }
#pragma unroll
        for (int k = 0; k < kArgmaxPerThread; ++k) {
            const size_t i = base + (size_t)k * stride;
            const unsigned long long kk = i < n ? argmax_key(v[k], (uint32_t)i) : 0ull;
            key = kk > key ? kk : key;
        }
    }
    argmax_store_wg(key, slots + blockIdx.x, s_keys, kArgmaxThreads / 64);
}

__global__ __launch_bounds__(kSlotThreads) void argmax_slots_kernel(const unsigned long long *__restrict__ slots,
                                                                    int n, int32_t *index) {
    __shared__ unsigned long long s_keys[kSlotThreads / 64];
    __shared__ unsigned long long s_out;
    unsigned long long key = 0ull;
    for (int base = threadIdx.x; base < n; base += 4 * kSlotThreads) {
        unsigned long long v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = base + k * kSlotThreads < n ? slots[base + k * kSlotThreads] : 0ull;
#pragma unroll
        for (int k = 0; k < 4; ++k) key = v[k] > key ? v[k] : key;
    }
    argmax_store_wg(key, &s_out, s_keys, kSlotThreads / 64);
    if (threadIdx.x == 0) *index = argmax_index(s_out);
}

jk_status launch_argmax_slots(hipStream_t s, const unsigned long long *slots, int n, int32_t *index) {
    hipLaunchKernelGGL(argmax_slots_kernel, dim3(1), dim3(kSlotThreads), 0, s, slots, n, index);
    return check_launch("argmax_slots_kernel");
}

jk_status launch_argmax(hipStream_t s, const float *x, size_t n, int32_t *index, void *ws) {
    // kArgmaxPerThread elements per thread, at most kArgmaxMaxWgs workgroups
    const size_t per_wg = (size_t)kArgmaxThreads * kArgmaxPerThread;
    const size_t wgs = std::min<size_t>(kArgmaxMaxWgs, std::max<size_t>(1, (n + per_wg - 1) / per_wg));
    auto *slots = static_cast<unsigned long long *>(ws);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3((unsigned)wgs), dim3(kArgmaxThreads), 0, s, x, n, slots);
    JK_TRY(check_launch("argmax_partial_kernel"));
    return launch_argmax_slots(s, slots, (int)wgs, index);
}

// One 8-byte slot per workgroup: the standalone argmax launches at most kArgmaxMaxWgs, a fused
// GEMV at most one workgroup per output row.
size_t argmax_ws_bytes(size_t n) { return 8 * (n + kArgmaxMaxWgs); }

}  // namespace jk
