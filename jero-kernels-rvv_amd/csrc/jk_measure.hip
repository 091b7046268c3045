// jk_measure.hip -- a plain streaming read of device memory, the ceiling each GEMV launch is
// measured against: the same byte count read once, with the same launch path (a stream, a graph of
// back-to-back launches), and no arithmetic. No counterpart in the reference; it exists so that
// the "fraction of the streaming ceiling" figures come from a committed kernel.
#include "jk_device.hpp"
#include "jk_internal.hpp"

namespace jk {

constexpr int kReadThreads = 256;
constexpr int kReadPerLane = 8;  // 16-byte loads in flight per lane

// Workgroup g reads the 32 KB span g * 32 KB ..: load i of the workgroup covers 4 KB, each wave
// 1 KB of consecutive 16-byte pieces (one fully coalesced global_load_dwordx4 per lane).
// Non-temporal loads, as the GEMVs stream their weights. The xor of everything read is stored
// only if it equals a constant, so the loads cannot be removed and nothing is written in practice.
__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const u32x4 *__restrict__ p, size_t n16,
                                                                   unsigned *__restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * (kReadThreads * kReadPerLane) + threadIdx.x;
    u32x4 v[kReadPerLane];
#pragma unroll
    for (int i = 0; i < kReadPerLane; ++i) {
        const size_t idx = base + (size_t)i * kReadThreads;
        v[i] = idx < n16 ? __builtin_nontemporal_load(p + idx) : u32x4{0, 0, 0, 0};
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < kReadPerLane; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace jk

using namespace jk;

extern "C" {

jk_status jk_measure_stream_read(jk_stream s, const void *buf, size_t bytes, uint32_t *sink) {
    clear_error();
    if (!buf || !sink) return fail(JK_TENSOR_BOUNDS, "measure_stream_read: null buffer");
    if (bytes == 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(buf) & 15) != 0)
        return fail(JK_TENSOR_BOUNDS, "measure_stream_read: %zu bytes at %p: need a non-zero multiple of 16 bytes, "
                                      "16-byte aligned", bytes, buf);
    const size_t n16 = bytes / 16;
    const size_t per_wg = (size_t)kReadThreads * kReadPerLane;
    const size_t grid = (n16 + per_wg - 1) / per_wg;
    if (grid > 0x7fffffffu) return fail(JK_TENSOR_BOUNDS, "measure_stream_read: %zu bytes is too large", bytes);
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(kReadThreads), 0, (hipStream_t)s,
                       static_cast<const u32x4 *>(buf), n16, sink);
    return check_launch("measure_stream_read");
}

}  // extern "C"
