// jk_noalloc.hip -- the entry point that allocates nothing: the GEMV with argmax fused into its
// store phase (jk_gemv_q8_argmax) with its argmax slots in a file-scope device array instead of
// a caller workspace, for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Every GPU the library runs on holds its own copy of `scratch` until the process ends. Host
// code never uses the array's name as an address: the address of each device's copy comes from
// hipGetSymbolAddress, called once per device with that device current (from jk_init, or from
// the first call on a device) and kept in `g_scratch`.
//
// Every call on one GPU shares that GPU's array. A call overwrites every slot it reads (each
// workgroup of the GEMV stores its slot before the reduction launch reads it), so nothing needs
// clearing between calls; calls that overlap on one GPU (different streams, or host threads
// without ordering between them) race on the slots and must not be issued.
#include <mutex>

#include "jk_internal.hpp"

namespace jk {

// One 8-byte argmax key per GEMV workgroup (argmax_ws_bytes): room for weights of up to
// kNoAllocMaxRows output rows.
constexpr size_t kNoAllocMaxRows = (size_t)1 << 18;
constexpr size_t kNoAllocScratchBytes = (kNoAllocMaxRows + 1024) * 8;

static __device__ __align__(256) unsigned long long scratch[kNoAllocScratchBytes / 8];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch[kMaxDevices];

// Address of `scratch` on the current device (looked up once per device).
static jk_status scratch_ptr(void **out) {
    int dev = 0;
    JK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(JK_DEVICE_ERROR, "gemv_q8_argmax_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(JK_DEVICE_ERROR, "hipGetSymbolAddress(scratch) returned a null address");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return JK_OK;
}

// Called by jk_init with the chosen device current.
jk_status noalloc_setup() {
    void *p = nullptr;
    return scratch_ptr(&p);
}

}  // namespace jk

using namespace jk;

extern "C" {

jk_status jk_gemv_q8_argmax_noalloc(jk_stream s, const jk_weight *w, const void *x_q8, const float *x_f32,
                                    size_t x_len, float *y, int32_t *index) {
    GemvJob j;
    JK_TRY(gemv_argmax_job("gemv_q8_argmax_noalloc", w, x_q8, x_f32, x_len, y, index, &j));
    if ((size_t)w->dev.rows > kNoAllocMaxRows || argmax_ws_bytes((size_t)w->dev.rows) > kNoAllocScratchBytes)
        return fail(JK_TENSOR_BOUNDS,
                    "gemv_q8_argmax_noalloc: %d output rows exceed the %zu this entry point's static scratch holds",
                    w->dev.rows, kNoAllocMaxRows);
    void *p = nullptr;
    JK_TRY(scratch_ptr(&p));
    j.am_slots = static_cast<unsigned long long *>(p);
    return launch_gemv_group((hipStream_t)s, &j, 1);
}

}  // extern "C"
