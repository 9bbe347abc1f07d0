// The allocation-free variant of chk_lm_head_argmax: the same LM head and
// argmax kernels, with their per-workgroup argmax partials (value and row
// index per workgroup and input row) in a file-scope device array instead
// of device memory allocated per call.  For callers that cannot allocate
// (code under graph capture, serving loops that forbid hipMalloc).
//
// The array is a host-side stand-in in host code: its device address is
// looked up once per device (hipGetSymbolAddress, on the entry point's
// first call with that device current) and only that address is passed to
// kernels.  That first call must not be under stream capture (it is
// refused there); every later call only enqueues the two kernels on the
// caller's stream and never waits on it, so it can be captured into a
// graph.  Launch errors are reported; errors of the kernels themselves
// surface at the caller's next synchronisation.  Every call on a device
// shares that device's array; the kernels overwrite every partial they
// read, so nothing needs clearing, and calls that overlap on one device
// race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdexcept>
#include <string>

#include "cherenkov/kernels.h"
#include "kernels_internal.h"

namespace chk {

constexpr uint32_t NOALLOC_PARTS = 1024;  // LM head workgroups (argmax partials per row)
constexpr uint64_t NOALLOC_SCRATCH_BYTES = (uint64_t)MAX_NB * NOALLOC_PARTS * (sizeof(float) + sizeof(uint32_t));
static_assert(NOALLOC_SCRATCH_BYTES == 32 * 1024, "argmax partials: 4 rows x 1024 workgroups x (f32 value, u32 row)");

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static void* g_scratch_dev[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The device address of `scratch` on the current device; the lookup (first
// call on a device) is refused while `st` is capturing.
static uint8_t* scratch_address(hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) throw std::runtime_error("device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) throw std::runtime_error(std::string("hipStreamIsCapturing: ") + hipGetErrorString(e));
        if (cs != hipStreamCaptureStatusNone)
            throw std::runtime_error("the first call on a device resolves the scratch address and must not be captured");
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    return static_cast<uint8_t*>(g_scratch_dev[dev]);
}

}  // namespace chk

using namespace chk;

extern "C" int chk_lm_head_argmax_noalloc(const void* w, const void* s, const void* b, uint32_t out, uint32_t in,
                                          const float* x, uint32_t nb, float* logits, uint32_t* ids, void* stream) {
    try {
        if (nb < 1 || nb > (uint32_t)MAX_NB) throw std::runtime_error("nb must be 1..=4");
        if (in % 64 || in == 0) throw std::runtime_error("in must be a positive multiple of 64");
        if (out == 0 || out % 8) throw std::runtime_error("out must be a positive multiple of 8");
        hipStream_t st = (hipStream_t)stream;
        uint8_t* base = scratch_address(st);
        float* pv = reinterpret_cast<float*>(base);
        uint32_t* pi = reinterpret_cast<uint32_t*>(base + (uint64_t)MAX_NB * NOALLOC_PARTS * sizeof(float));
        launch_lm_head(Q4Mat{(const uint32_t*)w, (const uint16_t*)s, (const uint16_t*)b, out, in}, x, logits, pv, pi,
                       NOALLOC_PARTS, ids, (int)nb, st);
        hipError_t e = hipPeekAtLastError();
        if (e != hipSuccess) throw std::runtime_error(std::string("HIP launch error ") + hipGetErrorString(e));
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}
