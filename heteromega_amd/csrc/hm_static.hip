// hm_ffn_forward_static: hm_ffn_forward with the library's own device scratch instead of a caller workspace.
//
// The scratch is one file-scope device array per GPU (the loader gives each device that runs the library its
// own copy, held until the process ends). Host code never passes the array's name to a kernel or a copy: on
// the host that name is a stand-in, not a device address. Each device's address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address is used.
//
// Nothing in the scratch has to start at zero: the FFN's kernels write the SwiGLU activation and every split
// partial before anything reads them. Calls on one GPU share its scratch, so calls that overlap in time on one
// GPU (two streams, two host threads) race; calls on one stream run one after the other and are safe.
#include "../../include/hm_w4a16.h"
#include "hm_internal.hpp"

#include <hip/hip_runtime.h>

#include <mutex>

namespace {

constexpr size_t kScratchBytes = HM_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};

// The device address of this device's scratch array (looked up on the first call per device).
hipError_t scratch_address(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return e;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        return hipErrorInvalidDevice;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            return e;
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

} // namespace

extern "C" hm_status hm_ffn_forward_static(const hm_ffn *f, void *y, int64_t ldy, const void *x, int64_t ldx, int64_t M,
                                           int64_t ch_begin, int64_t ch_end, void *stream) {
    if (f == nullptr || M <= 0) {
        return hm::set_error(HM_INVALID_ARGUMENT, "hm_ffn_forward_static: null handle or M <= 0");
    }
    const size_t need = hm_ffn_workspace_bytes(f, M);
    if (need > kScratchBytes) {
        return hm::set_error(HM_WORKSPACE_TOO_SMALL,
                             "hm_ffn_forward_static: M = %lld needs %zu bytes of scratch, more than the static %zu bytes; "
                             "use hm_ffn_forward with a workspace",
                             static_cast<long long>(M), need, kScratchBytes);
    }
    void *ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) {
        return hm::set_error(HM_HIP_ERROR, "hm_ffn_forward_static: hipGetSymbolAddress of the scratch: %s", hipGetErrorString(e));
    }
    return hm_ffn_forward(f, y, ldy, x, ldx, M, ch_begin, ch_end, ws, kScratchBytes, stream);
}
