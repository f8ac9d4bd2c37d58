// lutmoe_moe_forward_noalloc: the MoE layer of lutmoe_moe_forward with the
// library's own device scratch in place of a caller workspace, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  It calls no hipMalloc,
// hipFree or allocating library routine.
//
// The scratch is one file-scope device array per GPU, kScratchBytes long,
// held until the process ends.  Host code reaches it only through the device
// address hipGetSymbolAddress returns for the current device (looked up once
// per device, by lutmoe_noalloc_prepare or else on the first call there; the
// lookup may load the library's code object, so it is done before any graph
// capture); the array's name in host code is a host-side stand-in and is
// never passed to a kernel.  Every call on a GPU
// uses that GPU's array, which keeps the last call's contents: calls that
// overlap in time on one GPU race (serialise them, e.g. on one stream).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;   // 32 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

uint8_t* g_scratch[kMaxDevices];
int g_setup_rc[kMaxDevices];
std::once_flag g_once[kMaxDevices];

// The device address of this device's scratch (looked up on the first call
// on the device).  No part of the layer's workspace needs to start at zero:
// every kernel writes what it later reads within the same call.
int device_scratch(uint8_t** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return LUTMOE_EHIP;
    if (dev < 0 || dev >= kMaxDevices) return LUTMOE_EUNSUPPORTED;
    std::call_once(g_once[dev], [dev]() {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            g_setup_rc[dev] = LUTMOE_EHIP;
            return;
        }
        g_scratch[dev] = (uint8_t*)p;
        g_setup_rc[dev] = LUTMOE_OK;
    });
    *out = g_scratch[dev];
    return g_setup_rc[dev];
}

}  // namespace

extern "C" int lutmoe_noalloc_prepare(void) {
    uint8_t* ws = nullptr;
    return device_scratch(&ws);
}

extern "C" int lutmoe_moe_forward_noalloc(const lutmoe_moe_desc* d, const void* x, const float* topk_w,
                                          const int32_t* topk_ids, int T, int k, void* out, int out_dtype,
                                          int force_path, void* stream) {
    using namespace lutmoe_host;
    if (!topk_w || !topk_ids) return T == 0 ? LUTMOE_OK : LUTMOE_EINVAL;
    if (!d || T < 0 || k <= 0) return LUTMOE_EINVAL;
    if (T == 0) return LUTMOE_OK;
    const size_t need = lutmoe_moe_workspace_size(d, T, k);
    if (need == 0) return LUTMOE_EINVAL;
    if (need > kScratchBytes) {
        char msg[160];
        snprintf(msg, sizeof(msg),
                 "lutmoe_moe_forward_noalloc: %d tokens need %zu bytes of scratch, the static scratch holds %zu",
                 T, need, kScratchBytes);
        set_last_error_text(msg);
        return LUTMOE_EWORKSPACE;
    }
    set_last_error_text("");
    uint8_t* ws = nullptr;
    const int rc = device_scratch(&ws);
    if (rc) return rc;
    return moe_forward_impl(d, x, topk_w, topk_ids, nullptr, T, k, 0, 1.0f, out, out_dtype, ws, kScratchBytes,
                            force_path, LUTMOE_STAGE_ALL, stream);
}
