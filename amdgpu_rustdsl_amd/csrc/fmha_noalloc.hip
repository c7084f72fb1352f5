// fmha_noalloc.hip - the allocation-free variant of fmha_fwd_hd128_mxfp8_auto (include/fmha_mxfp8.h).
//
// The only device memory the path needs beyond the caller's inputs and outputs is the KV split's workspace: fp32-sized
// partial rows and the base-2 LSE of every split. This variant takes no workspace argument. It uses `scratch`, a
// file-scope device array of FMHA_NOALLOC_SCRATCH_BYTES, instead, and calls no allocating routine.
//
// Host code may not pass `scratch` itself to a kernel: on the host that name is a stand-in, not a device address. Its
// device address is looked up once per device with hipGetSymbolAddress (each device holds its own copy of the array)
// and kept in g_scratch[dev]; only that pointer goes to the kernels.
//
// Every call on one device shares that device's array, and the array keeps the last call's partials: the split
// kernel writes every partial row and LSE entry the combine reads, so nothing needs clearing, but two calls that
// overlap on one device (different streams, no ordering) race on it.
//
// Compiled by hipcc as single-source HIP (the array's code object is registered with the HIP runtime when the library
// loads); the FMHA kernels themselves live in the embedded code object of fmha_host.cpp.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "../../include/fmha_mxfp8.h"
#include "module_cache.h"

static __device__ __align__(256) uint8_t scratch[FMHA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_mu;

// The device address of this device's `scratch` (looked up on the first call on the device, with it current).
int scratch_ptr(void** out, char* err, size_t errlen) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        fmha_internal::set_err(err, errlen, "hipGetDevice: %s", hipGetErrorString(e));
        return FMHA_ERR_NO_DEVICE;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        fmha_internal::set_err(err, errlen, "device %d out of range", dev);
        return FMHA_ERR_NO_DEVICE;
    }
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                fmha_internal::set_err(err, errlen, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
                return FMHA_ERR_HIP;
            }
            // the FMHA code object too, so that no later call loads anything
            const int rc = fmha_mxfp8_init(err, errlen);
            if (rc != FMHA_OK) return rc;
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return FMHA_OK;
}

}  // namespace

extern "C" int fmha_fwd_hd128_mxfp8_auto_noalloc(const fmha_mxfp8_params* p, void* stream, int* path_out, int* splits_out,
                                                 char* err, size_t errlen) {
    if (!p) return fmha_internal::fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-ARGS", "null params");
    // the KV split the one-call entry would run, and the scratch it needs (the rules themselves are the entry's)
    size_t need = 0;
    if (p->B >= 1 && p->H >= 1 && p->S >= 1 && p->SK >= 1 && !p->causal) {
        int splits = 0;
        int path = p->path;
        if (path < 0) path = fmha_mxfp8_select_path(p->B, p->H, p->S, p->SK, &splits);
        else if (path == FMHA_PATH_KVSPLIT) splits = p->splits > 0 ? p->splits : 4;
        // an invalid split count is left to the entry, which reports it (GV-HOST-PATH)
        if (path == FMHA_PATH_KVSPLIT && (splits == 2 || splits == 4 || splits == 8))
            need = fmha_mxfp8_workspace_bytes(p->B, p->H, p->S, splits);
    }
    if (need > (size_t)FMHA_NOALLOC_SCRATCH_BYTES) {
        fmha_internal::set_err(err, errlen,
                               "GV-HOST-WORKSPACE: the KV split needs %zu workspace bytes, more than the %zu of the "
                               "allocation-free entry's scratch; use fmha_fwd_hd128_mxfp8_auto with a workspace",
                               need, (size_t)FMHA_NOALLOC_SCRATCH_BYTES);
        return FMHA_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    const int rc = scratch_ptr(&ws, err, errlen);
    if (rc != FMHA_OK) return rc;
    return fmha_fwd_hd128_mxfp8_auto(p, ws, (size_t)FMHA_NOALLOC_SCRATCH_BYTES, stream, path_out, splits_out, err, errlen);
}
