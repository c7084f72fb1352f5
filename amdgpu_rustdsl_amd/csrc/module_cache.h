// module_cache.h - per-device loading of a code object embedded in this library (internal to the library).
//
// Each code object is loaded once per device with hipModuleLoadData, under a mutex, and its kernel handles are
// cached; later calls take an acquire load of the per-device flag only.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/fmha_mxfp8.h"

namespace fmha_internal {

inline void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

inline int fail(char* err, size_t errlen, int code, const char* prefix, const char* msg) {
    set_err(err, errlen, "%s: %s", prefix, msg);
    return code;
}

// One embedded code object and the names of the kernels it must provide.
template <int N>
class ModuleCache {
public:
    ModuleCache(const unsigned char* begin, const unsigned char* end, const char* const (&names)[N])
        : begin_(begin), end_(end), names_(names) {}

    // Kernel handles for the current device (FMHA_OK), or FMHA_ERR_NO_DEVICE with a message.
    int get(hipFunction_t** out, char* err, size_t errlen) {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) {
            set_err(err, errlen, "hipGetDevice: %s", hipGetErrorString(e));
            return FMHA_ERR_NO_DEVICE;
        }
        if (dev < 0 || dev >= kMaxDevices) {
            set_err(err, errlen, "device %d out of range", dev);
            return FMHA_ERR_NO_DEVICE;
        }
        Dev& d = dev_[dev];
        if (!d.loaded.load(std::memory_order_acquire)) {
            std::lock_guard<std::mutex> lk(mu_);
            if (!d.loaded.load(std::memory_order_relaxed)) {
                hipModule_t mod = nullptr;
                e = hipModuleLoadData(&mod, begin_);
                if (e != hipSuccess) {
                    set_err(err, errlen, "hipModuleLoadData (gfx950 code object, %zu bytes): %s", (size_t)(end_ - begin_),
                            hipGetErrorString(e));
                    return FMHA_ERR_NO_DEVICE;
                }
                for (int i = 0; i < N; ++i) {
                    e = hipModuleGetFunction(&d.fn[i], mod, names_[i]);
                    if (e != hipSuccess) {
                        set_err(err, errlen, "hipModuleGetFunction(%s): %s", names_[i], hipGetErrorString(e));
                        (void)hipModuleUnload(mod);
                        return FMHA_ERR_NO_DEVICE;
                    }
                }
                d.mod = mod;
                d.loaded.store(true, std::memory_order_release);
            }
        }
        *out = d.fn;
        return FMHA_OK;
    }

    // Launches kernel `which` with the kernarg bytes passed by HIP_LAUNCH_PARAM_BUFFER_POINTER.
    int launch(int which, const void* args, size_t nbytes, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block, void* stream,
               char* err, size_t errlen) {
        hipFunction_t* fns = nullptr;
        int rc = get(&fns, err, errlen);
        if (rc != FMHA_OK) return rc;
        size_t sz = nbytes;
        void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(args), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                         HIP_LAUNCH_PARAM_END};
        hipError_t e = hipModuleLaunchKernel(fns[which], gx, gy, gz, block, 1, 1, 0, (hipStream_t)stream, nullptr, extra);
        if (e != hipSuccess) {
            set_err(err, errlen, "hipModuleLaunchKernel(%s): %s", names_[which], hipGetErrorString(e));
            return FMHA_ERR_HIP;
        }
        return FMHA_OK;
    }

private:
    static constexpr int kMaxDevices = 64;
    struct Dev {
        std::atomic<bool> loaded{false};
        hipModule_t mod = nullptr;
        hipFunction_t fn[N] = {};
    };
    const unsigned char* begin_;
    const unsigned char* end_;
    const char* const (&names_)[N];
    Dev dev_[kMaxDevices];
    std::mutex mu_;
};

}  // namespace fmha_internal
