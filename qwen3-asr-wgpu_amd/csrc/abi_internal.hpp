// abi_internal.hpp -- definitions shared by the C ABI translation units
// (qasr_attn.hip: contexts, KV pools, attention; decoder.hip: the whole text
// decoder around it): the opaque handle structs and the error reporting.
#pragma once

#include <cstdarg>
#include <cstdio>
#include <string>

#include "kernels.hpp"
#include "qasr_attn.h"

namespace qasr_abi {

// qasr_last_error()'s message (one per host thread, shared by every unit).
inline thread_local std::string g_err;

inline int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

inline int hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? QASR_ENOMEM : QASR_EDEVICE, "%s: %s", what,
                hipGetErrorString(e));
}

// Makes `dev` current for the scope of an ABI call and restores the caller's.
struct DeviceScope {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceScope(int dev) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace qasr_abi

#define HIP_TRY(expr, what)                                          \
    do {                                                             \
        hipError_t e_ = (expr);                                      \
        if (e_ != hipSuccess) return qasr_abi::hip_fail(e_, what);   \
    } while (0)

struct qasr_ctx {
    qasr_attn_cfg cfg;
    int device;
    qasr::f16* cos = nullptr;
    qasr::f16* sin = nullptr;
    int rope_rows = 0;
    float scale_log2;
    int cus = 256;  // compute units of the device (the decode planner's workgroup budget)
    float* scratch = nullptr;  // device address of the no-allocation prefill scratch on `device`
};

struct qasr_kv {
    qasr_ctx* ctx;
    int slots;
    int cap;
    qasr::f16* base = nullptr;
    size_t bytes = 0;
    // decode split-K workspace
    float* dws_acc = nullptr;
    float* dws_ml = nullptr;
    uint32_t* dws_ctr = nullptr;
    int64_t dws_items = 0;
    // prefill split workspace (grown on demand)
    float* pws_o = nullptr;
    float* pws_ml = nullptr;
    uint32_t* pws_ctr = nullptr;
    int64_t pws_items = 0;
};
