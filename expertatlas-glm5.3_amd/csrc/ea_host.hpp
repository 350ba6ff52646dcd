// Host-side plumbing shared by the entry points: per-device context, status mapping, launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <stdint.h>

#include "ea_exl3.h"

namespace ea {

struct DevCtx {
    bool ready = false;
    int device = -1;
    int cus = 0;
    size_t lds_optin = 0;
    int* status = nullptr;  // device int: a kernel's recorded error (unsupported width), 0 = none
    // A second stream (default priority) and two events for launches that run beside the caller's stream inside
    // one call: fork (side waits for the caller's work so far), join (the caller waits for the side's launches).
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    // This device's copy of the decode layer's file-scope scratch array (ea_ffn_moe_decode_static), from
    // hipGetSymbolAddress at ea_init; the array's name is not a device address in host code.
    void* static_scratch = nullptr;
};

// ea_init's set-up of the decode layer's file-scope scratch on the current device (ea_decode_layer.hip): resolves and
// clears this device's copy of the array into c.static_scratch.
int dl_static_setup(DevCtx& c);

// Run `side_work(side stream)` beside `main_work(s)`: both start after everything already on s, and s waits for
// both before anything later. Serialised per device (the side stream and events are shared).
int fork_join(hipStream_t s, const std::function<int(hipStream_t)>& side_work,
              const std::function<int(hipStream_t)>& main_work);

// The context of the current device; nullptr before ea_init on it.
DevCtx* ctx();

inline int hip_status(hipError_t e) {
    if (e == hipSuccess) return EA_OK;
    if (e == hipErrorOutOfMemory) return EA_OUT_OF_DEVICE_MEMORY;
    return EA_HIP_FAILED;
}

// Status of the launch just issued.
inline int launched() { return hip_status(hipGetLastError()); }

inline hipStream_t as_stream(ea_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

template <typename T>
__host__ __device__ inline T* dptr(uint64_t a) {
    return reinterpret_cast<T*>(static_cast<uintptr_t>(a));
}

// Fills n 32-bit words at p with v by a kernel (capturable; no hipMemsetAsync).
int fill_words(hipStream_t s, void* p, uint32_t v, size_t n);

// Device-side error codes written into DevCtx::status.
enum DeviceError : int { DEV_UNSUPPORTED_WIDTH = EA_UNSUPPORTED_WIDTH, DEV_SYNC_TIMEOUT = EA_SYNC_TIMEOUT };

}  // namespace ea

#define EA_REQUIRE_CTX(c)                 \
    ea::DevCtx* c = ea::ctx();            \
    if (!c || !c->ready) return EA_NOT_INITIALIZED
