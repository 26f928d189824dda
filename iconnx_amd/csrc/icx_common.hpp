// Shared helpers for the iconnx_hip library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/iconnx_hip.h"

namespace icx {

// Per-host-thread message of the last failure, returned by icx_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define ICX_FAIL(status, ...)             \
    do {                                  \
        ::icx::set_error(__VA_ARGS__);    \
        return (status);                  \
    } while (0)

#define ICX_HIP_CHECK(call)                                                           \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess)                                                         \
            ICX_FAIL(ICX_ERR_HIP, "%s: %s (%s:%d)", #call, hipGetErrorString(e_),     \
                     __FILE__, __LINE__);                                             \
    } while (0)

// Launch-error check after a <<<>>> launch.
#define ICX_LAUNCH_CHECK(what)                                                        \
    do {                                                                              \
        hipError_t e_ = hipGetLastError();                                            \
        if (e_ != hipSuccess)                                                         \
            ICX_FAIL(ICX_ERR_HIP, "%s launch: %s", what, hipGetErrorString(e_));      \
    } while (0)

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline size_t cdiv(size_t a, size_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte streaming (non-temporal) store for outputs written once and not re-read by the
// same kernel: on gfx950 it lifts a read+write stream from ~5.3 to ~6.9 TB/s.
__device__ __forceinline__ void store_nt(float4* p, float4 v) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<f4v*>(p));
}

__device__ __forceinline__ void store_nt_u32(uint32_t* p, uint32_t v) {
    __builtin_nontemporal_store(v, p);
}

// int8 / uint8 operand description used by the GEMM entry points.
inline bool is_int8_kind(int dt) { return dt == ICX_I8 || dt == ICX_U8; }

}  // namespace icx
