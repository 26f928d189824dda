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

// ---- DynamicQuantizeLinear's range of a kernel's output ---------------------------------
// A kernel whose output feeds a DynamicQuantizeLinear can leave the min / max that the DQL
// forward takes over it (src/operators/dynamic_quantize_linear.rs:56-69: both start at 0.0,
// NaN is skipped): one running pair per thread, one (min, max) per block in
// `part[blockIdx.x]`, folded by the DQL's quantize launch.  Min and max are exact, so the
// partition into blocks does not change the result.  fminf / fmaxf (v_min / v_max) return
// the other operand for a quiet NaN — the only NaN arithmetic produces — and may keep -0.0
// where the reference's `v < mn ? v : mn` keeps +0.0; a zero minimum of either sign gives
// the same scale ((max - min) / 255) and zero point (rne(0 - min / scale)), and the fold in
// the quantize launch uses the reference's comparison, so the DQL outputs are the same.
__device__ __forceinline__ void range_acc(float v, float& mn, float& mx) {
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
}

// Every thread of a block of NT threads calls this (it synchronises).
template <int NT>
__device__ __forceinline__ void block_range_store(float mn, float mx, float2* part) {
    __shared__ float smn[NT / 64], smx[NT / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float omn = __shfl_xor(mn, off, 64), omx = __shfl_xor(mx, off, 64);
        range_acc(omn, mn, mx);
        range_acc(omx, mn, mx);
    }
    if ((threadIdx.x & 63) == 0) {
        smn[threadIdx.x >> 6] = mn;
        smx[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < NT / 64; ++w) {
            range_acc(smn[w], mn, mx);
            range_acc(smx[w], mn, mx);
        }
        part[blockIdx.x] = make_float2(mn, mx);
    }
}

// Most partials any producing kernel leaves (the DQL quantize launch folds them).
constexpr int kMaxRangeParts = 1024;

// Most output segments of one GEMM launch (sibling linears over one input, e.g. Q / K / V).
constexpr int kMaxSegments = 4;

// int8 / uint8 operand description used by the GEMM entry points.
inline bool is_int8_kind(int dt) { return dt == ICX_I8 || dt == ICX_U8; }

}  // namespace icx
