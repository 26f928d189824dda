// DynamicQuantizeLinear's arithmetic (src/operators/dynamic_quantize_linear.rs:32-112),
// shared by the DQL launches and the GEMM that quantizes its own output:
//   * min/max start at 0.0 and skip NaN (:56-69) — `v < mn ? v : mn` keeps that exactly,
//     including +0.0 winning over -0.0;
//   * scale = (max-min)/255 and zp = clamp(rne(0 - min/scale)) in f64 (:89-91);
//   * y = clamp(rne(x / scale) + zp) with the division in f64 (:97-103), NaN -> 0.
// Per-element rounding.  |x / scale| <= 255 because min <= 0 <= max.  The fast path forms
// q = x * fl32(1/scale) in f32: two roundings of relative size <= 2^-24 each give
// |q - x/scale| <= 255 * 2^-23 < 3.1e-5.  When q is farther than 1e-4 from a half-integer,
// rne(q) equals rne of the exact quotient and of its f64 rounding (which is within
// 255 * 2^-53 of it).  Otherwise — and for NaN, subnormal x, or a scale outside
// [1e-30, 1e30] — the f64 division is performed as the reference does.  The f64 path itself
// uses x * (1/scale) and falls back to the correctly rounded division within 1e-9 of a tie.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace icx {
namespace dql {

struct alignas(16) DqlParams {
    double s;     // f64 scale (0 for the constant-input sentinel)
    double inv;   // 1/s
    float inv32;  // fl32(1/s), used when `fast`
    int zp;
    int zero;     // min == max
    int fast;     // scale in [1e-30, 1e30]
};

__device__ __forceinline__ void acc_minmax(float v, float& mn, float& mx) {
    mn = (v < mn) ? v : mn;  // NaN compares false: skipped
    mx = (v > mx) ? v : mx;
}

__device__ __forceinline__ void acc4(float4 v, float& mn, float& mx) {
    acc_minmax(v.x, mn, mx);
    acc_minmax(v.y, mn, mx);
    acc_minmax(v.z, mn, mx);
    acc_minmax(v.w, mn, mx);
}

__device__ __forceinline__ void wave_minmax(float& mn, float& mx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float omn = __shfl_xor(mn, off, 64);
        float omx = __shfl_xor(mx, off, 64);
        acc_minmax(omn, mn, mx);
        acc_minmax(omx, mn, mx);
    }
}

// Block-wide (min, max) over NT threads; result valid in every thread.
template <int NT>
__device__ __forceinline__ void block_minmax(float& mn, float& mx) {
    __shared__ float smn[NT / 64], smx[NT / 64];
    wave_minmax(mn, mx);
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smn[wid] = mn;
        smx[wid] = mx;
    }
    __syncthreads();
    mn = smn[0];
    mx = smx[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
        acc_minmax(smn[w], mn, mx);
        acc_minmax(smx[w], mn, mx);
    }
}

__device__ __forceinline__ int clamp_u8(double q) {
    if (q != q) return 0;  // NaN -> 0 (Rust saturating `as u8`)
    q = q < 0.0 ? 0.0 : q;
    q = q > 255.0 ? 255.0 : q;
    return (int)q;
}

__device__ __forceinline__ DqlParams make_params(float mn, float mx) {
    DqlParams p;
    const double mnd = (double)mn, mxd = (double)mx;
    if (mnd == mxd) {
        p.s = 0.0;
        p.inv = 0.0;
        p.inv32 = 0.0f;
        p.zp = 0;
        p.zero = 1;
        p.fast = 0;
        return p;
    }
    p.s = (mxd - mnd) / 255.0;
    p.zp = clamp_u8(rint(0.0 - mnd / p.s));
    p.inv = 1.0 / p.s;
    p.inv32 = (float)p.inv;
    p.zero = 0;
    p.fast = (p.s >= 1e-30 && p.s <= 1e30) ? 1 : 0;
    return p;
}

// Reference-exact f64 path.
__device__ __forceinline__ uint32_t quant1_f64(float x, const DqlParams& p) {
    const double xd = (double)x;
    const double q = xd * p.inv;
    const double fr = q - floor(q);
    double r;
    if (fabs(fr - 0.5) < 1e-9)
        r = rint(xd / p.s);  // near a tie: the correctly rounded quotient decides
    else
        r = rint(q);
    return (uint32_t)clamp_u8(r + (double)p.zp);
}

__device__ __forceinline__ uint32_t quant1(float x, const DqlParams& p) {
    if (p.zero) return 0u;
    const float q = x * p.inv32;
    const float r = rintf(q);
    const float tie_dist = fabsf(fabsf(q - r) - 0.5f);  // q - r is exact (Sterbenz)
    // NaN fails every comparison and so takes the exact path, as do subnormal inputs.
    const bool ok = p.fast && tie_dist > 1e-4f && (fabsf(x) >= 1.17549435e-38f || x == 0.0f);
    if (!ok) return quant1_f64(x, p);
    int v = (int)r + p.zp;
    v = v < 0 ? 0 : v;
    v = v > 255 ? 255 : v;
    return (uint32_t)v;
}

// Four elements at once.  With `fast` (a scale in [1e-30, 1e30]) t = fma(x, fl32(1/s), zp)
// and r = rne(t) decide every element with |t - r| < 0.4999.  The elements of a DQL lie in
// [min, max] with max - min = 255 s, so |x/s| <= 255 and |t| < 256: t is within
// 255·2^-24 (the reciprocal's rounding) + 2^-17 (the fma's) < 2.4e-5 of x/s + zp, so r is
// rne(x/s) + zp (no tie lies within the margin, so shifting by the integer zp cannot flip a
// tie's rounding) — the condition of quant1 without its tie-distance arithmetic.  Subnormal
// x give t = zp.  NaN and inf make t - r NaN, which fails the test and goes to quant1.
__device__ __forceinline__ uint32_t quant4(float4 v, const DqlParams& p) {
    if (p.fast) {
        const float zf = (float)p.zp;
        const float t0 = __builtin_fmaf(v.x, p.inv32, zf), t1 = __builtin_fmaf(v.y, p.inv32, zf);
        const float t2 = __builtin_fmaf(v.z, p.inv32, zf), t3 = __builtin_fmaf(v.w, p.inv32, zf);
        const float r0 = rintf(t0), r1 = rintf(t1), r2 = rintf(t2), r3 = rintf(t3);
        const bool ok = fabsf(t0 - r0) < 0.4999f && fabsf(t1 - r1) < 0.4999f &&
                        fabsf(t2 - r2) < 0.4999f && fabsf(t3 - r3) < 0.4999f;
        if (ok) {
            // v_cvt_pk_u8_f32 clamps the integer r to [0, 255] and writes it into its byte of
            // the word (checked on the MI355X: clamp and round-to-nearest-even, the other
            // bytes kept), one instruction per element instead of med3, convert, shift and or
            uint32_t q = __builtin_amdgcn_cvt_pk_u8_f32(r0, 0, 0u);
            q = __builtin_amdgcn_cvt_pk_u8_f32(r1, 1, q);
            q = __builtin_amdgcn_cvt_pk_u8_f32(r2, 2, q);
            return __builtin_amdgcn_cvt_pk_u8_f32(r3, 3, q);
        }
    }
    return quant1(v.x, p) | (quant1(v.y, p) << 8) | (quant1(v.z, p) << 16) |
           (quant1(v.w, p) << 24);
}


}  // namespace dql
}  // namespace icx
