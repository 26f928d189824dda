// DynamicQuantizeLinear on gfx950: a two-launch, HBM-bound path.
//
//   launch 1  dql_minmax_kernel   — block b reduces one contiguous slice of x (float4 loads,
//             4 in flight per lane) to a (min, max) pair, wave64 shuffles + LDS.
//   launch 2  dql_quantize_kernel / dql_quantize_rows_kernel — the same grid over the same
//             slices: block b first folds the <= 1024 partial pairs (8 KB, L2-resident)
//             and derives scale / zero point itself, so no grid-wide counter or memset is
//             needed (safe to capture in a graph), then quantizes its slice (row mode also
//             writes the row sums of y).
//   Block b of both launches runs on the same XCD (b mod 8) and reads the same bytes, so
//   launch 2 re-reads x from that XCD's L2 (small tensors) or the Infinity Cache.
//
// Semantics follow DynamicQuantizeLinear::forward
// (src/operators/dynamic_quantize_linear.rs:32-112):
//   * min/max start at 0.0 and skip NaN (:56-69) — `v < mn ? v : mn` keeps that exactly,
//     including +0.0 winning over -0.0;
//   * scale = (max-min)/255 and zp = clamp(rne(0 - min/scale)) in f64 (:89-91);
//   * y = clamp(rne(x / scale) + zp) with the division in f64 (:97-103), NaN -> 0.
//
// Per-element rounding.  |x / scale| <= 255 because min <= 0 <= max.  The fast path forms
// q = x * fl32(1/scale) in f32: two roundings of relative size <= 2^-24 each give
// |q - x/scale| <= 255 * 2^-23 < 3.1e-5.  When q is farther than 1e-4 from a half-integer,
// rne(q) equals rne of the exact quotient and of its f64 rounding (which is within
// 255 * 2^-53 of it).  Otherwise — and for NaN, subnormal x, or a scale outside
// [1e-30, 1e30] — the f64 division is performed as the reference does.  The f64 path itself
// uses x * (1/scale) and falls back to the correctly rounded division within 1e-9 of a tie.
#include "icx_common.hpp"
#include "internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 1024;
constexpr int kU = 8;  // float4 loads per lane in flight in the streaming loops

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

// Block-wide (min, max); result valid in every thread.
__device__ __forceinline__ void block_minmax(float& mn, float& mx) {
    __shared__ float smn[kThreads / 64], smx[kThreads / 64];
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
    for (int w = 1; w < kThreads / 64; ++w) {
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

// Four elements at once.  With `fast` (a scale in [1e-30, 1e30]) the f32 quotient q and
// r = rne(q) decide every element with |q - r| < 0.4999 (the condition of quant1 written
// without its tie-distance arithmetic: |q - r| <= 0.5 always).  Subnormal x need no
// separate test here: |q| < 2e-8 then, so r = 0 = rne of the exact quotient.  NaN and inf
// make q - r NaN, which fails the test and goes to quant1.
__device__ __forceinline__ uint32_t quant4(float4 v, const DqlParams& p) {
    if (p.fast) {
        const float q0 = v.x * p.inv32, q1 = v.y * p.inv32, q2 = v.z * p.inv32, q3 = v.w * p.inv32;
        const float r0 = rintf(q0), r1 = rintf(q1), r2 = rintf(q2), r3 = rintf(q3);
        const bool ok = fabsf(q0 - r0) < 0.4999f && fabsf(q1 - r1) < 0.4999f &&
                        fabsf(q2 - r2) < 0.4999f && fabsf(q3 - r3) < 0.4999f;
        if (ok) {
            const uint32_t a = (uint32_t)__builtin_amdgcn_fmed3f(r0 + (float)p.zp, 0.0f, 255.0f);
            const uint32_t b = (uint32_t)__builtin_amdgcn_fmed3f(r1 + (float)p.zp, 0.0f, 255.0f);
            const uint32_t c = (uint32_t)__builtin_amdgcn_fmed3f(r2 + (float)p.zp, 0.0f, 255.0f);
            const uint32_t d = (uint32_t)__builtin_amdgcn_fmed3f(r3 + (float)p.zp, 0.0f, 255.0f);
            return a | (b << 8) | (c << 16) | (d << 24);
        }
    }
    return quant1(v.x, p) | (quant1(v.y, p) << 8) | (quant1(v.z, p) << 16) |
           (quant1(v.w, p) << 24);
}

__device__ __forceinline__ uint32_t bytesum4(uint32_t q) {
    return __builtin_amdgcn_udot4(q, 0x01010101u, 0u, false);
}

// Slice of this block: `units` units of `unit` elements split as evenly as possible over
// the grid; the last block also takes the `tail` elements past units * unit.
struct Slice {
    size_t e0, e1;
};

__device__ __forceinline__ Slice slice_of(size_t units, size_t unit, size_t tail) {
    const size_t G = gridDim.x, b = blockIdx.x;
    const size_t per = units / G, rem = units % G;
    const size_t u0 = b * per + (b < rem ? b : rem);
    const size_t u1 = u0 + per + (b < rem ? 1 : 0);
    Slice s{u0 * unit, u1 * unit};
    if (b == G - 1) s.e1 += tail;
    return s;
}

// Reduce the partials of launch 1 (every block of launch 2 does this redundantly).  The
// first 4 * kThreads partials (all of them for the grids used here) are requested at once;
// a missing one reads as (0, 0), which never moves a range that starts at (0, 0).
__device__ __forceinline__ DqlParams fold_partials(const float2* __restrict__ part, int G) {
    float mn = 0.0f, mx = 0.0f;
    float2 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = threadIdx.x + u * kThreads;
        v[u] = i < G ? part[i] : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        acc_minmax(v[u].x, mn, mx);
        acc_minmax(v[u].y, mn, mx);
    }
    for (int i = threadIdx.x + 4 * kThreads; i < G; i += kThreads) {
        const float2 w = part[i];
        acc_minmax(w.x, mn, mx);
        acc_minmax(w.y, mn, mx);
    }
    block_minmax(mn, mx);
    return make_params(mn, mx);
}

// `vec`: x is 16-byte aligned and unit % 4 == 0, so a slice is whole float4s (+ tail).
__global__ void __launch_bounds__(kThreads)
dql_minmax_kernel(const float* __restrict__ x, size_t units, size_t unit, size_t tail, int vec,
                  float2* __restrict__ part) {
    const Slice sl = slice_of(units, unit, tail);
    float mn = 0.0f, mx = 0.0f;
    const size_t t = threadIdx.x;
    size_t scalar_from = sl.e0;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const size_t b4 = sl.e0 / 4, end4 = b4 + (sl.e1 - sl.e0) / 4;
        // kU float4 per lane requested before any is reduced (128 B per lane in flight); the
        // last batch is guarded per load rather than walked one load at a time.  A skipped
        // load reads as 0.0, which never moves a range that starts at (0, 0).
        for (size_t i = b4 + t; i < end4; i += kU * kThreads) {
            float4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                v[u] = i + u * kThreads < end4 ? x4[i + u * kThreads] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < kU; ++u) acc4(v[u], mn, mx);
        }
        scalar_from = end4 * 4;
    }
    for (size_t j = scalar_from + t; j < sl.e1; j += kThreads) acc_minmax(x[j], mn, mx);
    block_minmax(mn, mx);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(mn, mx);
}

// Flat quantize of this block's slice: lane-consecutive float4 in, 4 bytes out.
// `vec`: x 16-byte and y 4-byte aligned (unit == 4).
__global__ void __launch_bounds__(kThreads)
dql_quantize_kernel(const float* __restrict__ x, size_t units, size_t unit, size_t tail, int vec,
                    uint8_t* __restrict__ y, const float2* __restrict__ part, int G,
                    float* __restrict__ y_scale, uint8_t* __restrict__ y_zp) {
    const Slice sl = slice_of(units, unit, tail);
    const size_t t = threadIdx.x;
    size_t scalar_from = sl.e0;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        uint32_t* y4 = reinterpret_cast<uint32_t*>(y);
        const size_t b4 = sl.e0 / 4, end4 = b4 + (sl.e1 - sl.e0) / 4;
        size_t i = b4 + t;
        // the lane's first kU float4 are requested before the partials are folded, so the
        // fold's loads and barriers overlap them; every batch is guarded per element, so a
        // short last batch still has all its loads in flight at once
        float4 v[kU];
#pragma unroll
        for (int j = 0; j < kU; ++j)
            if (i + j * kThreads < end4) v[j] = x4[i + j * kThreads];
        const DqlParams p = fold_partials(part, G);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *y_scale = (float)p.s;
            *y_zp = (uint8_t)p.zp;
        }
        while (true) {
#pragma unroll
            for (int j = 0; j < kU; ++j)
                if (i + j * kThreads < end4) y4[i + j * kThreads] = quant4(v[j], p);
            i += kU * kThreads;
            if (i >= end4) break;
#pragma unroll
            for (int j = 0; j < kU; ++j)
                if (i + j * kThreads < end4) v[j] = x4[i + j * kThreads];
        }
        for (size_t j = end4 * 4 + t; j < sl.e1; j += kThreads) y[j] = (uint8_t)quant1(x[j], p);
        return;
    }
    const DqlParams p = fold_partials(part, G);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *y_scale = (float)p.s;
        *y_zp = (uint8_t)p.zp;
    }
    for (size_t j = scalar_from + t; j < sl.e1; j += kThreads) y[j] = (uint8_t)quant1(x[j], p);
}

// Row mode: the slices are whole rows; one wave per row at a time, and the row sums of y
// (u8 summed as int32) are written too.  `vec`: x 16-byte and y 4-byte aligned and
// row_len % 4 == 0.
__global__ void __launch_bounds__(kThreads)
dql_quantize_rows_kernel(const float* __restrict__ x, size_t rows, size_t row_len, int vec,
                         uint8_t* __restrict__ y, int32_t* __restrict__ rowsum,
                         const float2* __restrict__ part, int G, float* __restrict__ y_scale,
                         uint8_t* __restrict__ y_zp) {
    const DqlParams p = fold_partials(part, G);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *y_scale = (float)p.s;
        *y_zp = (uint8_t)p.zp;
    }
    const Slice sl = slice_of(rows, 1, 0);  // a range of rows
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    constexpr size_t kWaves = kThreads / 64;
    if (vec) {
        // Two rows per wave at a time (r and r + kWaves), four float4 of each per lane in
        // flight, so a wave never waits on a single row's loads.
        const size_t n4 = row_len / 4;
        for (size_t r = sl.e0 + wid; r < sl.e1; r += 2 * kWaves) {
            const size_t r2 = r + kWaves;
            const bool two = r2 < sl.e1;
            const float4* xa = reinterpret_cast<const float4*>(x + r * row_len);
            const float4* xb = reinterpret_cast<const float4*>(x + (two ? r2 : r) * row_len);
            uint32_t* ya = reinterpret_cast<uint32_t*>(y + r * row_len);
            uint32_t* yb = reinterpret_cast<uint32_t*>(y + (two ? r2 : r) * row_len);
            uint32_t sa = 0, sb = 0;
            for (size_t i = lane; i < n4; i += 4 * 64) {
                float4 va[4], vb[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (i + 64 * j < n4) va[j] = xa[i + 64 * j];
                    if (two && i + 64 * j < n4) vb[j] = xb[i + 64 * j];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (i + 64 * j < n4) {
                        const uint32_t q = quant4(va[j], p);
                        ya[i + 64 * j] = q;
                        sa += bytesum4(q);
                    }
                    if (two && i + 64 * j < n4) {
                        const uint32_t q = quant4(vb[j], p);
                        yb[i + 64 * j] = q;
                        sb += bytesum4(q);
                    }
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                sa += __shfl_xor(sa, off, 64);
                sb += __shfl_xor(sb, off, 64);
            }
            if (lane == 0) {
                rowsum[r] = (int32_t)sa;
                if (two) rowsum[r2] = (int32_t)sb;
            }
        }
        return;
    }
    for (size_t r = sl.e0 + wid; r < sl.e1; r += kWaves) {
        const float* xr = x + r * row_len;
        uint8_t* yr = y + r * row_len;
        uint32_t s = 0;
        for (size_t i = lane; i < row_len; i += 64) {
            const uint32_t q = quant1(xr[i], p);
            yr[i] = (uint8_t)q;
            s += q;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) rowsum[r] = (int32_t)s;
    }
}


}  // namespace

// The single-launch path: aligned operands, whole float4s, and a slice that fits kFRegs
// float4 per lane (flat) or whole rows that do (row mode).
extern "C" size_t icx_dql_workspace_size(size_t) { return sizeof(float2) * kMaxBlocks; }

// The quantize launch alone, folding partials a producing kernel left (the same grid choice
// and kernels as the second launch below).
int icx::dql_from_parts(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                        int32_t* rowsum, size_t row_len, const float2* part, int n_part) {
    if (!x || !y || !y_scale || !y_zp || !part || n_part <= 0)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DynamicQuantizeLinear: null pointer or no partials");
    if (rowsum && (row_len == 0 || n % row_len != 0))
        ICX_FAIL(ICX_ERR_SHAPE, "DynamicQuantizeLinear: row_len %zu does not divide n = %zu", row_len, n);
    const bool x16 = icx::aligned16(x), y4 = (reinterpret_cast<uintptr_t>(y) & 3u) == 0;
    if (rowsum) {
        const size_t units = n / row_len;
        const size_t rpw = std::max<size_t>(1, icx::cdiv(units, (size_t)4 * kMaxBlocks));
        const int G = (int)std::max<size_t>(1, std::min<size_t>({(size_t)kMaxBlocks, icx::cdiv(units, 4 * rpw), units}));
        const int rvec = (x16 && y4 && row_len % 4 == 0) ? 1 : 0;
        hipLaunchKernelGGL(dql_quantize_rows_kernel, dim3(G), dim3(kThreads), 0, s, x, units, row_len, rvec, y,
                           rowsum, part, n_part, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_rows_kernel");
        return ICX_OK;
    }
    size_t units, unit, tail;
    if (x16 && y4) {
        units = n / 4;
        unit = 4;
        tail = n % 4;
    } else {
        units = n;
        unit = 1;
        tail = 0;
    }
    const int G = (int)std::max<size_t>(1, std::min<size_t>({(size_t)kMaxBlocks, icx::cdiv(n, (size_t)kThreads * 16), units}));
    const int qvec = (x16 && y4 && unit == 4) ? 1 : 0;
    hipLaunchKernelGGL(dql_quantize_kernel, dim3(G), dim3(kThreads), 0, s, x, units, unit, tail, qvec, y, part,
                       n_part, y_scale, y_zp);
    ICX_LAUNCH_CHECK("dql_quantize_kernel");
    return ICX_OK;
}

extern "C" int icx_dynamic_quantize_linear(icx_stream_t stream, const float* x, size_t n,
                                           uint8_t* y, float* y_scale, uint8_t* y_zp,
                                           int32_t* opt_rowsum, size_t row_len, void* ws,
                                           size_t ws_bytes) {
    icx::clear_error();
    if (!x || !y || !y_scale || !y_zp)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DynamicQuantizeLinear: null pointer argument");
    if (!ws || ws_bytes < icx_dql_workspace_size(n))
        ICX_FAIL(ICX_ERR_WORKSPACE, "DynamicQuantizeLinear: workspace of %zu bytes needed",
                 icx_dql_workspace_size(n));
    if (opt_rowsum && (row_len == 0 || n % row_len != 0))
        ICX_FAIL(ICX_ERR_SHAPE, "DynamicQuantizeLinear: row_len %zu does not divide n = %zu",
                 row_len, n);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    float2* part = reinterpret_cast<float2*>(ws);
    const bool x16 = icx::aligned16(x), y4 = (reinterpret_cast<uintptr_t>(y) & 3u) == 0;
    // Partition: rows in row mode, float4 groups (or single elements) otherwise.  Both
    // launches use the same grid, so block b reads the same slice twice; ~4 float4 per lane.
    size_t units, unit, tail;
    if (opt_rowsum) {
        units = n / row_len;
        unit = row_len;
        tail = 0;
    } else if (x16 && y4) {
        units = n / 4;
        unit = 4;
        tail = n % 4;
    } else {
        units = n;
        unit = 1;
        tail = 0;
    }
    size_t want = icx::cdiv(n, (size_t)kThreads * 16);
    if (opt_rowsum) {
        // the same number of rows for every wave: rows_per_wave * 4 waves per block
        const size_t rpw = std::max<size_t>(1, icx::cdiv(units, (size_t)4 * kMaxBlocks));
        want = icx::cdiv(units, 4 * rpw);
    }
    const int G = (int)std::max<size_t>(1, std::min<size_t>({(size_t)kMaxBlocks, want, units}));
    const int vec1 = (x16 && unit % 4 == 0) ? 1 : 0;
    hipLaunchKernelGGL(dql_minmax_kernel, dim3(G), dim3(kThreads), 0, s, x, units, unit, tail,
                       vec1, part);
    ICX_LAUNCH_CHECK("dql_minmax_kernel");
    if (opt_rowsum) {
        const int rvec = (x16 && y4 && row_len % 4 == 0) ? 1 : 0;
        hipLaunchKernelGGL(dql_quantize_rows_kernel, dim3(G), dim3(kThreads), 0, s, x, units,
                           row_len, rvec, y, opt_rowsum, part, G, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_rows_kernel");
    } else {
        const int qvec = (x16 && y4 && unit == 4) ? 1 : 0;
        hipLaunchKernelGGL(dql_quantize_kernel, dim3(G), dim3(kThreads), 0, s, x, units, unit,
                           tail, qvec, y, part, G, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_kernel");
    }
    return ICX_OK;
}
