// DynamicQuantizeLinear on gfx950: a two-launch, HBM-bound path.
//
//   launch 1  dql_minmax_kernel   — each block reduces a grid-stride share of x (float4
//             loads, 4 in flight per lane) to one (min, max) pair, wave64 shuffles + LDS.
//   launch 2  dql_quantize_*      — a persistent grid; every block first folds the <=512
//             partial pairs (4 KB, L2-resident) and derives scale / zero point itself, so
//             no grid-wide counter or memset is needed (safe to capture in a graph), then
//             quantizes 16 elements per lane (4 x float4 in, one 16-byte store out).
//
// Semantics follow DynamicQuantizeLinear::forward
// (src/operators/dynamic_quantize_linear.rs:32-112):
//   * min/max start at 0.0 and skip NaN (:56-69) — `v < mn ? v : mn` keeps that exactly,
//     including +0.0 winning over -0.0;
//   * scale = (max-min)/255 and zp = clamp(rne(0 - min/scale)) in f64 (:89-91);
//   * y = clamp(rne(x / scale) + zp) with the division in f64 (:97-103), NaN -> 0.
// The per-element quotient is formed as x * (1/scale) in f64 (error < 2^-51 * 255 ~ 1e-13
// in absolute terms since |x/scale| <= 255); only when that product lies within 1e-9 of a
// half-integer — where rounding could depend on the last bits — is the correctly rounded
// f64 division performed, so the result equals the reference's f64 division bit for bit.
#include "icx_common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPartials = 512;

struct alignas(16) DqlParams {
    double s;    // f64 scale (0 for the constant-input sentinel)
    double inv;  // 1/s
    int zp;
    int zero;    // min == max
};

__device__ __forceinline__ void acc_minmax(float v, float& mn, float& mx) {
    mn = (v < mn) ? v : mn;  // NaN compares false: skipped
    mx = (v > mx) ? v : mx;
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
        p.zp = 0;
        p.zero = 1;
        return p;
    }
    p.s = (mxd - mnd) / 255.0;
    p.zp = clamp_u8(rint(0.0 - mnd / p.s));
    p.inv = 1.0 / p.s;
    p.zero = 0;
    return p;
}

__device__ __forceinline__ uint32_t quant1(float x, const DqlParams& p) {
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

__device__ __forceinline__ uint32_t quant4(float4 v, const DqlParams& p) {
    return quant1(v.x, p) | (quant1(v.y, p) << 8) | (quant1(v.z, p) << 16) |
           (quant1(v.w, p) << 24);
}

// Reduce the partials of launch 1 (every block of launch 2 does this redundantly).
__device__ __forceinline__ DqlParams fold_partials(const float2* __restrict__ part, int G) {
    float mn = 0.0f, mx = 0.0f;
    for (int i = threadIdx.x; i < G; i += kThreads) {
        float2 v = part[i];
        acc_minmax(v.x, mn, mx);
        acc_minmax(v.y, mn, mx);
    }
    block_minmax(mn, mx);
    return make_params(mn, mx);
}

__global__ void __launch_bounds__(kThreads)
dql_minmax_kernel(const float* __restrict__ x, size_t n, int vec, float2* __restrict__ part) {
    float mn = 0.0f, mx = 0.0f;
    const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * kThreads;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const size_t n4 = n / 4;
        size_t i = tid;
        for (; i + 3 * stride < n4; i += 4 * stride) {
            float4 a = x4[i], b = x4[i + stride], c = x4[i + 2 * stride], d = x4[i + 3 * stride];
            acc_minmax(a.x, mn, mx); acc_minmax(a.y, mn, mx); acc_minmax(a.z, mn, mx); acc_minmax(a.w, mn, mx);
            acc_minmax(b.x, mn, mx); acc_minmax(b.y, mn, mx); acc_minmax(b.z, mn, mx); acc_minmax(b.w, mn, mx);
            acc_minmax(c.x, mn, mx); acc_minmax(c.y, mn, mx); acc_minmax(c.z, mn, mx); acc_minmax(c.w, mn, mx);
            acc_minmax(d.x, mn, mx); acc_minmax(d.y, mn, mx); acc_minmax(d.z, mn, mx); acc_minmax(d.w, mn, mx);
        }
        for (; i < n4; i += stride) {
            float4 a = x4[i];
            acc_minmax(a.x, mn, mx); acc_minmax(a.y, mn, mx); acc_minmax(a.z, mn, mx); acc_minmax(a.w, mn, mx);
        }
        for (size_t j = n4 * 4 + tid; j < n; j += stride) acc_minmax(x[j], mn, mx);
    } else {
        for (size_t j = tid; j < n; j += stride) acc_minmax(x[j], mn, mx);
    }
    block_minmax(mn, mx);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(mn, mx);
}

__global__ void __launch_bounds__(kThreads)
dql_quantize_flat_kernel(const float* __restrict__ x, size_t n, int vec, uint8_t* __restrict__ y,
                         const float2* __restrict__ part, int G, float* __restrict__ y_scale,
                         uint8_t* __restrict__ y_zp) {
    const DqlParams p = fold_partials(part, G);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *y_scale = (float)p.s;
        *y_zp = (uint8_t)p.zp;
    }
    const size_t tid = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * kThreads;
    if (vec) {
        // 16 elements per lane per step: four float4 loads, one 16-byte store.
        const float4* x4 = reinterpret_cast<const float4*>(x);
        uint4* y16 = reinterpret_cast<uint4*>(y);
        const size_t n16 = n / 16;
        for (size_t i = tid; i < n16; i += stride) {
            float4 a = x4[4 * i], b = x4[4 * i + 1], c = x4[4 * i + 2], d = x4[4 * i + 3];
            uint4 o;
            if (p.zero) {
                o = make_uint4(0, 0, 0, 0);
            } else {
                o.x = quant4(a, p);
                o.y = quant4(b, p);
                o.z = quant4(c, p);
                o.w = quant4(d, p);
            }
            y16[i] = o;
        }
        for (size_t j = n16 * 16 + tid; j < n; j += stride)
            y[j] = p.zero ? 0 : (uint8_t)quant1(x[j], p);
    } else {
        for (size_t j = tid; j < n; j += stride) y[j] = p.zero ? 0 : (uint8_t)quant1(x[j], p);
    }
}

// One wave per row; also emits the row sums of y (u8 summed as int32).
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
    const int lane = threadIdx.x & 63;
    const size_t wave = (size_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const size_t nwaves = (size_t)gridDim.x * (kThreads / 64);
    for (size_t r = wave; r < rows; r += nwaves) {
        const float* xr = x + r * row_len;
        uint8_t* yr = y + r * row_len;
        uint32_t s = 0;
        if (vec) {
            const float4* x4 = reinterpret_cast<const float4*>(xr);
            uint32_t* y4 = reinterpret_cast<uint32_t*>(yr);
#pragma unroll 4
            for (size_t i = lane; i < row_len / 4; i += 64) {
                uint32_t q = p.zero ? 0u : quant4(x4[i], p);
                y4[i] = q;
                s += (q & 0xFF) + ((q >> 8) & 0xFF) + ((q >> 16) & 0xFF) + (q >> 24);
            }
        } else {
            for (size_t i = lane; i < row_len; i += 64) {
                uint32_t q = p.zero ? 0u : quant1(xr[i], p);
                yr[i] = (uint8_t)q;
                s += q;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) rowsum[r] = (int32_t)s;
    }
}

}  // namespace

extern "C" size_t icx_dql_workspace_size(size_t) { return sizeof(float2) * kMaxPartials; }

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
    const int vec = icx::aligned16(x) ? 1 : 0;
    // Launch 1: enough blocks for ~16 float4 per lane, capped at kMaxPartials.
    int G = (int)std::min<size_t>(kMaxPartials, std::max<size_t>(1, icx::cdiv(n, (size_t)kThreads * 16)));
    hipLaunchKernelGGL(dql_minmax_kernel, dim3(G), dim3(kThreads), 0, s, x, n, vec, part);
    ICX_LAUNCH_CHECK("dql_minmax_kernel");
    if (opt_rowsum) {
        const size_t rows = n / row_len;
        const int rvec =
            (vec && row_len % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 3u) == 0) ? 1 : 0;
        const int blocks = (int)std::min<size_t>(2048, std::max<size_t>(1, icx::cdiv(rows, kThreads / 64)));
        hipLaunchKernelGGL(dql_quantize_rows_kernel, dim3(blocks), dim3(kThreads), 0, s, x, rows,
                           row_len, rvec, y, opt_rowsum, part, G, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_rows_kernel");
    } else {
        const int qvec = (vec && icx::aligned16(y)) ? 1 : 0;
        const int blocks = (int)std::min<size_t>(2048, std::max<size_t>(1, icx::cdiv(n, (size_t)kThreads * 16)));
        hipLaunchKernelGGL(dql_quantize_flat_kernel, dim3(blocks), dim3(kThreads), 0, s, x, n, qvec,
                           y, part, G, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_flat_kernel");
    }
    return ICX_OK;
}
