// HBM-bound elementwise kernels: the standalone fused chain, Cast INT32 -> FLOAT and
// DequantizeLinear, plus the library's error / version plumbing.
#include <cstring>

#include "chain.hpp"

namespace icx {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int validate_chain(const icx_chain* ch, const char* who) {
    if (ch->n_ops < 0 || ch->n_ops > ICX_MAX_CHAIN)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: chain length %d outside [0, %d]", who, ch->n_ops,
                 ICX_MAX_CHAIN);
    for (int i = 0; i < ch->n_ops; ++i) {
        const icx_chain_op& o = ch->ops[i];
        if (o.op < ICX_OP_ADD || o.op > ICX_OP_DIV)
            ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: chain op %d has unknown op code %d", who, i, o.op);
        if (!o.p0) ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: chain op %d has a null operand", who, i);
        if (o.kind0 < ICX_BCAST_SCALAR || o.kind0 > ICX_BCAST_FULL ||
            (o.p1 && (o.kind1 < ICX_BCAST_SCALAR || o.kind1 > ICX_BCAST_FULL)))
            ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: chain op %d has an unknown broadcast kind", who, i);
    }
    return ICX_OK;
}

}  // namespace icx

namespace {

constexpr int kThreads = 256;

// rows x cols, cols % 4 == 0, 16-byte aligned X / Y: one float4 per lane per step, four
// steps in flight.  Column operands are read through L1/L2 (a few KB, reused by every row).
__global__ void __launch_bounds__(kThreads)
chain_vec4_kernel(const float4* __restrict__ X, uint32_t n4, uint32_t cols4, size_t cols,
                  icx_chain ch, float4* __restrict__ Y) {
    const uint32_t stride = gridDim.x * kThreads;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const uint32_t r = i / cols4;
        const size_t c = (size_t)(i - r * cols4) * 4;
        float4 v = X[i];
        v.x = icx::apply_chain(ch, v.x, r, c + 0, cols);
        v.y = icx::apply_chain(ch, v.y, r, c + 1, cols);
        v.z = icx::apply_chain(ch, v.z, r, c + 2, cols);
        v.w = icx::apply_chain(ch, v.w, r, c + 3, cols);
        Y[i] = v;
    }
}

__global__ void __launch_bounds__(kThreads)
chain_scalar_kernel(const float* __restrict__ X, size_t n, size_t cols, icx_chain ch,
                    float* __restrict__ Y) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const size_t r = i / cols, c = i - r * cols;
        Y[i] = icx::apply_chain(ch, X[i], r, c, cols);
    }
}

__global__ void __launch_bounds__(kThreads)
cast_i32_f32_kernel(const int32_t* __restrict__ x, size_t n, float* __restrict__ y) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        y[i] = (float)x[i];  // v_cvt_f32_i32: round to nearest even
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
dequantize_kernel(const T* __restrict__ x, const float* __restrict__ scale,
                  const T* __restrict__ zp, size_t n, size_t axis_size, size_t inner,
                  float* __restrict__ y) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const size_t a = axis_size == 1 ? 0 : (i / inner) % axis_size;
        const float xf = (float)x[i];
        const float zf = zp ? (float)zp[a] : 0.0f;
        y[i] = __fmul_rn(__fsub_rn(xf, zf), scale[a]);
    }
}

unsigned grid_for(size_t work, size_t per_block, unsigned cap) {
    size_t b = icx::cdiv(work, per_block);
    if (b < 1) b = 1;
    return (unsigned)(b > cap ? cap : b);
}

}  // namespace

extern "C" const char* icx_status_str(int status) {
    switch (status) {
        case ICX_OK: return "ok";
        case ICX_ERR_INVALID_ARG: return "invalid argument";
        case ICX_ERR_SHAPE: return "shape mismatch";
        case ICX_ERR_DTYPE: return "unsupported dtype";
        case ICX_ERR_WORKSPACE: return "workspace too small";
        case ICX_ERR_HIP: return "HIP runtime error";
        case ICX_ERR_UNSUPPORTED: return "unsupported";
        default: return "unknown status";
    }
}

extern "C" const char* icx_last_error(void) { return icx::g_err; }

extern "C" const char* icx_version(void) {
    return "iconnx_hip 0.1 gfx950 (int8 MFMA 32x32x32, LDS double-buffered)";
}

extern "C" int icx_fused_chain_f32(icx_stream_t stream, const float* X, size_t rows,
                                   size_t cols, const icx_chain* chain, float* Y) {
    icx::clear_error();
    if (!X || !Y || !chain) ICX_FAIL(ICX_ERR_INVALID_ARG, "fused_chain: null pointer argument");
    int rc = icx::validate_chain(chain, "fused_chain");
    if (rc) return rc;
    const size_t n = rows * cols;
    if (n == 0) return ICX_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (cols % 4 == 0 && icx::aligned16(X) && icx::aligned16(Y) && n / 4 < 0xffffffffull) {
        const uint32_t n4 = (uint32_t)(n / 4);
        hipLaunchKernelGGL(chain_vec4_kernel, dim3(grid_for(n4, kThreads * 4, 8192)), dim3(kThreads),
                           0, s, reinterpret_cast<const float4*>(X), n4, (uint32_t)(cols / 4), cols,
                           *chain, reinterpret_cast<float4*>(Y));
        ICX_LAUNCH_CHECK("chain_vec4_kernel");
    } else {
        hipLaunchKernelGGL(chain_scalar_kernel, dim3(grid_for(n, kThreads * 4, 8192)), dim3(kThreads),
                           0, s, X, n, cols, *chain, Y);
        ICX_LAUNCH_CHECK("chain_scalar_kernel");
    }
    return ICX_OK;
}

extern "C" int icx_cast_i32_f32(icx_stream_t stream, const int32_t* x, size_t n, float* y) {
    icx::clear_error();
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Cast: null pointer argument");
    if (n == 0) return ICX_OK;
    hipLaunchKernelGGL(cast_i32_f32_kernel, dim3(grid_for(n, kThreads * 4, 8192)), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, n, y);
    ICX_LAUNCH_CHECK("cast_i32_f32_kernel");
    return ICX_OK;
}

extern "C" int icx_dequantize_linear_f32(icx_stream_t stream, const void* x, int x_dtype,
                                         const float* scale, const void* zp, size_t n,
                                         size_t axis_size, size_t inner, float* y) {
    icx::clear_error();
    if (!x || !scale || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "DequantizeLinear: null pointer argument");
    if (axis_size == 0 || inner == 0)
        ICX_FAIL(ICX_ERR_SHAPE, "DequantizeLinear: axis_size and inner must be positive");
    if (n == 0) return ICX_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(grid_for(n, kThreads * 4, 8192)), block(kThreads);
    switch (x_dtype) {
        case ICX_I8:
            hipLaunchKernelGGL(dequantize_kernel<int8_t>, grid, block, 0, s,
                               reinterpret_cast<const int8_t*>(x), scale,
                               reinterpret_cast<const int8_t*>(zp), n, axis_size, inner, y);
            break;
        case ICX_U8:
            hipLaunchKernelGGL(dequantize_kernel<uint8_t>, grid, block, 0, s,
                               reinterpret_cast<const uint8_t*>(x), scale,
                               reinterpret_cast<const uint8_t*>(zp), n, axis_size, inner, y);
            break;
        case ICX_I32:
            hipLaunchKernelGGL(dequantize_kernel<int32_t>, grid, block, 0, s,
                               reinterpret_cast<const int32_t*>(x), scale,
                               reinterpret_cast<const int32_t*>(zp), n, axis_size, inner, y);
            break;
        default:
            ICX_FAIL(ICX_ERR_DTYPE, "DequantizeLinear: input dtype %d unsupported (must be Int8, UInt8, or Int32)", x_dtype);
    }
    ICX_LAUNCH_CHECK("dequantize_kernel");
    return ICX_OK;
}
