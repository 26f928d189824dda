// HBM-bound elementwise kernels: the standalone fused chain, Cast INT32 -> FLOAT and
// DequantizeLinear, plus the library's error / version plumbing.
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "chain.hpp"
#include "internal.hpp"

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
        if (o.op < ICX_OP_ADD || o.op > ICX_OP_MUL_SAVED)
            ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: chain op %d has unknown op code %d", who, i, o.op);
        if (o.op > ICX_OP_DIV) continue;  // operand-free step
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

// rows x cols with cols % 4 == 0 and 16-byte aligned X / Y.  The grid stride (in float4)
// is a multiple of cols / 4, so each thread always works on the same 4 columns: their
// chain operands are computed once into a thread-private LDS slot, and each step is four
// float4 loads in flight, the chain applied op by op (one uniform branch per op, straight
// IEEE arithmetic over the 16 values) and four float4 stores.
template <int MODE>
__global__ void __launch_bounds__(kThreads)
chain_cols_kernel(const float4* __restrict__ X, uint32_t n4, uint32_t cols4, icx_chain ch,
                  uint32_t codes, float4* __restrict__ Y) {
    __shared__ float4 sop[ICX_MAX_CHAIN][kThreads];
    const uint32_t i0 = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t stride = gridDim.x * kThreads;
    const size_t c = (size_t)(i0 % cols4) * 4;
    {
        float o[4][ICX_MAX_CHAIN];
#pragma unroll
        for (int e = 0; e < 4; ++e) icx::load_col_operands(ch, c + e, o[e]);
#pragma unroll
        for (int k = 0; k < ICX_MAX_CHAIN; ++k)
            if (k < ch.n_ops) sop[k][threadIdx.x] = make_float4(o[0][k], o[1][k], o[2][k], o[3][k]);
    }
    auto opnd = [&](int k) { return sop[k][threadIdx.x]; };
    uint32_t i = i0;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = X[i + u * stride];
        icx::run_chain4<MODE>(codes, ch.n_ops, v, opnd);
#pragma unroll
        for (int u = 0; u < 4; ++u) icx::store_nt(&Y[i + u * stride], v[u]);
    }
    for (; i < n4; i += stride) {
        float4 v[1] = {X[i]};
        icx::run_chain4<MODE>(codes, ch.n_ops, v, opnd);
        icx::store_nt(&Y[i], v[0]);
    }
}

// General layout: every operand fetched per element.
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

// Gather of whole rows: data viewed as [outer, axis_len, row] (row = the bytes of the inner
// dimensions), out as [outer, n_idx, row]; one wave per output row, VEC-byte chunks (16 when
// rows and pointers allow it).  An index is taken from the end when negative and clamped into
// [0, axis_len) when still outside, as the reference's gather kernels do.
template <int VEC>
__global__ void __launch_bounds__(kThreads)
gather_rows_kernel(const uint8_t* __restrict__ data, const void* __restrict__ indices, int idx64,
                   size_t n_idx, size_t axis_len, size_t row_bytes, size_t rows,
                   uint8_t* __restrict__ out) {
    typedef typename std::conditional<VEC == 16, uint4, typename std::conditional<VEC == 4, uint32_t,
                                                                                   uint8_t>::type>::type T;
    const int lane = threadIdx.x & 63;
    const size_t waves = (size_t)gridDim.x * (kThreads / 64);
    for (size_t r = (size_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); r < rows; r += waves) {
        const size_t o = r / n_idx, i = r - o * n_idx;
        long long k = idx64 ? reinterpret_cast<const long long*>(indices)[i]
                            : (long long)reinterpret_cast<const int*>(indices)[i];
        if (k < 0) k += (long long)axis_len;
        if (k < 0) k = 0;
        if (k >= (long long)axis_len) k = (long long)axis_len - 1;
        const T* src = reinterpret_cast<const T*>(data + (o * axis_len + (size_t)k) * row_bytes);
        T* dst = reinterpret_cast<T*>(out + r * row_bytes);
        const size_t n = row_bytes / VEC;
        for (size_t c = lane; c < n; c += 64) dst[c] = src[c];
    }
}

// Gather of rows of an 8-bit table [axis_len, cols] followed by its per-tensor
// DequantizeLinear, in one pass (an INT8 model's embedding lookup): y[r, c] =
// (float(table[k_r, c]) - float(zp)) * scale with dequantize_kernel's roundings, k_r under
// gather_rows_kernel's index rules; one wave per output row, four table bytes per lane step.
template <typename T>
__global__ void __launch_bounds__(kThreads)
gather_dequant_kernel(const T* __restrict__ table, const void* __restrict__ indices, int idx64, size_t n_idx,
                      size_t axis_len, size_t cols, const float* __restrict__ scale, const T* __restrict__ zp,
                      float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const size_t waves = (size_t)gridDim.x * (kThreads / 64);
    const float sc = scale[0], zf = zp ? (float)zp[0] : 0.0f;
    for (size_t r = (size_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); r < n_idx; r += waves) {
        long long k = idx64 ? reinterpret_cast<const long long*>(indices)[r]
                            : (long long)reinterpret_cast<const int*>(indices)[r];
        if (k < 0) k += (long long)axis_len;
        if (k < 0) k = 0;
        if (k >= (long long)axis_len) k = (long long)axis_len - 1;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(table + (size_t)k * cols);
        float4* dst = reinterpret_cast<float4*>(y + r * cols);
        for (size_t c = lane; c < cols / 4; c += 64) {
            const uint32_t v = src[c];
            float4 o;
            o.x = __fmul_rn(__fsub_rn((float)(T)(v & 0xff), zf), sc);
            o.y = __fmul_rn(__fsub_rn((float)(T)((v >> 8) & 0xff), zf), sc);
            o.z = __fmul_rn(__fsub_rn((float)(T)((v >> 16) & 0xff), zf), sc);
            o.w = __fmul_rn(__fsub_rn((float)(T)(v >> 24), zf), sc);
            dst[c] = o;
        }
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
        case ICX_ERR_KERNEL: return "kernel reported a failure on the device";
        default: return "unknown status";
    }
}

extern "C" const char* icx_last_error(void) { return icx::g_err; }

extern "C" const char* icx_version(void) {
    return "iconnx_hip 0.2 gfx950 (int8 MFMA 32x32x32, LDS-DMA multistage)";
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
    const size_t cols4 = cols / 4;
    // grid: a multiple of lcm(256, cols4) threads so the stride keeps each thread's columns
    size_t g = 1, a = kThreads, bq = cols4;
    while (bq) { size_t tt = a % bq; a = bq; bq = tt; }  // a = gcd(256, cols4)
    const size_t unit_blocks = cols4 ? cols4 / a : 1;    // lcm(256, cols4) / 256
    if (cols4) g = std::max<size_t>(1, 1024 / unit_blocks) * unit_blocks;
    if (cols % 4 == 0 && cols4 > 0 && icx::aligned16(X) && icx::aligned16(Y) &&
        n / 4 < 0x7fffffffull && icx::chain_is_col_only(*chain) && unit_blocks <= 8192) {
        if (icx::chain_mode(*chain) == 2)
            hipLaunchKernelGGL(chain_cols_kernel<2>, dim3((unsigned)g), dim3(kThreads), 0, s,
                               reinterpret_cast<const float4*>(X), (uint32_t)(n / 4), (uint32_t)cols4,
                               *chain, icx::chain_codes(*chain), reinterpret_cast<float4*>(Y));
        else
            hipLaunchKernelGGL(chain_cols_kernel<0>, dim3((unsigned)g), dim3(kThreads), 0, s,
                               reinterpret_cast<const float4*>(X), (uint32_t)(n / 4), (uint32_t)cols4,
                               *chain, icx::chain_codes(*chain), reinterpret_cast<float4*>(Y));
        ICX_LAUNCH_CHECK("chain_cols_kernel");
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

int icx::gather_dequant_f32(hipStream_t s, const void* table, int dtype, size_t axis_len, size_t cols,
                            const void* indices, int idx_dtype, size_t n_idx, const float* scale, const void* zp,
                            float* y) {
    if (dtype != ICX_U8 && dtype != ICX_I8)
        ICX_FAIL(ICX_ERR_DTYPE, "Gather+DequantizeLinear: table dtype %d (must be UInt8 or Int8)", dtype);
    if (idx_dtype != ICX_I64 && idx_dtype != ICX_I32)
        ICX_FAIL(ICX_ERR_DTYPE, "Gather+DequantizeLinear: indices dtype %d (must be Int64 or Int32)", idx_dtype);
    if (n_idx == 0 || cols == 0) return ICX_OK;
    if (axis_len == 0) ICX_FAIL(ICX_ERR_SHAPE, "Gather+DequantizeLinear: %zu indices into an empty table", n_idx);
    if (!table || !indices || !scale || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Gather+DequantizeLinear: null pointer");
    if (cols % 4 || (reinterpret_cast<uintptr_t>(table) & 3) || !icx::aligned16(y))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "Gather+DequantizeLinear: rows of %zu bytes or unaligned operands", cols);
    const dim3 grid(grid_for(n_idx, kThreads / 64, 8192)), block(kThreads);
    const int i64 = idx_dtype == ICX_I64;
    if (dtype == ICX_U8)
        hipLaunchKernelGGL(gather_dequant_kernel<uint8_t>, grid, block, 0, s, static_cast<const uint8_t*>(table),
                           indices, i64, n_idx, axis_len, cols, scale, static_cast<const uint8_t*>(zp), y);
    else
        hipLaunchKernelGGL(gather_dequant_kernel<int8_t>, grid, block, 0, s, static_cast<const int8_t*>(table),
                           indices, i64, n_idx, axis_len, cols, scale, static_cast<const int8_t*>(zp), y);
    ICX_LAUNCH_CHECK("gather_dequant_kernel");
    return ICX_OK;
}

extern "C" int icx_gather(icx_stream_t stream, const void* data, size_t elem_bytes, size_t outer,
                          size_t axis_len, size_t inner, const void* indices, int idx_dtype,
                          size_t n_idx, void* out) {
    icx::clear_error();
    if (idx_dtype != ICX_I64 && idx_dtype != ICX_I32)
        ICX_FAIL(ICX_ERR_DTYPE, "Gather: indices dtype %d unsupported (must be Int64 or Int32)", idx_dtype);
    if (elem_bytes == 0) ICX_FAIL(ICX_ERR_INVALID_ARG, "Gather: zero element size");
    const size_t rows = outer * n_idx, row_bytes = inner * elem_bytes;
    if (rows == 0 || row_bytes == 0) return ICX_OK;
    if (axis_len == 0) ICX_FAIL(ICX_ERR_SHAPE, "Gather: %zu indices into an empty axis", n_idx);
    if (!data || !indices || !out) ICX_FAIL(ICX_ERR_INVALID_ARG, "Gather: null pointer argument");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(grid_for(rows, kThreads / 64, 8192)), block(kThreads);
    const uintptr_t align = reinterpret_cast<uintptr_t>(data) | reinterpret_cast<uintptr_t>(out) | row_bytes;
    const auto* d = reinterpret_cast<const uint8_t*>(data);
    auto* o = reinterpret_cast<uint8_t*>(out);
    const int i64 = idx_dtype == ICX_I64;
    if (align % 16 == 0)
        hipLaunchKernelGGL(gather_rows_kernel<16>, grid, block, 0, s, d, indices, i64, n_idx, axis_len, row_bytes,
                           rows, o);
    else if (align % 4 == 0)
        hipLaunchKernelGGL(gather_rows_kernel<4>, grid, block, 0, s, d, indices, i64, n_idx, axis_len, row_bytes,
                           rows, o);
    else
        hipLaunchKernelGGL(gather_rows_kernel<1>, grid, block, 0, s, d, indices, i64, n_idx, axis_len, row_bytes,
                           rows, o);
    ICX_LAUNCH_CHECK("gather_rows_kernel");
    return ICX_OK;
}
