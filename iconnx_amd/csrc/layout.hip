// Data-movement and mask kernels for the shape plumbing of an exported encoder (the
// DistilBERT-INT8 export's reshape targets, position ids and attention mask), which the graph
// executor runs on device tensors:
//   * one strided copy for Slice, Expand and each input of Concat (gpu_slice_nd / gpu_expand /
//     gpu_concat, src/cuda/ops/layout/mod.rs),
//   * Equal with broadcasting, to Bool (gpu_equal via elementwise.rs:333),
//   * Where with three-way broadcasting (layout.rs:62-134, which materialises every operand to
//     the output shape first; here the broadcast is in the index arithmetic),
//   * Cast between the integer, Bool and Float32 types of those graphs (src/operators/cast.rs),
//   * Add / Sub / Mul / Div of f32 tensors under broadcasting the fused chain kernel does not
//     cover (the position embeddings [1, S, D] added to [B, S, D]),
//   * the upload of a small tensor computed on the host (Shape results and what the executor
//     folds from them) through kernel arguments, so that a captured graph replays it.
// All of them move at most a few MB per call, once per layer at most: they are written for
// correctness on any rank (up to 8), stride and element size, with the output dimensions
// merged on the host wherever every operand's strides allow, not tuned.
#include <hip/hip_runtime.h>

#include <cstring>

#include "icx_common.hpp"
#include "internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxOps = 3;

// Output dimensions and, per operand, the element stride of each dimension (0 where the
// operand is broadcast); operand 0 of a strided copy is the output itself.
template <typename I>
struct Nd {
    int rank;
    I dims[icx::kLayoutMaxRank];
    I st[kMaxOps][icx::kLayoutMaxRank];
    I off[kMaxOps];
};

template <typename I, int NOPS>
__device__ __forceinline__ void offsets_of(const Nd<I>& nd, I e, I (&o)[NOPS]) {
#pragma unroll
    for (int k = 0; k < NOPS; ++k) o[k] = nd.off[k];
    for (int d = nd.rank - 1; d >= 0; --d) {
        const I n = nd.dims[d];
        const I i = d ? e % n : e;
        e = d ? e / n : e;
#pragma unroll
        for (int k = 0; k < NOPS; ++k) o[k] += i * nd.st[k][d];
    }
}

template <typename T, typename I>
__global__ void __launch_bounds__(kThreads)
strided_copy_kernel(const T* __restrict__ x, T* __restrict__ y, Nd<I> nd, I total) {
    for (I e = (I)blockIdx.x * kThreads + threadIdx.x; e < total; e += (I)gridDim.x * kThreads) {
        I o[2];
        offsets_of<I, 2>(nd, e, o);
        y[o[0]] = x[o[1]];
    }
}

template <typename T, typename I>
__global__ void __launch_bounds__(kThreads)
equal_kernel(const T* __restrict__ a, const T* __restrict__ b, uint8_t* __restrict__ y, Nd<I> nd, I total) {
    for (I e = (I)blockIdx.x * kThreads + threadIdx.x; e < total; e += (I)gridDim.x * kThreads) {
        I o[2];
        offsets_of<I, 2>(nd, e, o);
        y[e] = a[o[0]] == b[o[1]] ? 1 : 0;
    }
}

template <typename T, typename I>
__global__ void __launch_bounds__(kThreads)
where_kernel(const uint8_t* __restrict__ c, const T* __restrict__ x, const T* __restrict__ yv, T* __restrict__ out,
             Nd<I> nd, I total) {
    for (I e = (I)blockIdx.x * kThreads + threadIdx.x; e < total; e += (I)gridDim.x * kThreads) {
        I o[3];
        offsets_of<I, 3>(nd, e, o);
        out[e] = c[o[0]] ? x[o[1]] : yv[o[2]];
    }
}

// Rust's `as`: integers wrap or widen, integers to Float32 round to nearest even, Float32 to
// an integer type is NaN -> 0, saturating, else toward zero.
// Add / Sub / Mul / Div of two f32 tensors under general numpy broadcasting, one IEEE
// rounding per element (the reference's ops after maybe_expand, src/cuda/executor/
// elementwise.rs:54-200).
template <typename I>
__global__ void __launch_bounds__(kThreads)
binary_f32_kernel(int op, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y, Nd<I> nd,
                  I total) {
    for (I e = (I)blockIdx.x * kThreads + threadIdx.x; e < total; e += (I)gridDim.x * kThreads) {
        I o[2];
        offsets_of<I, 2>(nd, e, o);
        const float u = a[o[0]], v = b[o[1]];
        y[e] = op == ICX_OP_ADD ? __fadd_rn(u, v) : op == ICX_OP_SUB ? __fsub_rn(u, v)
             : op == ICX_OP_MUL ? __fmul_rn(u, v) : __fdiv_rn(u, v);
    }
}

template <typename S, typename D>
__device__ __forceinline__ D convert(S v) {
    return (D)v;
}
template <>
__device__ __forceinline__ int64_t convert<float, int64_t>(float v) {
    return v != v ? 0 : v <= -9223372036854775808.0f ? INT64_MIN : v >= 9223372036854775808.0f ? INT64_MAX : (int64_t)v;
}
template <>
__device__ __forceinline__ int32_t convert<float, int32_t>(float v) {
    return v != v ? 0 : v <= -2147483648.0f ? INT32_MIN : v >= 2147483648.0f ? INT32_MAX : (int32_t)v;
}

template <typename S, typename D>
__global__ void __launch_bounds__(kThreads)
cast_kernel(const S* __restrict__ x, D* __restrict__ y, size_t n, int to_bool) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (size_t)gridDim.x * kThreads) {
        const S v = x[i];
        y[i] = to_bool ? (D)(v != (S)0 ? 1 : 0) : convert<S, D>(v);
    }
}

constexpr int kUploadChunk = 2048;  // bytes per launch, passed as the kernel's argument
struct Chunk {
    unsigned char b[kUploadChunk];
};

__global__ void __launch_bounds__(kThreads) upload_kernel(Chunk c, unsigned char* __restrict__ dst, int n) {
    for (int i = threadIdx.x; i < n; i += kThreads) dst[i] = c.b[i];
}

constexpr int kMaxBlocks = 16384;

unsigned blocks_for(size_t total) {
    const size_t b = icx::cdiv(total, (size_t)kThreads);
    return (unsigned)(b < (size_t)kMaxBlocks ? (b ? b : 1) : (size_t)kMaxBlocks);
}

// Drop unit dimensions and merge neighbours that every operand walks contiguously, so that
// the per-element index arithmetic has as few divisions as the layout allows.
void merge_dims(int& rank, int64_t* dims, int64_t (*st)[icx::kLayoutMaxRank], int nops) {
    int r = 0;
    for (int d = 0; d < rank; ++d) {
        if (dims[d] == 1) continue;
        if (r > 0) {
            bool ok = true;
            for (int k = 0; k < nops; ++k) ok = ok && st[k][r - 1] == st[k][d] * dims[d];
            if (ok) {
                dims[r - 1] *= dims[d];
                for (int k = 0; k < nops; ++k) st[k][r - 1] = st[k][d];
                continue;
            }
        }
        dims[r] = dims[d];
        for (int k = 0; k < nops; ++k) st[k][r] = st[k][d];
        ++r;
    }
    if (r == 0) {  // a single element
        dims[0] = 1;
        for (int k = 0; k < nops; ++k) st[k][0] = 0;
        r = 1;
    }
    rank = r;
}

// Fill an Nd of index type I; false when some offset would not fit I.
template <typename I>
bool make_nd(Nd<I>& nd, int rank, const int64_t* dims, int64_t (*st)[icx::kLayoutMaxRank], const int64_t* off,
             int nops, int64_t total) {
    const int64_t lim = sizeof(I) == 4 ? (int64_t)0x7fffffff : INT64_MAX;
    // the grid-stride loop steps the element index past `total` by up to a grid's threads
    if (total > lim - (int64_t)kMaxBlocks * kThreads) return false;
    nd.rank = rank;
    for (int d = 0; d < rank; ++d) nd.dims[d] = (I)dims[d];
    for (int k = 0; k < kMaxOps; ++k) {
        nd.off[k] = k < nops ? (I)off[k] : 0;
        int64_t lo = k < nops ? off[k] : 0, hi = lo;
        for (int d = 0; d < rank; ++d) {
            const int64_t s = k < nops ? st[k][d] : 0;
            nd.st[k][d] = (I)s;
            const int64_t span = s * (dims[d] - 1);
            if (span < 0) lo += span; else hi += span;
        }
        if (lo < -lim || hi > lim) return false;
    }
    return true;
}

template <typename T, typename I>
void launch_copy(hipStream_t s, const void* x, void* y, const Nd<I>& nd, int64_t total) {
    hipLaunchKernelGGL((strided_copy_kernel<T, I>), dim3(blocks_for(total)), dim3(kThreads), 0, s,
                       static_cast<const T*>(x), static_cast<T*>(y), nd, (I)total);
}

template <typename I>
int copy_es(hipStream_t s, const void* x, void* y, size_t es, const Nd<I>& nd, int64_t total) {
    switch (es) {
        case 1: launch_copy<uint8_t, I>(s, x, y, nd, total); break;
        case 2: launch_copy<uint16_t, I>(s, x, y, nd, total); break;
        case 4: launch_copy<uint32_t, I>(s, x, y, nd, total); break;
        case 8: launch_copy<uint64_t, I>(s, x, y, nd, total); break;
        default: ICX_FAIL(ICX_ERR_DTYPE, "strided copy: element size %zu unsupported", es);
    }
    ICX_LAUNCH_CHECK("strided_copy_kernel");
    return ICX_OK;
}

template <typename T, typename I>
int launch_equal(hipStream_t s, const void* a, const void* b, uint8_t* y, const Nd<I>& nd, int64_t total) {
    hipLaunchKernelGGL((equal_kernel<T, I>), dim3(blocks_for(total)), dim3(kThreads), 0, s,
                       static_cast<const T*>(a), static_cast<const T*>(b), y, nd, (I)total);
    ICX_LAUNCH_CHECK("equal_kernel");
    return ICX_OK;
}

template <typename I>
int equal_dt(hipStream_t s, int dtype, const void* a, const void* b, uint8_t* y, const Nd<I>& nd, int64_t total) {
    switch (dtype) {
        case ICX_I8: return launch_equal<int8_t, I>(s, a, b, y, nd, total);
        case ICX_U8:
        case ICX_BOOL: return launch_equal<uint8_t, I>(s, a, b, y, nd, total);
        case ICX_I32: return launch_equal<int32_t, I>(s, a, b, y, nd, total);
        case ICX_F32: return launch_equal<float, I>(s, a, b, y, nd, total);
        case ICX_I64: return launch_equal<int64_t, I>(s, a, b, y, nd, total);
        default: ICX_FAIL(ICX_ERR_DTYPE, "Equal: dtype %d unsupported", dtype);
    }
}

template <typename T, typename I>
int launch_where(hipStream_t s, const uint8_t* c, const void* x, const void* yv, void* out, const Nd<I>& nd,
                 int64_t total) {
    hipLaunchKernelGGL((where_kernel<T, I>), dim3(blocks_for(total)), dim3(kThreads), 0, s, c,
                       static_cast<const T*>(x), static_cast<const T*>(yv), static_cast<T*>(out), nd, (I)total);
    ICX_LAUNCH_CHECK("where_kernel");
    return ICX_OK;
}

template <typename I>
int where_es(hipStream_t s, size_t es, const uint8_t* c, const void* x, const void* yv, void* out, const Nd<I>& nd,
             int64_t total) {
    switch (es) {
        case 1: return launch_where<uint8_t, I>(s, c, x, yv, out, nd, total);
        case 2: return launch_where<uint16_t, I>(s, c, x, yv, out, nd, total);
        case 4: return launch_where<uint32_t, I>(s, c, x, yv, out, nd, total);
        case 8: return launch_where<uint64_t, I>(s, c, x, yv, out, nd, total);
        default: ICX_FAIL(ICX_ERR_DTYPE, "Where: element size %zu unsupported", es);
    }
}

int check_rank(int rank, const char* who) {
    if (rank < 0 || rank > icx::kLayoutMaxRank) ICX_FAIL(ICX_ERR_UNSUPPORTED, "%s: rank %d > %d", who, rank, icx::kLayoutMaxRank);
    return ICX_OK;
}

int64_t total_of(int rank, const int64_t* dims) {
    int64_t t = 1;
    for (int d = 0; d < rank; ++d) t *= dims[d];
    return t;
}

template <typename S, typename D>
int launch_cast(hipStream_t s, const void* x, void* y, size_t n, int to_bool) {
    hipLaunchKernelGGL((cast_kernel<S, D>), dim3(blocks_for(n)), dim3(kThreads), 0, s, static_cast<const S*>(x),
                       static_cast<D*>(y), n, to_bool);
    ICX_LAUNCH_CHECK("cast_kernel");
    return ICX_OK;
}

template <typename S>
int cast_from(hipStream_t s, const void* x, int dst, void* y, size_t n) {
    switch (dst) {
        case ICX_F32: return launch_cast<S, float>(s, x, y, n, 0);
        case ICX_I64: return launch_cast<S, int64_t>(s, x, y, n, 0);
        case ICX_I32: return launch_cast<S, int32_t>(s, x, y, n, 0);
        case ICX_BOOL: return launch_cast<S, uint8_t>(s, x, y, n, 1);
        default: ICX_FAIL(ICX_ERR_UNSUPPORTED, "Cast: target dtype %d unsupported", dst);
    }
}

}  // namespace

int icx::strided_copy(hipStream_t s, const void* x, void* y, size_t es, int rank, const int64_t* dims,
                      const int64_t* x_strides, int64_t x_off, const int64_t* y_strides, int64_t y_off) {
    if (int rc = check_rank(rank, "strided copy")) return rc;
    const int64_t total = total_of(rank, dims);
    if (total == 0) return ICX_OK;
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "strided copy: null pointer");
    int64_t d[kLayoutMaxRank], st[kMaxOps][kLayoutMaxRank];
    for (int i = 0; i < rank; ++i) {
        d[i] = dims[i];
        st[0][i] = y_strides[i];
        st[1][i] = x_strides[i];
    }
    int r = rank;
    merge_dims(r, d, st, 2);
    const int64_t off[2] = {y_off, x_off};
    Nd<int32_t> n32;
    if (make_nd(n32, r, d, st, off, 2, total)) return copy_es(s, x, y, es, n32, total);
    Nd<int64_t> n64;
    make_nd(n64, r, d, st, off, 2, total);
    return copy_es(s, x, y, es, n64, total);
}

int icx::compare_equal(hipStream_t s, int dtype, const void* a, const int64_t* a_strides, const void* b,
                       const int64_t* b_strides, int rank, const int64_t* dims, uint8_t* y) {
    if (int rc = check_rank(rank, "Equal")) return rc;
    const int64_t total = total_of(rank, dims);
    if (total == 0) return ICX_OK;
    if (!a || !b || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Equal: null pointer");
    int64_t d[kLayoutMaxRank], st[kMaxOps][kLayoutMaxRank];
    // the output is dense: its own strides ride along as a third operand so that merging
    // keeps y's flat index equal to the element index
    int64_t ys = 1;
    for (int i = rank - 1; i >= 0; --i) {
        d[i] = dims[i];
        st[0][i] = a_strides[i];
        st[1][i] = b_strides[i];
        st[2][i] = ys;
        ys *= dims[i];
    }
    int r = rank;
    merge_dims(r, d, st, 3);
    const int64_t off[2] = {0, 0};
    Nd<int32_t> n32;
    if (make_nd(n32, r, d, st, off, 2, total)) return equal_dt(s, dtype, a, b, y, n32, total);
    Nd<int64_t> n64;
    make_nd(n64, r, d, st, off, 2, total);
    return equal_dt(s, dtype, a, b, y, n64, total);
}

int icx::select_where(hipStream_t s, size_t es, const uint8_t* c, const int64_t* c_strides, const void* x,
                      const int64_t* x_strides, const void* yv, const int64_t* y_strides, int rank,
                      const int64_t* dims, void* out) {
    if (int rc = check_rank(rank, "Where")) return rc;
    const int64_t total = total_of(rank, dims);
    if (total == 0) return ICX_OK;
    if (!c || !x || !yv || !out) ICX_FAIL(ICX_ERR_INVALID_ARG, "Where: null pointer");
    // four operands (three inputs and the dense output) would not fit Nd's three stride
    // rows: merge only where the output is contiguous too, checked through a fourth row
    int64_t d[kLayoutMaxRank], st[kMaxOps + 1][kLayoutMaxRank];
    int64_t os = 1;
    for (int i = rank - 1; i >= 0; --i) {
        d[i] = dims[i];
        st[0][i] = c_strides[i];
        st[1][i] = x_strides[i];
        st[2][i] = y_strides[i];
        st[3][i] = os;
        os *= dims[i];
    }
    int r = rank;
    merge_dims(r, d, st, 4);
    const int64_t off[3] = {0, 0, 0};
    Nd<int32_t> n32;
    if (make_nd(n32, r, d, st, off, 3, total)) return where_es(s, es, c, x, yv, out, n32, total);
    Nd<int64_t> n64;
    make_nd(n64, r, d, st, off, 3, total);
    return where_es(s, es, c, x, yv, out, n64, total);
}

int icx::binary_f32(hipStream_t s, int op, const float* a, const int64_t* a_strides, const float* b,
                    const int64_t* b_strides, int rank, const int64_t* dims, float* y) {
    if (int rc = check_rank(rank, "binary op")) return rc;
    if (op < ICX_OP_ADD || op > ICX_OP_DIV) ICX_FAIL(ICX_ERR_INVALID_ARG, "binary op: code %d", op);
    const int64_t total = total_of(rank, dims);
    if (total == 0) return ICX_OK;
    if (!a || !b || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "binary op: null pointer");
    int64_t d[kLayoutMaxRank], st[kMaxOps][kLayoutMaxRank];
    int64_t ys = 1;
    for (int i = rank - 1; i >= 0; --i) {
        d[i] = dims[i];
        st[0][i] = a_strides[i];
        st[1][i] = b_strides[i];
        st[2][i] = ys;
        ys *= dims[i];
    }
    int r = rank;
    merge_dims(r, d, st, 3);
    const int64_t off[2] = {0, 0};
    Nd<int32_t> n32;
    if (make_nd(n32, r, d, st, off, 2, total)) {
        hipLaunchKernelGGL((binary_f32_kernel<int32_t>), dim3(blocks_for(total)), dim3(kThreads), 0, s, op, a, b, y,
                           n32, (int32_t)total);
    } else {
        Nd<int64_t> n64;
        make_nd(n64, r, d, st, off, 2, total);
        hipLaunchKernelGGL((binary_f32_kernel<int64_t>), dim3(blocks_for(total)), dim3(kThreads), 0, s, op, a, b, y,
                           n64, total);
    }
    ICX_LAUNCH_CHECK("binary_f32_kernel");
    return ICX_OK;
}

int icx::cast_any(hipStream_t s, int src, const void* x, int dst, void* y, size_t n) {
    if (n == 0) return ICX_OK;
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Cast: null pointer");
    switch (src) {
        case ICX_F32: return cast_from<float>(s, x, dst, y, n);
        case ICX_I64: return cast_from<int64_t>(s, x, dst, y, n);
        case ICX_I32: return cast_from<int32_t>(s, x, dst, y, n);
        case ICX_I8: return cast_from<int8_t>(s, x, dst, y, n);
        case ICX_U8:
        case ICX_BOOL: return cast_from<uint8_t>(s, x, dst, y, n);
        default: ICX_FAIL(ICX_ERR_UNSUPPORTED, "Cast: source dtype %d unsupported", src);
    }
}

int icx::upload_bytes(hipStream_t s, const void* host, size_t bytes, void* dev) {
    if (bytes == 0) return ICX_OK;
    if (!host || !dev) ICX_FAIL(ICX_ERR_INVALID_ARG, "upload: null pointer");
    if (bytes > kUploadMaxBytes) ICX_FAIL(ICX_ERR_UNSUPPORTED, "upload: %zu bytes > %zu", bytes, kUploadMaxBytes);
    for (size_t o = 0; o < bytes; o += kUploadChunk) {
        Chunk c;
        const size_t n = bytes - o < (size_t)kUploadChunk ? bytes - o : (size_t)kUploadChunk;
        std::memset(c.b, 0, sizeof(c.b));
        std::memcpy(c.b, static_cast<const unsigned char*>(host) + o, n);
        hipLaunchKernelGGL(upload_kernel, dim3(1), dim3(kThreads), 0, s, c, static_cast<unsigned char*>(dev) + o, (int)n);
        ICX_LAUNCH_CHECK("upload_kernel");
    }
    return ICX_OK;
}
