// MatMulInteger on gfx950 int8 MFMA, with the dequant / bias / elementwise epilogue fused
// into the store.
//
// Operand handling.  MFMA int8 multiplies signed bytes only, so unsigned operands are
// shifted into i8: a' = a - alpha, b' = b - beta (alpha, beta = 128 for u8, 0 for i8; the
// shift is an XOR with 0x80 per byte).  Then, exactly in (wrapping) int32,
//
//   sum_k (a - azp)(b - bzp_n) = sum_k a'b'  +  (beta - bzp_n) * Ra'_m
//                              + (alpha - azp) * Cb'_n + K (alpha - azp)(beta - bzp_n)
//
// with Ra'_m = sum_k a'[m,k] (from the raw row sum: Ra - alpha*K) and Cb'_n the column sum
// of b' computed once when the weight is packed.  The identity holds modulo 2^32, so the
// result equals the reference GPU kernel's wrapping accumulator too
// (src/cuda/ops/quantize_kernels.rs:136-154) and the checked CPU forward
// (src/operators/matmul_integer.rs:239-267) whenever that one does not panic.
//
// Weights are packed once to B'^T [N,K] (K contiguous) so A and B tiles have the same
// shape: the kernel is an "NT" GEMM whose 16-byte global loads and 16-byte LDS fragment
// reads are all contiguous.
//
// Tiling (v1): 256 threads = 4 waves (2x2), block tile 128x128, K step 64, LDS double
// buffered (2 x 2 x 128 x 80 B = 40 KB, rows padded by 16 B), each wave a 64x64 sub-tile
// of 2x2 v_mfma_i32_32x32x32_i8.  Blocks are remapped so each XCD (blockIdx % 8) works on
// a contiguous, M-grouped range of tiles that shares A/B panels in its own L2.
#include "chain.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 16;  // bytes per LDS row (padding against bank conflicts)
constexpr int GROUP_M = 8;

enum { OUT_I32 = 0, OUT_F32 = 1 };

struct GemmArgs {
    const int8_t* A;   // [M,K] raw (u8 or i8 bytes)
    const int8_t* Bp;  // packed [N,K] i8 (already shifted)
    void* C;           // int32 or float [M,N]
    const int32_t* colsum;      // Cb'[N]
    const int32_t* rowsum_raw;  // Ra[M] (raw A bytes) or null when not needed
    const void* a_zp;           // scalar (A dtype) or null
    const void* b_zp;           // [b_zp_len] (B dtype) or null
    int M, N, K;
    int tiles_m, tiles_n;
    uint32_t a_xor;  // 0x80808080 when A is u8
    int alpha, beta;
    int a_zp_u8, b_zp_u8, b_zp_len;
    icx_chain chain;
};

__device__ __forceinline__ int load_zp(const void* p, int is_u8, int idx) {
    if (!p) return 0;
    return is_u8 ? (int)reinterpret_cast<const uint8_t*>(p)[idx]
                 : (int)reinterpret_cast<const int8_t*>(p)[idx];
}

// 16 bytes of row `row` starting at column `k` of a [rows, K] byte matrix; zero outside.
template <bool VEC>
__device__ __forceinline__ uint4 load16(const int8_t* base, int rows, int K, int row, int k,
                                        uint32_t xr) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row >= rows) return v;
    const int8_t* p = base + (size_t)row * K + k;
    if (VEC) {
        if (k < K) {
            v = *reinterpret_cast<const uint4*>(p);
            v.x ^= xr; v.y ^= xr; v.z ^= xr; v.w ^= xr;
        }
    } else {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (k + j < K) {
                uint32_t b = (uint8_t)p[j] ^ (xr & 0xFFu);
                w[j >> 2] |= b << (8 * (j & 3));
            }
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    return v;
}

template <bool VEC, int OUT>
__global__ void __launch_bounds__(kThreads) gemm_i8_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * LDS_STRIDE];

    // ---- tile assignment: XCD-contiguous, then GROUP_M-grouped ------------------------
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int per_group = GROUP_M * g.tiles_n;
    const int group = bid / per_group;
    const int first_m = group * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int in_group = bid - group * per_group;
    const int tm = first_m + in_group % gsz;
    const int tn = in_group / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int lr = lane & 31, lk = (lane >> 5) * 16;

    // global -> register staging: 2 chunks of 16 B per operand per thread
    const int r0 = t >> 2, c0 = (t & 3) * 16;  // chunk t
    const int r1 = r0 + 64;                     // chunk t + 256
    uint4 ra0, ra1, rb0, rb1;

    auto gload = [&](int k0) {
        ra0 = load16<VEC>(g.A, g.M, g.K, m0 + r0, k0 + c0, g.a_xor);
        ra1 = load16<VEC>(g.A, g.M, g.K, m0 + r1, k0 + c0, g.a_xor);
        rb0 = load16<VEC>(g.Bp, g.N, g.K, n0 + r0, k0 + c0, 0u);
        rb1 = load16<VEC>(g.Bp, g.N, g.K, n0 + r1, k0 + c0, 0u);
    };
    auto sstore = [&](int st) {
        *reinterpret_cast<uint4*>(&sA[st][r0 * LDS_STRIDE + c0]) = ra0;
        *reinterpret_cast<uint4*>(&sA[st][r1 * LDS_STRIDE + c0]) = ra1;
        *reinterpret_cast<uint4*>(&sB[st][r0 * LDS_STRIDE + c0]) = rb0;
        *reinterpret_cast<uint4*>(&sB[st][r1 * LDS_STRIDE + c0]) = rb1;
    };

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int KT = (g.K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int8_t* pa = &sA[cur][(wm * 64 + lr) * LDS_STRIDE + ks * 32 + lk];
            const int8_t* pb = &sB[cur][(wn * 64 + lr) * LDS_STRIDE + ks * 32 + lk];
            v4i a0 = *reinterpret_cast<const v4i*>(pa);
            v4i a1 = *reinterpret_cast<const v4i*>(pa + 32 * LDS_STRIDE);
            v4i b0 = *reinterpret_cast<const v4i*>(pb);
            v4i b1 = *reinterpret_cast<const v4i*>(pb + 32 * LDS_STRIDE);
            acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: zero-point correction, then int32 store or Cast + chain ------------
    const int azp = load_zp(g.a_zp, g.a_zp_u8, 0);
    const uint32_t amz = (uint32_t)(g.alpha - azp);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = n0 + wn * 64 + j * 32 + lr;
        if (col >= g.N) continue;
        const int bzp = load_zp(g.b_zp, g.b_zp_u8, g.b_zp_len == 1 ? 0 : col);
        const uint32_t colfac = (uint32_t)(g.beta - bzp);
        const uint32_t colterm =
            amz * (uint32_t)g.colsum[col] + (uint32_t)g.K * amz * colfac;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= g.M) continue;
                uint32_t v = (uint32_t)acc[i][j][r] + colterm;
                if (g.rowsum_raw) {
                    const uint32_t ra = (uint32_t)g.rowsum_raw[row] - (uint32_t)g.alpha * (uint32_t)g.K;
                    v += colfac * ra;
                }
                const size_t off = (size_t)row * g.N + col;
                if (OUT == OUT_I32) {
                    reinterpret_cast<int32_t*>(g.C)[off] = (int32_t)v;
                } else {
                    float f = (float)(int32_t)v;  // Cast INT32 -> FLOAT, round to nearest even
                    f = icx::apply_chain(g.chain, f, row, col, g.N);
                    reinterpret_cast<float*>(g.C)[off] = f;
                }
            }
        }
    }
}

// ---- weight packing -------------------------------------------------------------------
// B [K,N] -> packed[N][K] = B^T - beta (i8).  64x64 byte tiles through LDS.
__global__ void __launch_bounds__(kThreads)
pack_weight_kernel(const uint8_t* __restrict__ B, int K, int N, uint32_t xr,
                   int8_t* __restrict__ packed) {
    __shared__ uint8_t tile[64][64 + 4];
    const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int t = threadIdx.x;
    // load: 64 rows (k) x 64 bytes (n); thread t covers row t/4, 16 bytes at (t%4)*16
    {
        const int kr = t >> 2, nc = (t & 3) * 16;
        const int k = k0 + kr;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int n = n0 + nc + j;
            tile[kr][nc + j] = (k < K && n < N) ? (uint8_t)(B[(size_t)k * N + n] ^ (xr & 0xFF)) : 0;
        }
    }
    __syncthreads();
    // store: packed row n = n0 + t/4, bytes k0 + (t%4)*16 .. +16
    {
        const int nr = t >> 2, kc = (t & 3) * 16;
        const int n = n0 + nr;
        if (n < N) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int k = k0 + kc + j;
                if (k < K) packed[(size_t)n * K + k] = (int8_t)tile[kc + j][nr];
            }
        }
    }
}

// Sum of each packed row (== column sums of b'), one wave per row.
__global__ void __launch_bounds__(kThreads)
packed_colsum_kernel(const int8_t* __restrict__ packed, int K, int N, int32_t* __restrict__ colsum) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (n >= N) return;
    const int8_t* p = packed + (size_t)n * K;
    int s = 0;
    for (int k = lane; k < K; k += 64) s += (int)p[k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) colsum[n] = s;
}

// Raw row sums of A (bytes as u8 or i8), one wave per row.
__global__ void __launch_bounds__(kThreads)
rowsum_kernel(const void* __restrict__ A, int is_u8, int M, int K, int32_t* __restrict__ rowsum) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (m >= M) return;
    int s = 0;
    if (is_u8) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(A) + (size_t)m * K;
        for (int k = lane; k < K; k += 64) s += (int)p[k];
    } else {
        const int8_t* p = reinterpret_cast<const int8_t*>(A) + (size_t)m * K;
        for (int k = lane; k < K; k += 64) s += (int)p[k];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) rowsum[m] = s;
}

// Workspace layout for icx_matmul_integer / icx_qlinear_f32.
struct WsLayout {
    size_t packed_off, colsum_off, rowsum_off, total;
};

WsLayout ws_layout(size_t M, size_t K, size_t N, int b_packed) {
    WsLayout w{};
    size_t off = 0;
    if (!b_packed) {
        w.packed_off = off;
        off = icx::align_up(off + N * K, 256);
        w.colsum_off = off;
        off = icx::align_up(off + 4 * N, 256);
    }
    w.rowsum_off = off;
    off = icx::align_up(off + 4 * M, 256);
    w.total = off;
    return w;
}

int pack_weight_impl(hipStream_t s, const void* B, int b_dtype, size_t K, size_t N,
                     int8_t* packed, int32_t* colsum) {
    const uint32_t xr = b_dtype == ICX_U8 ? 0x80808080u : 0u;
    if (K > 0 && N > 0) {
        dim3 grid((unsigned)icx::cdiv(N, 64), (unsigned)icx::cdiv(K, 64));
        hipLaunchKernelGGL(pack_weight_kernel, grid, dim3(kThreads), 0, s,
                           reinterpret_cast<const uint8_t*>(B), (int)K, (int)N, xr, packed);
        ICX_LAUNCH_CHECK("pack_weight_kernel");
    }
    if (N > 0) {
        hipLaunchKernelGGL(packed_colsum_kernel, dim3((unsigned)icx::cdiv(N, kThreads / 64)),
                           dim3(kThreads), 0, s, packed, (int)K, (int)N, colsum);
        ICX_LAUNCH_CHECK("packed_colsum_kernel");
    }
    return ICX_OK;
}

int gemm_common(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype,
                int b_packed, const int32_t* b_colsum, size_t M, size_t K, size_t N,
                const void* a_zp, const void* b_zp, size_t b_zp_len, const int32_t* a_rowsum,
                const icx_chain* chain, void* C, int out_kind, void* ws, size_t ws_bytes,
                const char* who) {
    if (!A || !B || !C) ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: null A, B or output pointer", who);
    if (!icx::is_int8_kind(a_dtype))
        ICX_FAIL(ICX_ERR_DTYPE, "%s: a dtype %d unsupported (must be Int8 or UInt8)", who, a_dtype);
    if (!icx::is_int8_kind(b_dtype))
        ICX_FAIL(ICX_ERR_DTYPE, "%s: b dtype %d unsupported (must be Int8 or UInt8)", who, b_dtype);
    if (b_zp && b_zp_len != 1 && b_zp_len != N)
        ICX_FAIL(ICX_ERR_SHAPE, "%s: b_zero_point length %zu must be 1 or N = %zu", who, b_zp_len, N);
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff)
        ICX_FAIL(ICX_ERR_SHAPE, "%s: dimensions must fit in int32", who);
    if (b_packed && !b_colsum)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: packed weights need their colsum", who);
    if (chain) {
        int rc = icx::validate_chain(chain, who);
        if (rc) return rc;
    }
    const WsLayout L = ws_layout(M, K, N, b_packed);
    if (M == 0 || N == 0) return ICX_OK;
    if (!ws || ws_bytes < L.total)
        ICX_FAIL(ICX_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)", who, L.total, ws_bytes);

    char* wsb = reinterpret_cast<char*>(ws);
    const int8_t* Bp = reinterpret_cast<const int8_t*>(B);
    const int32_t* colsum = b_colsum;
    if (!b_packed) {
        int8_t* pk = reinterpret_cast<int8_t*>(wsb + L.packed_off);
        int32_t* cs = reinterpret_cast<int32_t*>(wsb + L.colsum_off);
        int rc = pack_weight_impl(s, B, b_dtype, K, N, pk, cs);
        if (rc) return rc;
        Bp = pk;
        colsum = cs;
    }
    const int alpha = a_dtype == ICX_U8 ? 128 : 0;
    const int beta = b_dtype == ICX_U8 ? 128 : 0;
    // The row term is needed unless beta - bzp_n == 0 for every n.  With a device-side zp
    // the value is unknown on the host, so any present b_zp (or a u8 B) requires it.
    const bool need_rowsum = (beta != 0) || (b_zp != nullptr);
    const int32_t* rowsum = nullptr;
    if (need_rowsum) {
        if (a_rowsum) {
            rowsum = a_rowsum;
        } else {
            int32_t* rs = reinterpret_cast<int32_t*>(wsb + L.rowsum_off);
            hipLaunchKernelGGL(rowsum_kernel, dim3((unsigned)icx::cdiv(M, kThreads / 64)),
                               dim3(kThreads), 0, s, A, a_dtype == ICX_U8 ? 1 : 0, (int)M,
                               (int)K, rs);
            ICX_LAUNCH_CHECK("rowsum_kernel");
            rowsum = rs;
        }
    }

    GemmArgs g{};
    g.A = reinterpret_cast<const int8_t*>(A);
    g.Bp = Bp;
    g.C = C;
    g.colsum = colsum;
    g.rowsum_raw = rowsum;
    g.a_zp = a_zp;
    g.b_zp = b_zp;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.tiles_m = (int)icx::cdiv(M, BM);
    g.tiles_n = (int)icx::cdiv(N, BN);
    g.a_xor = a_dtype == ICX_U8 ? 0x80808080u : 0u;
    g.alpha = alpha;
    g.beta = beta;
    g.a_zp_u8 = a_dtype == ICX_U8;
    g.b_zp_u8 = b_dtype == ICX_U8;
    g.b_zp_len = (int)(b_zp ? b_zp_len : 1);
    if (chain) g.chain = *chain;
    else g.chain.n_ops = 0;

    const bool vec = (K % 16 == 0) && icx::aligned16(A) && icx::aligned16(Bp);
    const unsigned blocks = (unsigned)(g.tiles_m * g.tiles_n);
    if (out_kind == OUT_I32) {
        if (vec) hipLaunchKernelGGL((gemm_i8_kernel<true, OUT_I32>), dim3(blocks), dim3(kThreads), 0, s, g);
        else hipLaunchKernelGGL((gemm_i8_kernel<false, OUT_I32>), dim3(blocks), dim3(kThreads), 0, s, g);
    } else {
        if (vec) hipLaunchKernelGGL((gemm_i8_kernel<true, OUT_F32>), dim3(blocks), dim3(kThreads), 0, s, g);
        else hipLaunchKernelGGL((gemm_i8_kernel<false, OUT_F32>), dim3(blocks), dim3(kThreads), 0, s, g);
    }
    ICX_LAUNCH_CHECK("gemm_i8_kernel");
    return ICX_OK;
}

}  // namespace

extern "C" size_t icx_packed_weight_bytes(size_t K, size_t N) { return K * N; }

extern "C" int icx_pack_weight(icx_stream_t stream, const void* B, int b_dtype, size_t K,
                               size_t N, int8_t* packed, int32_t* colsum) {
    icx::clear_error();
    if (!B || !packed || !colsum) ICX_FAIL(ICX_ERR_INVALID_ARG, "pack_weight: null pointer");
    if (!icx::is_int8_kind(b_dtype))
        ICX_FAIL(ICX_ERR_DTYPE, "pack_weight: b dtype %d unsupported (must be Int8 or UInt8)", b_dtype);
    if (K > 0x7fffffff || N > 0x7fffffff) ICX_FAIL(ICX_ERR_SHAPE, "pack_weight: dims exceed int32");
    return pack_weight_impl(reinterpret_cast<hipStream_t>(stream), B, b_dtype, K, N, packed, colsum);
}

extern "C" size_t icx_matmul_integer_workspace_size(size_t M, size_t K, size_t N, int b_packed) {
    return ws_layout(M, K, N, b_packed).total;
}

extern "C" int icx_matmul_integer(icx_stream_t stream, const void* A, int a_dtype,
                                  const void* B, int b_dtype, int b_packed,
                                  const int32_t* b_colsum, size_t M, size_t K, size_t N,
                                  const void* a_zp, const void* b_zp, size_t b_zp_len,
                                  const int32_t* a_rowsum, int32_t* C, void* ws,
                                  size_t ws_bytes) {
    icx::clear_error();
    return gemm_common(reinterpret_cast<hipStream_t>(stream), A, a_dtype, B, b_dtype, b_packed,
                       b_colsum, M, K, N, a_zp, b_zp, b_zp_len, a_rowsum, nullptr, C, OUT_I32,
                       ws, ws_bytes, "MatMulInteger");
}

extern "C" int icx_qlinear_f32(icx_stream_t stream, const void* A, int a_dtype, const void* B,
                               int b_dtype, int b_packed, const int32_t* b_colsum, size_t M,
                               size_t K, size_t N, const void* a_zp, const void* b_zp,
                               size_t b_zp_len, const int32_t* a_rowsum,
                               const icx_chain* chain, float* Y, void* ws, size_t ws_bytes) {
    icx::clear_error();
    return gemm_common(reinterpret_cast<hipStream_t>(stream), A, a_dtype, B, b_dtype, b_packed,
                       b_colsum, M, K, N, a_zp, b_zp, b_zp_len, a_rowsum, chain, Y, OUT_F32, ws,
                       ws_bytes, "QLinear");
}
