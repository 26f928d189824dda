// fp32 ops around the quantized linears of a DistilBERT-shaped encoder, on gfx950:
//
//   LayerNormalization (last axis, optionally of x + residual)
//       src/operators/layer_normalization.rs:25-80 — eight lanes per row, each summing the
//       strided slice x[j], x[j+8], ... in order, combined as ndarray 0.16's unrolled_fold
//       does (the reference's mean_axis over a contiguous axis); every step one f32
//       rounding, so the result is bit-identical to that restatement.
//   Softmax (last axis)            src/operators/softmax.rs:25-40, same reduction layout.
//   Transpose (rank <= 6)          src/operators/transpose.rs:10-40.
//   MatMul f32 (batched)           src/operators/matmul.rs:20-150; LDS-tiled FMA kernel.
//   Attention (fused)              the decomposed Reshape/Transpose/MatMul/scale/Softmax/
//       MatMul/Transpose/Reshape subgraph of a BERT self-attention, over [B, S, H*D]
//       activations, with fp32 MFMA (v_mfma_f32_16x16x4f32): two blocks per (batch, head),
//       each of four waves of 16 queries; S^T = K Q^T leaves every lane one query's scores in
//       the A-operand layout of the P V product, so the softmax stays in registers.
#include "chain.hpp"
#include "icx_common.hpp"
#include "internal.hpp"
#include "qexchange.hpp"
#include <cmath>

#include <algorithm>

namespace {

constexpr int kThreads = 256;

// ---- row reductions in the unrolled_fold order ------------------------------------------
// Lane j (0..7) of an 8-lane group holds partial p_j; every lane of the group returns
// acc = 0 + (p0+p4) + (p1+p5) + (p2+p6) + (p3+p7), before the leftover elements.
__device__ __forceinline__ float combine8(float p) {
    const float p0 = __shfl(p, 0, 8), p1 = __shfl(p, 1, 8), p2 = __shfl(p, 2, 8),
                p3 = __shfl(p, 3, 8), p4 = __shfl(p, 4, 8), p5 = __shfl(p, 5, 8),
                p6 = __shfl(p, 6, 8), p7 = __shfl(p, 7, 8);
    float acc = 0.0f;
    acc = __fadd_rn(acc, __fadd_rn(p0, p4));
    acc = __fadd_rn(acc, __fadd_rn(p1, p5));
    acc = __fadd_rn(acc, __fadd_rn(p2, p6));
    acc = __fadd_rn(acc, __fadd_rn(p3, p7));
    return acc;
}

__device__ __forceinline__ float ln_in(const float* x, const float* res, size_t i) {
    return res ? __fadd_rn(x[i], res[i]) : x[i];
}

// 32 rows per block: 8 rows per wave, 8 lanes per row.  res_rows != 0: the residual has that
// many rows, row r of x adding residual row r % res_rows (a [S, cols] table broadcast over a
// [B, S, cols] x, e.g. position embeddings).
__global__ void __launch_bounds__(kThreads)
layer_norm_kernel(const float* __restrict__ x, const float* __restrict__ res, size_t res_rows, size_t rows,
                  size_t cols, const float* __restrict__ scale, const float* __restrict__ bias,
                  float eps, float* __restrict__ y) {
    const int lane = threadIdx.x & 63, j = lane & 7;
    const size_t row = (size_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (row >= rows) return;  // a whole 8-lane group leaves together
    const float* xr = x + row * cols;
    const float* rr = res ? res + (res_rows ? row % res_rows : row) * cols : nullptr;
    const size_t n8 = cols / 8 * 8;
    const float fcols = (float)cols;
    // mean
    float p = 0.0f;
    for (size_t i = j; i < n8; i += 8) p = __fadd_rn(p, ln_in(xr, rr, i));
    float acc = combine8(p);
    for (size_t i = n8; i < cols; ++i) acc = __fadd_rn(acc, ln_in(xr, rr, i));
    const float mean = __fdiv_rn(acc, fcols);
    // variance of the centred values
    p = 0.0f;
    for (size_t i = j; i < n8; i += 8) {
        const float c = __fsub_rn(ln_in(xr, rr, i), mean);
        p = __fadd_rn(p, __fmul_rn(c, c));
    }
    acc = combine8(p);
    for (size_t i = n8; i < cols; ++i) {
        const float c = __fsub_rn(ln_in(xr, rr, i), mean);
        acc = __fadd_rn(acc, __fmul_rn(c, c));
    }
    const float var = __fdiv_rn(acc, fcols);
    const float sd = sqrtf(__fadd_rn(var, eps));  // correctly rounded (build flag), as f32::sqrt
    float* yr = y + row * cols;
    for (size_t i = j; i < cols; i += 8) {
        const float c = __fsub_rn(ln_in(xr, rr, i), mean);
        yr[i] = __fadd_rn(__fmul_rn(__fdiv_rn(c, sd), scale ? scale[i] : 1.0f), bias ? bias[i] : -0.0f);
    }
}

// The same arithmetic, in the same order, for the BERT hidden sizes (cols = 8 * PER): a
// block of four waves normalises ROWS (4 or 8) consecutive rows.  All four stage the rows
// (x + residual, formed once) into LDS with float4 loads; the first 8·ROWS lanes of wave 0
// then run the order-fixed reductions — lane (r, j) walks its strided partial x[j], x[j+8],
// ... of row r from LDS into registers — and leave each row's mean and standard deviation in
// LDS; the output pass, independent per element, is spread over all 256 lanes with
// coalesced stores.  A staged row is cols + 8 floats long, so the strided reads of the rows
// fall into distinct banks.  Every block is resident at once and its phases (loads, the
// serial reductions, stores) are latency-bound, so more, smaller blocks finish sooner: 4 rows
// per block where the range partials allow it.
template <int PER, int ROWS>
__global__ void __launch_bounds__(256)
layer_norm_rows_kernel(const float* __restrict__ x, const float* __restrict__ res, size_t res_rows, size_t rows,
                        const float* __restrict__ scale, const float* __restrict__ bias, float eps,
                        float* __restrict__ y, float2* __restrict__ part) {
    constexpr int cols = 8 * PER, C4 = cols / 4, STRIDE = cols + 8;
    constexpr int PL = ROWS * C4 / 256;  // float4 per lane for ROWS rows
    static_assert(PL * 256 == ROWS * C4, "the rows split evenly over the block");
    __shared__ __attribute__((aligned(16))) float tile[ROWS * STRIDE];
    __shared__ float stat[2][ROWS];  // mean, sd per row
    const int t = threadIdx.x;
    const size_t row0 = (size_t)blockIdx.x * ROWS;
    const int nr = (int)(rows - row0 < ROWS ? rows - row0 : ROWS);
    const float4* x4 = reinterpret_cast<const float4*>(x + row0 * cols);
    const float4* r4 = res ? reinterpret_cast<const float4*>(res) : nullptr;
    {
        float4 v[PL], w[PL];
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const int q = t + u * 256;
            if (q < nr * C4) v[u] = x4[q];
        }
        if (r4) {
#pragma unroll
            for (int u = 0; u < PL; ++u) {
                const int q = t + u * 256;
                if (q < nr * C4)
                    w[u] = r4[res_rows ? ((row0 + q / C4) % res_rows) * C4 + q % C4 : row0 * C4 + q];
            }
        }
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const int q = t + u * 256;
            if (q < nr * C4) {
                float4 a = v[u];
                if (r4)
                    a = make_float4(__fadd_rn(a.x, w[u].x), __fadd_rn(a.y, w[u].y), __fadd_rn(a.z, w[u].z),
                                    __fadd_rn(a.w, w[u].w));
                *reinterpret_cast<float4*>(&tile[(q / C4) * STRIDE + (q % C4) * 4]) = a;
            }
        }
    }
    __syncthreads();
    if (t < 8 * ROWS) {
        const int r = t >> 3, j = t & 7;
        if (r < nr) {  // whole 8-lane groups
            // both passes read the row from LDS (a register copy of the lane's PER values
            // would cost PER VGPRs in every wave of the block, and with them occupancy)
            const float* tr = tile + r * STRIDE + j;
            float p = 0.0f;
#pragma unroll 16
            for (int k = 0; k < PER; ++k) p = __fadd_rn(p, tr[8 * k]);
            const float mean = __fdiv_rn(combine8(p), (float)cols);
            p = 0.0f;
#pragma unroll 16
            for (int k = 0; k < PER; ++k) {
                const float c = __fsub_rn(tr[8 * k], mean);
                p = __fadd_rn(p, __fmul_rn(c, c));
            }
            const float var = __fdiv_rn(combine8(p), (float)cols);
            if (j == 0) {
                stat[0][r] = mean;
                stat[1][r] = sqrtf(__fadd_rn(var, eps));
            }
        }
    }
    __syncthreads();
    float4* y4 = reinterpret_cast<float4*>(y + row0 * cols);
    const float4* s4 = reinterpret_cast<const float4*>(scale);
    const float4* b4 = reinterpret_cast<const float4*>(bias);
    float mn = 0.0f, mx = 0.0f;  // DQL range of y (when `part` is given)
#pragma unroll
    for (int u = 0; u < PL; ++u) {
        const int q = t + u * 256;
        if (q < nr * C4) {
            const int r = q / C4, c4 = q % C4;
            const float mean = stat[0][r], sd = stat[1][r];
            const float4 a = *reinterpret_cast<const float4*>(&tile[r * STRIDE + c4 * 4]);
            const float4 sc = s4 ? s4[c4] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            const float4 bi = b4 ? b4[c4] : make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
            float4 o;
            o.x = __fadd_rn(__fmul_rn(__fdiv_rn(__fsub_rn(a.x, mean), sd), sc.x), bi.x);
            o.y = __fadd_rn(__fmul_rn(__fdiv_rn(__fsub_rn(a.y, mean), sd), sc.y), bi.y);
            o.z = __fadd_rn(__fmul_rn(__fdiv_rn(__fsub_rn(a.z, mean), sd), sc.z), bi.z);
            o.w = __fadd_rn(__fmul_rn(__fdiv_rn(__fsub_rn(a.w, mean), sd), sc.w), bi.w);
            icx::store_nt(&y4[q], o);
            if (part) {
                icx::range_acc(o.x, mn, mx);
                icx::range_acc(o.y, mn, mx);
                icx::range_acc(o.z, mn, mx);
                icx::range_acc(o.w, mn, mx);
            }
        }
    }
    if (part) icx::block_range_store<256>(mn, mx, part);
}

__global__ void __launch_bounds__(kThreads)
softmax_kernel(const float* __restrict__ x, size_t rows, size_t cols, float* __restrict__ y) {
    const int lane = threadIdx.x & 63, j = lane & 7;
    const size_t row = (size_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (row >= rows) return;
    const float* xr = x + row * cols;
    float* yr = y + row * cols;
    float m = -INFINITY;
    for (size_t i = j; i < cols; i += 8) m = fmaxf(m, xr[i]);  // NaN-ignoring, as f32::max
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 8));
    const size_t n8 = cols / 8 * 8;
    float p = 0.0f;
    for (size_t i = j; i < n8; i += 8) {
        const float e = expf(__fsub_rn(xr[i], m));
        yr[i] = e;
        p = __fadd_rn(p, e);
    }
    float acc = combine8(p);
    for (size_t i = n8; i < cols; ++i) {
        const float e = expf(__fsub_rn(xr[i], m));
        if (j == 0) yr[i] = e;
        acc = __fadd_rn(acc, e);
    }
    // each lane reads back only the values it wrote itself (the tail belongs to lane 0)
    for (size_t i = j; i < n8; i += 8) yr[i] = __fdiv_rn(yr[i], acc);
    if (j == 0)
        for (size_t i = n8; i < cols; ++i) yr[i] = __fdiv_rn(yr[i], acc);
}

// ---- ReduceMean, Pow, Sqrt: the ops of a LayerNorm exported node by node ----------------
// ReduceMean over the last axis (or over every element, as one row): ndarray 0.16's
// mean_axis over a contiguous lane — unrolled_fold's eight partial sums, combined as
// combine8 does, then the < 8 leftover elements in order — divided by the lane length
// converted to f32 (src/operators/reduce_mean.rs:64-72).  Eight lanes per row, 32 rows per
// block.
__global__ void __launch_bounds__(kThreads)
reduce_mean_last_kernel(const float* __restrict__ x, size_t rows, size_t cols, float* __restrict__ y) {
    const int j = threadIdx.x & 7;
    const size_t row = (size_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (row >= rows) return;  // a whole 8-lane group leaves together
    const float* xr = x + row * cols;
    const size_t n8 = cols / 8 * 8;
    float p = 0.0f;
    for (size_t i = j; i < n8; i += 8) p = __fadd_rn(p, xr[i]);
    float acc = combine8(p);
    if (j) return;
    for (size_t i = n8; i < cols; ++i) acc = __fadd_rn(acc, xr[i]);
    y[row] = __fdiv_rn(acc, (float)cols);
}

// ReduceMean over an axis that is not the last: ndarray's sum_axis adds the sub-views along
// the axis one after the other into a zero array (res = 0 + x[.., 0, ..] + x[.., 1, ..] + ...),
// then mean_axis divides by the axis length.  One thread per output of [outer, inner].
__global__ void __launch_bounds__(kThreads)
reduce_mean_seq_kernel(const float* __restrict__ x, size_t outer, size_t axis_len, size_t inner,
                       float* __restrict__ y) {
    const size_t n = outer * inner, stride = (size_t)gridDim.x * kThreads;
    const float fa = (float)axis_len;
    for (size_t o = (size_t)blockIdx.x * kThreads + threadIdx.x; o < n; o += stride) {
        const float* p = x + (o / inner) * axis_len * inner + o % inner;
        float acc = 0.0f;
        for (size_t a = 0; a < axis_len; ++a) acc = __fadd_rn(acc, p[a * inner]);
        y[o] = __fdiv_rn(acc, fa);
    }
}

// Pow (src/operators/pow.rs:18-45): y = x ^ e, the exponent broadcast over x [rows, cols].
// An exponent of exactly 2 gives the correctly rounded square x * x — LayerNormalization's
// c * c — and any other exponent the device powf.
__global__ void __launch_bounds__(kThreads)
pow_kernel(const float* __restrict__ x, size_t rows, size_t cols, const float* __restrict__ e,
           int e_kind, float* __restrict__ y) {
    const size_t n = rows * cols, stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const float v = x[i];
        const float p = icx::load_bcast(e, e_kind, i / cols, i % cols, cols);
        y[i] = p == 2.0f ? __fmul_rn(v, v) : powf(v, p);
    }
}

// Sqrt (src/operators/sqrt.rs:18-30): the correctly rounded square root (f32::sqrt).
__global__ void __launch_bounds__(kThreads)
sqrt_kernel(const float* __restrict__ x, size_t n, float* __restrict__ y) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = sqrtf(x[i]);
}

// ---- transpose ---------------------------------------------------------------------------
struct TransposeArgs {
    int rank;
    int64_t out_dims[6];
    int64_t in_stride_of_out[6];  // input stride of output axis d
};

template <typename T>
__global__ void __launch_bounds__(kThreads)
transpose_kernel(const T* __restrict__ x, size_t n, TransposeArgs a, T* __restrict__ y) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t o = (size_t)blockIdx.x * kThreads + threadIdx.x; o < n; o += stride) {
        size_t rem = o, src = 0;
        for (int d = a.rank - 1; d >= 0; --d) {
            const size_t idx = rem % (size_t)a.out_dims[d];
            rem /= (size_t)a.out_dims[d];
            src += idx * (size_t)a.in_stride_of_out[d];
        }
        y[o] = x[src];
    }
}

// ---- batched f32 matmul: 64x64 tiles, 4x4 outputs per thread, K step 16 -----------------
__global__ void __launch_bounds__(kThreads)
matmul_f32_kernel(const float* __restrict__ A, const float* __restrict__ B, int M, int K, int N,
                  int b_broadcast, int tiles_n, float* __restrict__ C) {
    __shared__ float sa[16][64 + 4];
    __shared__ float sb[16][64 + 4];
    const int batch = blockIdx.y;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const float* a = A + (size_t)batch * M * K;
    const float* b = B + (b_broadcast ? 0 : (size_t)batch * K * N);
    float* c = C + (size_t)batch * M * N;
    const int t = threadIdx.x, tr = t / 16, tc = t % 16;
    const int m0 = tm * 64, n0 = tn * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 16) {
        for (int i = t; i < 16 * 64; i += kThreads) {
            const int kk = i % 16, mm = i / 16;  // A tile stored k-major
            const int gm = m0 + mm, gk = k0 + kk;
            sa[kk][mm] = (gm < M && gk < K) ? a[(size_t)gm * K + gk] : 0.0f;
            const int nn = i % 64, kb = i / 64;
            const int gn = n0 + nn, gk2 = k0 + kb;
            sb[kb][nn] = (gn < N && gk2 < K) ? b[(size_t)gk2 * N + gn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                av[u] = sa[kk][tr * 4 + u];
                bv[u] = sb[kk][tc * 4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] = fmaf(av[u], bv[v], acc[u][v]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int gm = m0 + tr * 4 + u;
        if (gm >= M) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int gn = n0 + tc * 4 + v;
            if (gn < N) c[(size_t)gm * N + gn] = acc[u][v];
        }
    }
}

// ---- fused self-attention, S <= 128, D == 64 --------------------------------------------
// One block per (batch, head, half of the queries): 4 waves of 16 queries each, so the
// 2 * B * H blocks give every CU three blocks (12 waves, three per SIMD) at the DistilBERT
// shape.  K and then V pass through one 35 KB LDS region: K for S^T, V (transposed) for P V,
// both held in registers from the start so the V load overlaps S^T.
//   S^T = K Q^T (*|/) scale (or Q scaled first): 8 key tiles of 16 x 16, contraction 64
//   P = softmax over the keys, in registers
//   ctx = P V: 4 tiles of 16 x 16, contraction S
// v_mfma_f32_16x16x4f32: A lane l = A[l % 16][l / 16], B lane l = B[l / 16][l % 16],
// D register r of lane l = D[4 (l / 16) + r][l % 16].
// Step s of the S^T contraction gives lane-group g = l / 16 dimension 16 g + s, so each lane
// reads its K row and Q row as 16 contiguous floats.  S^T leaves lane l with query l % 16
// and, in register r of key tile t, key 16 t + 4 (l / 16) + r — exactly P's A-operand layout
// for the P V step (t, r), whose 4-key contraction takes key 16 t + 4 g + r from group g, so P
// never leaves registers; the B operands of steps r = 0..3 are four consecutive keys of V^T.
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int ATT_S = 128, ATT_D = 64, ATT_QB = 64;  // keys, head size, queries per block
constexpr int ATT_MAX_S = icx::kAttentionMaxSeq;  // longest sequence (attention_long_kernel)
constexpr int K_STRIDE = ATT_D + 4;   // floats per LDS row of K: 16-byte reads conflict-free
constexpr int VT_STRIDE = ATT_S + 4;  // V^T rows [dim][key]
// Key k of V^T row d is stored at column k ^ vt_swz(d).  With the 132-float rows alone, the
// transposing stores (a wave writes 16 dims x 4 keys of one component per instruction) hit
// only 16 of the 64 banks; the XOR of bits 2-3 of the key by bits 4-5 of the dim spreads them
// over all 64, keeps every 4-key group contiguous and 16-byte aligned for the P V reads, and
// leaves those reads (16 dims of one 4-key group per 16 lanes) conflict-free as well.
__device__ __forceinline__ int vt_swz(int d) { return 4 * ((d >> 4) & 3); }
constexpr int ATT_LDS_FLOATS = ATT_S * K_STRIDE > ATT_D * VT_STRIDE ? ATT_S * K_STRIDE : ATT_D * VT_STRIDE;

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int S, H;
    int64_t ldq, ldk, ldv, ldo;  // row strides (elements) of the [B*S, *] activations
    float scale;
    int scale_div;  // 1: x / scale, 0: x * scale
    int scale_q;    // 1: applied to Q before the product, 0: to the scores
    float2* part;   // DQL range partials of out, one per block, or null
    float recip;      // 1 / scale when that is exact (a power of two), so x / scale == x * recip
    int recip_exact;  // bit for bit, and the division becomes a multiplication
    int qsplit;       // blocks per (batch, head): 2 when S > 64 (64 queries each), else 1
    // quantized output (attention_kernel<true>): the DynamicQuantizeLinear of out, written as
    // u8 (row stride ldo), scale and zero point, through qexchange.hpp's range exchange
    uint8_t* qy;
    float* q_scale;
    uint8_t* q_zp;
    unsigned* q_sync;
    unsigned long long q_wait;  // exchange wait limit, wall-clock ticks
    unsigned q_poison;          // test hook: a tag no block publishes
    // padding mask (an export's Where(mask, fill, scores) before the Softmax): key j of batch
    // b is masked when mask[b * mask_bs + j] != 0, its score then replaced by `fill`; null: none
    const uint8_t* mask;
    int64_t mask_bs;
    float fill;
};

__device__ __forceinline__ float apply_scale(float x, const AttnArgs& a) {
    if (!a.scale_div) return __fmul_rn(x, a.scale);
    return a.recip_exact ? __fmul_rn(x, a.recip) : __fdiv_rn(x, a.scale);
}

__device__ __forceinline__ float f4c(const float4& v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

// QOUT: the context is not stored; the blocks (all resident: the host launches no more than
// fit) trade their (min, max) through the range exchange (qexchange.hpp) and each writes its
// part of the DynamicQuantizeLinear of the context — y, scale and zero point bit-identical to that op
// applied to the f32 context (the same fold, parameters and per-element rounding,
// dql_core.hpp).
template <bool QOUT>
__global__ void __launch_bounds__(kThreads) attention_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[ATT_LDS_FLOATS];
    __shared__ uint8_t kmask[ATT_S];
    unsigned tag0 = 0;  // the exchange's tag, read early to hide its latency
    if (QOUT && threadIdx.x == 0) tag0 = icx::qx::read_tag(a.q_sync);
    // The two halves of a (batch, head) are blocks g and g + 8 of a group of 16, which the
    // hardware places on the same XCD (block i runs on XCD i % 8), so the second half's K and
    // V loads hit that XCD's L2.
    int pair = blockIdx.x, half = 0;
    if (a.qsplit == 2) {
        const int grp = blockIdx.x >> 4, in = blockIdx.x & 15;
        pair = grp * 8 + (in & 7);
        half = in >> 3;
        if ((int)gridDim.x & 15) {  // a partial last group: plain pairing
            pair = blockIdx.x >> 1;
            half = blockIdx.x & 1;
        }
    }
    const int b = pair / a.H, h = pair % a.H;
    const int S = a.S;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int qi = half * ATT_QB + 16 * w + lq;  // this lane's query row

    // the padding mask's byte for key t first: its load is then not the last one to land
    const uint8_t mk = a.mask && t < S ? a.mask[(int64_t)b * a.mask_bs + t] : (uint8_t)0;
    // every load in flight at once: K and V of (b, h) (rows past S are zero), and this lane's
    // Q row segment, dims [16 lg, 16 lg + 16)
    float4 kr[8], vr[8], qr[4];
    const int c4 = (t & 15) * 4;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int r = u * 16 + (t >> 4);
        kr[u] = vr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < S) {
            const size_t row = (size_t)b * S + r;
            kr[u] = *reinterpret_cast<const float4*>(a.k + row * a.ldk + h * ATT_D + c4);
            vr[u] = *reinterpret_cast<const float4*>(a.v + row * a.ldv + h * ATT_D + c4);
        }
    }
    const float* qp = a.q + ((size_t)b * S + qi) * a.ldq + h * ATT_D + 16 * lg;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        qr[u] = qi < S ? *reinterpret_cast<const float4*>(qp + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 8; ++u)
        *reinterpret_cast<float4*>(lds + (u * 16 + (t >> 4)) * K_STRIDE + c4) = kr[u];
    if (a.mask && t < S) kmask[t] = mk;  // read after the barrier below
    if (a.scale_q) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            qr[u].x = apply_scale(qr[u].x, a);
            qr[u].y = apply_scale(qr[u].y, a);
            qr[u].z = apply_scale(qr[u].z, a);
            qr[u].w = apply_scale(qr[u].w, a);
        }
    }
    __syncthreads();

    // S^T: A = K (lane = key), B = Q^T (lane = query); K fragments of tile kt+1 are read
    // during the MFMAs of tile kt, and tile kt-1's scores are scaled, masked and folded into
    // the row max then (VALU work under the MFMAs)
    v4f st[8];
    float4 kf[2][4];
    auto read_k = [&](int kt, float4 (&f)[4]) {
        const float* kp = lds + (16 * kt + lq) * K_STRIDE + 16 * lg;
#pragma unroll
        for (int u = 0; u < 4; ++u) f[u] = *reinterpret_cast<const float4*>(kp + 4 * u);
    };
    float m = -INFINITY;
    auto scale_mask_max = [&](int kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * kt + 4 * lg + r;
            float x = a.scale_q ? st[kt][r] : apply_scale(st[kt][r], a);
            if (key >= S) x = -INFINITY;
            else if (a.mask && kmask[key]) x = a.fill;  // masked_fill after the scale, as exported
            st[kt][r] = x;
            m = fmaxf(m, x);
        }
    };
    read_k(0, kf[0]);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        if (kt + 1 < 8) read_k(kt + 1, kf[(kt + 1) & 1]);
        st[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4c(kf[kt & 1][u], e), f4c(qr[u], e), st[kt], 0, 0, 0);
        if (kt > 0) scale_mask_max(kt - 1);
    }
    scale_mask_max(7);
    __syncthreads();  // every wave is done with K: the region takes V^T
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int r = (u * 16 + (t >> 4)) ^ vt_swz(c4);  // c4 .. c4 + 3 share bits 4-5
        lds[(c4 + 0) * VT_STRIDE + r] = vr[u].x;
        lds[(c4 + 1) * VT_STRIDE + r] = vr[u].y;
        lds[(c4 + 2) * VT_STRIDE + r] = vr[u].z;
        lds[(c4 + 3) * VT_STRIDE + r] = vr[u].w;
    }

    // softmax of row qi over its S keys: 32 in this lane, the rest in lanes l ^ 16, l ^ 32.
    // The row max is complete; the exponentials of key tile kt + 1 are computed during the
    // P V MFMAs of tile kt, and the context is divided by the row sum once at the end
    // (ctx = (sum_k e_k v_k) / sum_k e_k): the hardware exp2 and one reciprocal per row, within
    // a few ulp of expf and of e / sum, far inside the attention's tolerance.
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.0f;
    auto expo = [&](int kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __expf(__fsub_rn(st[kt][r], m));
            st[kt][r] = e;
            sum = __fadd_rn(sum, e);
        }
    };
    expo(0);
    __syncthreads();  // V^T written

    // ctx = P V: A = P from the S^T registers, B = V^T rows of dims 16 dt + lq
    v4f o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        float4 vq[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            vq[dt] = *reinterpret_cast<const float4*>(lds + (16 * dt + lq) * VT_STRIDE +
                                                      ((16 * kt + 4 * lg) ^ vt_swz(16 * dt + lq)));
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[kt][r], f4c(vq[dt], r), o[dt], 0, 0, 0);
        if (kt + 1 < 8) expo(kt + 1);
    }
    sum = __fadd_rn(sum, __shfl_xor(sum, 16, 64));
    sum = __fadd_rn(sum, __shfl_xor(sum, 32, 64));
    // lane l's context rows are queries 4 lg + r (of its 16): their sums sit in lanes 4 lg + r
    const float inv = __fdiv_rn(1.0f, sum);
    float inv_r[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv_r[r] = __shfl(inv, 4 * lg + r, 64);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[dt][r] = __fmul_rn(o[dt][r], inv_r[r]);
    // lane l holds ctx rows (queries) 16 w + 4 lg + r, dims 16 dt + lq
    if constexpr (QOUT) {
        __shared__ unsigned s_tag;
        float qmn = 0.0f, qmx = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (half * ATT_QB + 16 * w + 4 * lg + r >= S) continue;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) icx::range_acc(o[dt][r], qmn, qmx);
        }
        if (t == 0) s_tag = tag0;
        icx::dql::block_minmax<kThreads>(qmn, qmx);  // its barrier also publishes s_tag
        const unsigned tag = s_tag;
        if (t == 0) icx::qx::publish(a.q_sync, tag, qmn, qmx);
        bool ok;
        const icx::dql::DqlParams p = icx::qx::gather<kThreads>(a.q_sync, tag, tag ^ a.q_poison, a.q_wait, ok);
        // the block's 64 x 64 bytes go through LDS (free: every wave is past the gather's
        // barrier), then out as 16-byte row segments, four lanes per row
        uint8_t* qt = reinterpret_cast<uint8_t*>(lds);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t b4 = ok ? icx::dql::quant4(make_float4(o[0][r], o[1][r], o[2][r], o[3][r]), p) : 0u;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) qt[(16 * w + 4 * lg + r) * ATT_D + 16 * dt + lq] = (uint8_t)(b4 >> (8 * dt));
        }
        __syncthreads();
        const int qrow = half * ATT_QB + (t >> 2);
        if (qrow < S)
            *reinterpret_cast<uint4*>(a.qy + ((size_t)b * S + qrow) * a.ldo + h * ATT_D + 16 * (t & 3)) =
                *reinterpret_cast<const uint4*>(qt + (t >> 2) * ATT_D + 16 * (t & 3));
        if (t == 0) icx::qx::finish(a.q_sync, ok, p, a.q_scale, a.q_zp);
        return;
    }
    float mn = 0.0f, mx = 0.0f;  // DQL range of out (when a.part is given)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = half * ATT_QB + 16 * w + 4 * lg + r;
        if (row >= S) continue;
        float* dst = a.out + ((size_t)b * S + row) * a.ldo + h * ATT_D + lq;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            dst[16 * dt] = o[dt][r];
            if (a.part) icx::range_acc(o[dt][r], mn, mx);
        }
    }
    if (a.part) icx::block_range_store<kThreads>(mn, mx, a.part);
}

// Sequences longer than the 128 keys attention_kernel keeps in one LDS tile (BERT at 384 or
// 512, say): a block takes 64 queries of one (batch, head) and walks the keys in chunks of
// 128 with the running (online) softmax — per chunk the S^T tile, scale and mask exactly as
// attention_kernel forms them, the new row max m' = max(m, chunk max), the earlier partial
// sums and context rescaled by exp(m - m'), then P V of the chunk — and divides by the row sum
// once at the end.  The same MFMA layouts as attention_kernel (P stays in registers).  A row
// whose every score is -inf gives 0 / 0 = NaN, as the Softmax node does.  f32 context only.
// The blocks of one (batch, head) run on the same XCD (block i runs on XCD i % 8), so their
// K / V chunk loads hit that XCD's L2.
__global__ void __launch_bounds__(kThreads) attention_long_kernel(AttnArgs a, int nqt) {
    __shared__ __attribute__((aligned(16))) float lds[ATT_LDS_FLOATS];
    __shared__ uint8_t kmask[ATT_S];
    const int P = (int)(gridDim.x / (unsigned)nqt);  // (batch, head) pairs
    const int full = P / 8;
    int pair, qt;
    if ((int)blockIdx.x < full * 8 * nqt) {
        const int g = blockIdx.x / (8 * nqt), rem = blockIdx.x % (8 * nqt);
        qt = rem / 8;
        pair = g * 8 + rem % 8;
    } else {
        const int x = blockIdx.x - full * 8 * nqt;
        pair = full * 8 + x / nqt;
        qt = x % nqt;
    }
    const int b = pair / a.H, h = pair % a.H;
    const int S = a.S;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int qi = qt * ATT_QB + 16 * w + lq;  // this lane's query row
    const int c4 = (t & 15) * 4;

    float4 qr[4];
    const float* qp = a.q + ((size_t)b * S + qi) * a.ldq + h * ATT_D + 16 * lg;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        qr[u] = qi < S ? *reinterpret_cast<const float4*>(qp + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.scale_q) {
            qr[u].x = apply_scale(qr[u].x, a);
            qr[u].y = apply_scale(qr[u].y, a);
            qr[u].z = apply_scale(qr[u].z, a);
            qr[u].w = apply_scale(qr[u].w, a);
        }
    }
    float m = -INFINITY, sum = 0.0f;
    v4f o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = v4f{0.f, 0.f, 0.f, 0.f};
    v4f st[8];

    for (int key0 = 0; key0 < S; key0 += ATT_S) {
        // the chunk's mask bytes, K and V rows (rows past S are zero)
        const uint8_t mk = a.mask && t < ATT_S && key0 + t < S ? a.mask[(int64_t)b * a.mask_bs + key0 + t] : (uint8_t)0;
        float4 kr[8], vr[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int r = key0 + u * 16 + (t >> 4);
            kr[u] = vr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < S) {
                const size_t row = (size_t)b * S + r;
                kr[u] = *reinterpret_cast<const float4*>(a.k + row * a.ldk + h * ATT_D + c4);
                vr[u] = *reinterpret_cast<const float4*>(a.v + row * a.ldv + h * ATT_D + c4);
            }
        }
        __syncthreads();  // the previous chunk's P V reads of LDS are done
#pragma unroll
        for (int u = 0; u < 8; ++u)
            *reinterpret_cast<float4*>(lds + (u * 16 + (t >> 4)) * K_STRIDE + c4) = kr[u];
        if (t < ATT_S) kmask[t] = mk;
        __syncthreads();
        float mc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            float4 kf[4];
            const float* kp = lds + (16 * kt + lq) * K_STRIDE + 16 * lg;
#pragma unroll
            for (int u = 0; u < 4; ++u) kf[u] = *reinterpret_cast<const float4*>(kp + 4 * u);
            st[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4c(kf[u], e), f4c(qr[u], e), st[kt], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kc = 16 * kt + 4 * lg + r;
                float x = a.scale_q ? st[kt][r] : apply_scale(st[kt][r], a);
                if (key0 + kc >= S) x = -INFINITY;
                else if (a.mask && kmask[kc]) x = a.fill;
                st[kt][r] = x;
                mc = fmaxf(mc, x);
            }
        }
        mc = fmaxf(mc, __shfl_xor(mc, 16, 64));
        mc = fmaxf(mc, __shfl_xor(mc, 32, 64));
        const float mn = fmaxf(m, mc);
        const float mu = mn == -INFINITY ? 0.0f : mn;  // every score so far -inf: weights 0
        const float alpha = __expf(__fsub_rn(m, mu));
        m = mn;
        sum = __fmul_rn(sum, alpha);
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __expf(__fsub_rn(st[kt][r], mu));
                st[kt][r] = e;
                sum = __fadd_rn(sum, e);
            }
        // context rows are queries 4 lg + r: their factors sit in lanes 4 lg + r
        float alpha_r[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) alpha_r[r] = __shfl(alpha, 4 * lg + r, 64);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[dt][r] = __fmul_rn(o[dt][r], alpha_r[r]);
        __syncthreads();  // every wave is done with K: the region takes V^T
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int r = (u * 16 + (t >> 4)) ^ vt_swz(c4);
            lds[(c4 + 0) * VT_STRIDE + r] = vr[u].x;
            lds[(c4 + 1) * VT_STRIDE + r] = vr[u].y;
            lds[(c4 + 2) * VT_STRIDE + r] = vr[u].z;
            lds[(c4 + 3) * VT_STRIDE + r] = vr[u].w;
        }
        __syncthreads();
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            float4 vq[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
                vq[dt] = *reinterpret_cast<const float4*>(lds + (16 * dt + lq) * VT_STRIDE +
                                                          ((16 * kt + 4 * lg) ^ vt_swz(16 * dt + lq)));
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[kt][r], f4c(vq[dt], r), o[dt], 0, 0, 0);
        }
    }
    sum = __fadd_rn(sum, __shfl_xor(sum, 16, 64));
    sum = __fadd_rn(sum, __shfl_xor(sum, 32, 64));
    const float inv = __fdiv_rn(1.0f, sum);
    float inv_r[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv_r[r] = __shfl(inv, 4 * lg + r, 64);
    float mn = 0.0f, mx = 0.0f;  // DQL range of out (when a.part is given)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = qt * ATT_QB + 16 * w + 4 * lg + r;
        if (row >= S) continue;
        float* dst = a.out + ((size_t)b * S + row) * a.ldo + h * ATT_D + lq;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const float y = __fmul_rn(o[dt][r], inv_r[r]);
            dst[16 * dt] = y;
            if (a.part) icx::range_acc(y, mn, mx);
        }
    }
    if (a.part) icx::block_range_store<kThreads>(mn, mx, a.part);
}


template <int PER>
void launch_ln_rows(bool rows4, dim3 grid, hipStream_t s, const float* x, const float* res, size_t res_rows,
                    size_t rows, const float* scale, const float* bias, float eps, float* y, float2* part) {
    if (rows4)
        hipLaunchKernelGGL((layer_norm_rows_kernel<PER, 4>), grid, dim3(256), 0, s, x, res, res_rows, rows, scale,
                           bias, eps, y, part);
    else
        hipLaunchKernelGGL((layer_norm_rows_kernel<PER, 8>), grid, dim3(256), 0, s, x, res, res_rows, rows, scale,
                           bias, eps, y, part);
}

unsigned grid_for(size_t work, size_t per_block, unsigned cap) {
    size_t b = icx::cdiv(work, per_block);
    if (b < 1) b = 1;
    return (unsigned)(b > cap ? cap : b);
}

}  // namespace

int icx::layer_norm_f32(hipStream_t s, const float* x, const float* residual, size_t res_rows, size_t rows,
                        size_t cols, const float* scale, const float* bias, float eps, float* y, float2* part,
                        int* n_part) {
    if (n_part) *n_part = 0;
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "LayerNormalization: null pointer argument");
    if (cols == 0 && rows) ICX_FAIL(ICX_ERR_SHAPE, "LayerNormalization: empty normalized axis");
    if (rows == 0) return ICX_OK;
    if (res_rows && (!residual || rows % res_rows))
        ICX_FAIL(ICX_ERR_SHAPE, "LayerNormalization: %zu rows over a residual of %zu rows", rows, res_rows);
    // partials only from the LDS-staged kernel, one per block: blocks of 4 rows while their
    // partials fit, else of 8
    const bool rows4 = icx::cdiv(rows, 4) <= (size_t)icx::kMaxRangeParts;
    const dim3 g8((unsigned)icx::cdiv(rows, rows4 ? 4 : 8));
    float2* pp = (part && g8.x <= (unsigned)icx::kMaxRangeParts) ? part : nullptr;
    // the hidden sizes of the BERT family, float4-aligned: rows staged through LDS
    const bool a16 = icx::aligned16(x) && icx::aligned16(y) && icx::aligned16(scale) &&
                     icx::aligned16(bias) && (!residual || icx::aligned16(residual));
    switch (a16 ? cols : 0) {
        case 512: launch_ln_rows<64>(rows4, g8, s, x, residual, res_rows, rows, scale, bias, eps, y, pp); break;
        case 768: launch_ln_rows<96>(rows4, g8, s, x, residual, res_rows, rows, scale, bias, eps, y, pp); break;
        case 1024: launch_ln_rows<128>(rows4, g8, s, x, residual, res_rows, rows, scale, bias, eps, y, pp); break;
        default:
            pp = nullptr;
            hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)icx::cdiv(rows, 32)), dim3(kThreads), 0, s, x,
                               residual, res_rows, rows, cols, scale, bias, eps, y);
    }
    ICX_LAUNCH_CHECK("layer_norm_kernel");
    if (pp && n_part) *n_part = (int)g8.x;
    return ICX_OK;
}

extern "C" int icx_layer_norm_f32(icx_stream_t stream, const float* x, const float* residual,
                                  size_t rows, size_t cols, const float* scale,
                                  const float* bias, float eps, float* y) {
    icx::clear_error();
    return icx::layer_norm_f32(reinterpret_cast<hipStream_t>(stream), x, residual, 0, rows, cols, scale, bias,
                               eps, y, nullptr, nullptr);
}

extern "C" int icx_softmax_f32(icx_stream_t stream, const float* x, size_t rows, size_t cols,
                               float* y) {
    icx::clear_error();
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Softmax: null pointer argument");
    if (x == y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Softmax: input and output must not alias");
    if (rows == 0 || cols == 0) return ICX_OK;
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)icx::cdiv(rows, 32)), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, rows, cols, y);
    ICX_LAUNCH_CHECK("softmax_kernel");
    return ICX_OK;
}

extern "C" int icx_reduce_mean_f32(icx_stream_t stream, const float* x, size_t outer, size_t axis_len,
                                   size_t inner, int sequential, float* y) {
    icx::clear_error();
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "ReduceMean: null pointer argument");
    if (x == y) ICX_FAIL(ICX_ERR_INVALID_ARG, "ReduceMean: input and output must not alias");
    if (outer == 0 || inner == 0) return ICX_OK;
    if (axis_len == 0) ICX_FAIL(ICX_ERR_SHAPE, "ReduceMean: the reduced axis is empty (the mean is undefined)");
    if (!sequential && inner != 1)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "ReduceMean: the unrolled order needs a contiguous axis (inner == 1)");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (!sequential) {
        if (icx::cdiv(outer, 32) > 0x7fffffffu) ICX_FAIL(ICX_ERR_SHAPE, "ReduceMean: too many rows");
        hipLaunchKernelGGL(reduce_mean_last_kernel, dim3((unsigned)icx::cdiv(outer, 32)), dim3(kThreads), 0, s,
                           x, outer, axis_len, y);
        ICX_LAUNCH_CHECK("reduce_mean_last_kernel");
    } else {
        hipLaunchKernelGGL(reduce_mean_seq_kernel, dim3(grid_for(outer * inner, kThreads, 65536)), dim3(kThreads),
                           0, s, x, outer, axis_len, inner, y);
        ICX_LAUNCH_CHECK("reduce_mean_seq_kernel");
    }
    return ICX_OK;
}

extern "C" int icx_pow_f32(icx_stream_t stream, const float* x, size_t rows, size_t cols, const float* e,
                           int e_kind, float* y) {
    icx::clear_error();
    if (!x || !e || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Pow: null pointer argument");
    if (e_kind < ICX_BCAST_SCALAR || e_kind > ICX_BCAST_FULL)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "Pow: unknown exponent broadcast kind %d", e_kind);
    if (rows == 0 || cols == 0) return ICX_OK;
    hipLaunchKernelGGL(pow_kernel, dim3(grid_for(rows * cols, kThreads, 65536)), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, rows, cols, e, e_kind, y);
    ICX_LAUNCH_CHECK("pow_kernel");
    return ICX_OK;
}

extern "C" int icx_sqrt_f32(icx_stream_t stream, const float* x, size_t n, float* y) {
    icx::clear_error();
    if (!x || !y) ICX_FAIL(ICX_ERR_INVALID_ARG, "Sqrt: null pointer argument");
    if (n == 0) return ICX_OK;
    hipLaunchKernelGGL(sqrt_kernel, dim3(grid_for(n, kThreads, 65536)), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, n, y);
    ICX_LAUNCH_CHECK("sqrt_kernel");
    return ICX_OK;
}

extern "C" int icx_transpose(icx_stream_t stream, const void* x, size_t elem_bytes, int rank,
                             const int64_t* dims, const int* perm, void* y) {
    icx::clear_error();
    if (!x || !y || (rank && (!dims || !perm)))
        ICX_FAIL(ICX_ERR_INVALID_ARG, "Transpose: null pointer argument");
    if (rank < 0 || rank > 6) ICX_FAIL(ICX_ERR_UNSUPPORTED, "Transpose: rank %d outside [0, 6]", rank);
    if (elem_bytes != 1 && elem_bytes != 4)
        ICX_FAIL(ICX_ERR_DTYPE, "Transpose: element size %zu unsupported (1 or 4 bytes)", elem_bytes);
    TransposeArgs a{};
    a.rank = rank;
    int64_t in_stride[6];
    int64_t st = 1;
    size_t n = 1;
    bool seen[6] = {false, false, false, false, false, false};
    for (int d = rank - 1; d >= 0; --d) {
        if (dims[d] < 0) ICX_FAIL(ICX_ERR_SHAPE, "Transpose: negative dimension");
        in_stride[d] = st;
        st *= dims[d];
    }
    for (int d = 0; d < rank; ++d) {
        if (perm[d] < 0 || perm[d] >= rank || seen[perm[d]])
            ICX_FAIL(ICX_ERR_INVALID_ARG, "Transpose: perm is not a permutation of [0, %d)", rank);
        seen[perm[d]] = true;
        a.out_dims[d] = dims[perm[d]];
        a.in_stride_of_out[d] = in_stride[perm[d]];
        n *= (size_t)dims[perm[d]];
    }
    if (n == 0) return ICX_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(grid_for(n, kThreads * 4, 8192)), block(kThreads);
    if (elem_bytes == 4)
        hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, block, 0, s,
                           reinterpret_cast<const uint32_t*>(x), n, a, reinterpret_cast<uint32_t*>(y));
    else
        hipLaunchKernelGGL(transpose_kernel<uint8_t>, grid, block, 0, s,
                           reinterpret_cast<const uint8_t*>(x), n, a, reinterpret_cast<uint8_t*>(y));
    ICX_LAUNCH_CHECK("transpose_kernel");
    return ICX_OK;
}

extern "C" int icx_matmul_f32(icx_stream_t stream, const float* a, const float* b, size_t batch,
                              int b_broadcast, size_t M, size_t K, size_t N, float* c) {
    icx::clear_error();
    if (!a || !b || !c) ICX_FAIL(ICX_ERR_INVALID_ARG, "MatMul: null pointer argument");
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || batch > 65535)
        ICX_FAIL(ICX_ERR_SHAPE, "MatMul: dimensions out of range");
    if (batch == 0 || M == 0 || N == 0) return ICX_OK;
    const int tiles_n = (int)icx::cdiv(N, 64);
    const dim3 grid((unsigned)(icx::cdiv(M, 64) * tiles_n), (unsigned)batch);
    hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), a, b, (int)M, (int)K, (int)N,
                       b_broadcast ? 1 : 0, tiles_n, c);
    ICX_LAUNCH_CHECK("matmul_f32_kernel");
    return ICX_OK;
}

namespace {
// Shape checks and kernel arguments shared by the f32 and the quantized-output launches.
int attention_args(const float* q, const float* k, const float* v, size_t B, size_t S, size_t H, size_t D,
                   size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale, int scale_div, int scale_q,
                   const icx::AttnMask* mask, AttnArgs* a, size_t* blocks) {
    if (!q || !k || !v) ICX_FAIL(ICX_ERR_INVALID_ARG, "Attention: null pointer argument");
    if (D != (size_t)ATT_D || S == 0 || S > (size_t)ATT_MAX_S)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention: head size %zu / sequence %zu unsupported (D = 64, S <= %d)", D, S,
                 ATT_MAX_S);
    if (ldq < H * D || ldk < H * D || ldv < H * D || ldo < H * D || (ldq | ldk | ldv) % 4 ||
        !icx::aligned16(q) || !icx::aligned16(k) || !icx::aligned16(v))
        ICX_FAIL(ICX_ERR_SHAPE, "Attention: row strides must cover H*D and keep 16-byte alignment");
    // blocks per (batch, head): one per 64 queries (attention_kernel takes S <= 128 keys in
    // one tile: one or two blocks; attention_long_kernel walks longer ones in chunks)
    const size_t per = S > (size_t)ATT_S ? icx::cdiv(S, (size_t)ATT_QB) : (S > (size_t)ATT_QB ? 2 : 1);
    if (B * H * per > 0x3fffffff) ICX_FAIL(ICX_ERR_SHAPE, "Attention: too many (batch, head) pairs");
    *blocks = B * H * per;
    *a = AttnArgs{};
    a->q = q;
    a->k = k;
    a->v = v;
    a->S = (int)S;
    a->H = (int)H;
    a->ldq = (int64_t)ldq;
    a->ldk = (int64_t)ldk;
    a->ldv = (int64_t)ldv;
    a->ldo = (int64_t)ldo;
    a->scale = scale;
    a->scale_div = scale_div ? 1 : 0;
    a->scale_q = scale_q ? 1 : 0;
    a->qsplit = (int)per;
    if (mask && mask->keys) {
        a->mask = mask->keys;
        a->mask_bs = mask->batch_stride;
        a->fill = mask->fill;
    }
    // a power-of-two scale whose reciprocal is a normal float: x / scale == x * (1 / scale)
    int e = 0;
    const float m = std::frexp(scale, &e);
    const float r = 1.0f / scale;
    if (m == 0.5f && std::isnormal(scale) && std::isnormal(r)) {
        a->recip = r;
        a->recip_exact = 1;
    }
    return ICX_OK;
}
}  // namespace

int icx::attention_f32(hipStream_t s, const float* q, const float* k, const float* v, size_t B, size_t S,
                       size_t H, size_t D, size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale,
                       int scale_div, int scale_q, const AttnMask* mask, float* out, float2* part, int* n_part) {
    if (n_part) *n_part = 0;
    if (!out) ICX_FAIL(ICX_ERR_INVALID_ARG, "Attention: null pointer argument");
    AttnArgs a;
    size_t blocks;
    int rc = attention_args(q, k, v, B, S, H, D, ldq, ldk, ldv, ldo, scale, scale_div, scale_q, mask, &a, &blocks);
    if (rc) return rc;
    if (blocks == 0) return ICX_OK;
    a.out = out;
    float2* pp = (part && blocks <= (size_t)icx::kMaxRangeParts) ? part : nullptr;
    a.part = pp;
    if (S > (size_t)ATT_S) {
        hipLaunchKernelGGL(attention_long_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, a, a.qsplit);
        ICX_LAUNCH_CHECK("attention_long_kernel");
    } else {
        hipLaunchKernelGGL(attention_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
        ICX_LAUNCH_CHECK("attention_kernel");
    }
    if (pp && n_part) *n_part = (int)blocks;
    return ICX_OK;
}

int icx::attention_dql(hipStream_t s, const float* q, const float* k, const float* v, size_t B, size_t S,
                       size_t H, size_t D, size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale,
                       int scale_div, int scale_q, const AttnMask* mask, uint8_t* y, float* y_scale,
                       uint8_t* y_zp, unsigned* sync) {
    if (!y || !y_scale || !y_zp || !sync) ICX_FAIL(ICX_ERR_INVALID_ARG, "Attention+DQL: null pointer argument");
    if (S > (size_t)ATT_S) ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention+DQL: sequence %zu > %d", S, ATT_S);
    if (ldo % 16 || !icx::aligned16(y))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention+DQL: the u8 rows must keep 16-byte alignment");
    AttnArgs a;
    size_t blocks;
    int rc = attention_args(q, k, v, B, S, H, D, ldq, ldk, ldv, ldo, scale, scale_div, scale_q, mask, &a, &blocks);
    if (rc) return rc;
    if (blocks == 0 || blocks > (size_t)icx::kQoutMaxBlocks)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention+DQL: %zu blocks outside the exchange's 1..%d", blocks,
                 icx::kQoutMaxBlocks);
    // every block must be resident at once for the exchange: launch only what fits
    static int per_cu[64] = {0};
    int d = 0;
    ICX_HIP_CHECK(hipGetDevice(&d));
    if (d < 0 || d >= 64) ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention+DQL: device %d", d);
    if (!per_cu[d]) {
        int nb = 0;
        ICX_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, attention_kernel<true>, kThreads, 0));
        per_cu[d] = nb > 0 ? nb : -1;
    }
    if (per_cu[d] < 0 || blocks > (size_t)per_cu[d] * icx::num_cus())
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "Attention+DQL: %zu blocks exceed the %d resident ones", blocks,
                 per_cu[d] * icx::num_cus());
    a.qy = y;
    a.q_scale = y_scale;
    a.q_zp = y_zp;
    a.q_sync = sync;
    a.q_wait = icx::wall_ticks(icx::kExchangeWaitUs);
    if (const int f = icx::qout_fault_spin()) {  // test hook
        a.q_wait = icx::wall_ticks((unsigned)f);
        a.q_poison = 0x80000000u;
    }
    hipLaunchKernelGGL(attention_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
    ICX_LAUNCH_CHECK("attention_kernel");
    return ICX_OK;
}

extern "C" int icx_attention_f32(icx_stream_t stream, const float* q, const float* k,
                                 const float* v, size_t B, size_t S, size_t H, size_t D,
                                 size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale,
                                 int scale_div, int scale_q, float* out) {
    icx::clear_error();
    return icx::attention_f32(reinterpret_cast<hipStream_t>(stream), q, k, v, B, S, H, D, ldq, ldk, ldv, ldo,
                              scale, scale_div, scale_q, nullptr, out, nullptr, nullptr);
}
