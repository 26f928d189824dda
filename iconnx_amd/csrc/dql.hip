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
// A single-launch form (icx::dql_exchange, flat mode, no row sums; the graph executor's DQLs
// and icx_dynamic_quantize_linear_exchange): every block keeps 1, 2 or 4 float4 per lane of
// x in registers (up to 1024 resident blocks, 4 Mi elements), the blocks trade their
// (min, max) pairs through the range exchange of qexchange.hpp, and each block quantizes
// from its registers.  Kernel durations on MI355X: 9.1 us against 4.2 + 6.4 us for the two
// launches at 3.1 M elements, 8.3 against 3.3 + 4.8 us at 1 M, and one launch boundary less.
//
// Semantics and per-element rounding: dql_core.hpp (DynamicQuantizeLinear::forward,
// src/operators/dynamic_quantize_linear.rs:32-112).
#include "icx_common.hpp"
#include "internal.hpp"
#include "dql_core.hpp"
#include "qexchange.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 1024;
constexpr int kU = 8;  // float4 loads per lane in flight in the streaming loops

using namespace icx::dql;

// y's stores in the flat quantize launch: non-temporal for the stand-alone op, plain for
// the graph executor's DQLs.  Measured on MI355X: non-temporal stores take the dirty y lines
// out of the launch's end-of-kernel L2 write-back (cfg2 step: quantize 8.16 -> 6.84 us, the
// GEMM after it unchanged, 435 -> 442 TOPS), but the encoder's consumer GEMMs then run
// 0.4-0.6 us slower each (forward 1.03 -> 1.04 ms), and in the row-sum form the cfg4 step
// loses 2.6 us (921 -> 910 TOPS), so that form keeps plain stores.
template <bool NT>
__device__ __forceinline__ void put_y(uint32_t* p, uint32_t v) {
    if constexpr (NT)
        icx::store_nt_u32(p, v);
    else
        *p = v;
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

// Reduce the partials of launch 1 (every block of launch 2 does this redundantly).  All
// partials (at most kMaxPartials: the producers' grids are capped) are requested at once,
// by load_partials before the kernel requests its own data: a wave's loads complete in
// issue order, so the fold then waits for the partials alone and overlaps the data loads
// (requested after them, the fold waited for every data load: +1.6 us on a 4096 x 768
// quantize).  Both sets of loads are unconditional (clamped in-bounds index), since after
// a conditional load the compiler cannot count what is in flight and waits for everything:
// a lane past the last partial reads the last one again, which cannot move a min / max.
constexpr int kMaxPartials = 4 * kThreads;
static_assert(kMaxBlocks <= kMaxPartials && icx::kMaxRangeParts <= kMaxPartials,
              "every partial of a launch-1 grid or a range-leaving kernel is folded");
struct Partials {
    float2 v[4];
};
__device__ __forceinline__ Partials load_partials(const float2* __restrict__ part, int G) {
    Partials pv;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = threadIdx.x + u * kThreads;
        pv.v[u] = part[i < G ? i : G - 1];
    }
    return pv;
}
__device__ __forceinline__ DqlParams fold_partials(const Partials& pv) {
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        acc_minmax(pv.v[u].x, mn, mx);
        acc_minmax(pv.v[u].y, mn, mx);
    }
    block_minmax<kThreads>(mn, mx);
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
    block_minmax<kThreads>(mn, mx);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(mn, mx);
}

// Flat quantize of this block's slice: lane-consecutive float4 in, 4 bytes out (VEC: x
// 16-byte and y 4-byte aligned, unit == 4), else one element at a time.  (Two kernels, not a
// branch: with the scalar path beside it, the compiler hoisted the fold's first step above
// the data loads.)
template <bool NT, bool VEC>
__global__ void __launch_bounds__(kThreads)
dql_quantize_kernel(const float* __restrict__ x, size_t units, size_t unit, size_t tail,
                    uint8_t* __restrict__ y, const float2* __restrict__ part, int G,
                    float* __restrict__ y_scale, uint8_t* __restrict__ y_zp) {
    const Slice sl = slice_of(units, unit, tail);
    const size_t t = threadIdx.x;
    const Partials pv = load_partials(part, G);
    if constexpr (VEC) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        uint32_t* y4 = reinterpret_cast<uint32_t*>(y);
        const size_t b4 = sl.e0 / 4, end4 = b4 + (sl.e1 - sl.e0) / 4;
        size_t i = b4 + t;
        // the lane's first kU float4 are requested before the partials are folded, so the
        // fold's barriers overlap them (a slice holds at least one float4: past its end the
        // load repeats the last one, which is not stored); every later batch is guarded per
        // element, so a short last batch still has all its loads in flight at once
        float4 v[kU];
#pragma unroll
        for (int j = 0; j < kU; ++j) {
            const size_t k = i + j * kThreads;
            v[j] = x4[k < end4 ? k : end4 - 1];
        }
        __builtin_amdgcn_sched_barrier(0);  // the fold stays after the data loads' issue
        const DqlParams p = fold_partials(pv);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *y_scale = (float)p.s;
            *y_zp = (uint8_t)p.zp;
        }
        while (true) {
#pragma unroll
            for (int j = 0; j < kU; ++j)
                if (i + j * kThreads < end4) put_y<NT>(&y4[i + j * kThreads], quant4(v[j], p));
            i += kU * kThreads;
            if (i >= end4) break;
#pragma unroll
            for (int j = 0; j < kU; ++j)
                if (i + j * kThreads < end4) v[j] = x4[i + j * kThreads];
        }
        for (size_t j = end4 * 4 + t; j < sl.e1; j += kThreads) y[j] = (uint8_t)quant1(x[j], p);
    } else {
        const DqlParams p = fold_partials(pv);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *y_scale = (float)p.s;
            *y_zp = (uint8_t)p.zp;
        }
        for (size_t j = sl.e0 + t; j < sl.e1; j += kThreads) y[j] = (uint8_t)quant1(x[j], p);
    }
}

// Row mode: the slices are whole rows; one wave per row at a time, and the row sums of y
// (u8 summed as int32) are written too.  `vec`: x 16-byte and y 4-byte aligned and
// row_len % 4 == 0.
__global__ void __launch_bounds__(kThreads)
dql_quantize_rows_kernel(const float* __restrict__ x, size_t rows, size_t row_len, int vec,
                         uint8_t* __restrict__ y, int32_t* __restrict__ rowsum,
                         const float2* __restrict__ part, int G, float* __restrict__ y_scale,
                         uint8_t* __restrict__ y_zp) {
    const DqlParams p = fold_partials(load_partials(part, G));
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

// Single launch, flat mode: block b holds the float4s [256 U b, 256 U (b + 1)) of x in
// registers (U per lane, lane t the float4s 256 U b + 256 u + t), the last block also the
// n % 4 scalar tail.  The block's (min, max) goes through the exchange; once every block's
// pair is in, each block quantizes its registers and writes y.  A block whose wait ran out
// writes its part of y as 0 and counts itself in the exchange buffer's error word (block
// 0's, which every block then shares, also makes the scale NaN).  `poison` is 0 but for the
// fault test hook, which makes block 0's wait expect a tag no block publishes.
template <int U>
__global__ void __launch_bounds__(kThreads)
dql_exchange_kernel(const float* __restrict__ x, size_t n4, int tail, uint8_t* __restrict__ y,
                    float* __restrict__ y_scale, uint8_t* __restrict__ y_zp, unsigned* sync,
                    unsigned poison, unsigned long long wait) {
    const size_t i0 = (size_t)blockIdx.x * kThreads * U + threadIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        v[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);  // 0.0 never moves the range
    }
    const bool has_tail = blockIdx.x == gridDim.x - 1 && (int)threadIdx.x < tail;
    const float xt = has_tail ? x[n4 * 4 + threadIdx.x] : 0.0f;
    __shared__ unsigned s_tag;
    if (threadIdx.x == 0) s_tag = icx::qx::read_tag(sync);
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) acc4(v[u], mn, mx);
    acc_minmax(xt, mn, mx);
    block_minmax<kThreads>(mn, mx);  // (its barrier also shares s_tag)
    const unsigned tag = s_tag;
    if (threadIdx.x == 0) icx::qx::publish(sync, tag, mn, mx);
    bool ok;
    const DqlParams p = icx::qx::gather<kThreads>(sync, tag, tag ^ poison, wait, ok);
    uint32_t* y4 = reinterpret_cast<uint32_t*>(y);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        if (i < n4) y4[i] = ok ? quant4(v[u], p) : 0u;
    }
    if (has_tail) y[n4 * 4 + threadIdx.x] = ok ? (uint8_t)quant1(xt, p) : (uint8_t)0;
    if (threadIdx.x == 0) icx::qx::finish(sync, ok, p, y_scale, y_zp);
}

// Launch with U float4 per lane if the grid fits the exchange and is resident at once
// (occupancy per CU computed once per device): *launched tells whether it did; the return
// value is an ICX status.
template <int U>
int try_exchange(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                 unsigned* sync, bool* launched) {
    *launched = false;
    const size_t n4 = n / 4;
    const size_t G = icx::cdiv(std::max<size_t>(n4, 1), (size_t)kThreads * U);
    if (G > (size_t)icx::kQoutMaxBlocks) return ICX_OK;
    static int per_cu[64] = {0};
    int d = 0;
    ICX_HIP_CHECK(hipGetDevice(&d));
    if (d < 0 || d >= 64) return ICX_OK;
    if (!per_cu[d]) {
        int nb = 0;
        ICX_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, dql_exchange_kernel<U>, kThreads, 0));
        per_cu[d] = nb > 0 ? nb : -1;
    }
    if (per_cu[d] < 0 || G > (size_t)per_cu[d] * icx::num_cus()) return ICX_OK;
    unsigned long long wait = icx::wall_ticks(icx::kExchangeWaitUs);
    unsigned poison = 0;
    if (const int f = icx::qout_fault_spin()) {  // test hook
        wait = icx::wall_ticks((unsigned)f);
        poison = 0x80000000u;
    }
    hipLaunchKernelGGL(dql_exchange_kernel<U>, dim3((unsigned)G), dim3(kThreads), 0, s, x, n4, (int)(n % 4), y,
                       y_scale, y_zp, sync, poison, wait);
    ICX_LAUNCH_CHECK("dql_exchange_kernel");
    *launched = true;
    return ICX_OK;
}

}  // namespace

int icx::dql_exchange(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                      unsigned* sync) {
    if (!x || !y || !y_scale || !y_zp || !sync)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DQL exchange: null pointer");
    if (n == 0 || !icx::aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 3u) != 0)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL exchange: empty or unaligned operands");
    // the fewest float4 per lane whose grid fits: more blocks, more loads in flight
    bool done = false;
    int rc = try_exchange<1>(s, x, n, y, y_scale, y_zp, sync, &done);
    if (!rc && !done) rc = try_exchange<2>(s, x, n, y, y_scale, y_zp, sync, &done);
    if (!rc && !done) rc = try_exchange<4>(s, x, n, y, y_scale, y_zp, sync, &done);
    if (rc) return rc;
    if (!done)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL exchange: %zu elements need more than %d resident blocks of %d", n,
                 icx::kQoutMaxBlocks, kThreads * 16);
    return ICX_OK;
}

int icx::exchange_status(hipStream_t s, unsigned* sync) {
    if (!sync) ICX_FAIL(ICX_ERR_INVALID_ARG, "exchange status: null buffer");
    unsigned* word = sync + icx::kQoutErrWord;
    unsigned failed = 0;
    ICX_HIP_CHECK(hipMemcpyAsync(&failed, word, sizeof failed, hipMemcpyDeviceToHost, s));
    ICX_HIP_CHECK(hipStreamSynchronize(s));
    if (failed) {
        ICX_HIP_CHECK(hipMemsetAsync(word, 0, sizeof failed, s));
        ICX_HIP_CHECK(hipStreamSynchronize(s));
        ICX_FAIL(ICX_ERR_KERNEL,
                 "DynamicQuantizeLinear range exchange: %u failure record(s) since the last status check — a "
                 "launch that quantizes its own output (quantized-output GEMM or attention, single-launch DQL) had "
                 "blocks whose wait for the other blocks' ranges ran out (they were not all resident, e.g. other "
                 "work held CUs); its quantized output is invalid (y = 0, scale = NaN)",
                 failed);
    }
    return ICX_OK;
}

extern "C" size_t icx_exchange_buffer_size(void) { return icx::kQoutSyncBytes; }

extern "C" int icx_dynamic_quantize_linear_exchange(icx_stream_t stream, const float* x, size_t n, uint8_t* y,
                                                    float* y_scale, uint8_t* y_zp, void* sync) {
    icx::clear_error();
    return icx::dql_exchange(reinterpret_cast<hipStream_t>(stream), x, n, y, y_scale, y_zp,
                             static_cast<unsigned*>(sync));
}

extern "C" int icx_exchange_status(icx_stream_t stream, void* sync) {
    icx::clear_error();
    return icx::exchange_status(reinterpret_cast<hipStream_t>(stream), static_cast<unsigned*>(sync));
}

extern "C" size_t icx_dql_workspace_size(size_t) { return sizeof(float2) * kMaxBlocks; }

// The quantize launch alone, folding partials a producing kernel left (the same grid choice
// and kernels as the second launch below).
int icx::dql_from_parts(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                        int32_t* rowsum, size_t row_len, const float2* part, int n_part) {
    if (!x || !y || !y_scale || !y_zp || !part || n_part <= 0 || n_part > kMaxPartials)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DynamicQuantizeLinear: null pointer, or %d partials (1..%d)", n_part,
                 kMaxPartials);
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
    // float4 units only when there is at least one: the vector kernel's slices (G <= units)
    // then each hold a float4, which its first, unconditional loads read
    size_t units, unit, tail;
    if (x16 && y4 && n >= 4) {
        units = n / 4;
        unit = 4;
        tail = n % 4;
    } else {
        units = n;
        unit = 1;
        tail = 0;
    }
    const int G = (int)std::max<size_t>(1, std::min<size_t>({(size_t)kMaxBlocks, icx::cdiv(n, (size_t)kThreads * 16), units}));
    const int qvec = unit == 4 ? 1 : 0;
    if (qvec && units < (size_t)G) ICX_FAIL(ICX_ERR_INVALID_ARG, "DynamicQuantizeLinear: %d slices of %zu float4", G, units);
    if (qvec)
        hipLaunchKernelGGL((dql_quantize_kernel<false, true>), dim3(G), dim3(kThreads), 0, s, x, units, unit, tail, y,
                           part, n_part, y_scale, y_zp);
    else
        hipLaunchKernelGGL((dql_quantize_kernel<false, false>), dim3(G), dim3(kThreads), 0, s, x, units, unit, tail, y,
                           part, n_part, y_scale, y_zp);
    ICX_LAUNCH_CHECK("dql_quantize_kernel");
    return ICX_OK;
}

int icx::dql_two_launch(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                        int32_t* opt_rowsum, size_t row_len, void* ws, size_t ws_bytes, bool nt_y) {
    if (!x || !y || !y_scale || !y_zp)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DynamicQuantizeLinear: null pointer argument");
    if (!ws || ws_bytes < icx_dql_workspace_size(n))
        ICX_FAIL(ICX_ERR_WORKSPACE, "DynamicQuantizeLinear: workspace of %zu bytes needed",
                 icx_dql_workspace_size(n));
    if (opt_rowsum && (row_len == 0 || n % row_len != 0))
        ICX_FAIL(ICX_ERR_SHAPE, "DynamicQuantizeLinear: row_len %zu does not divide n = %zu",
                 row_len, n);
    float2* part = reinterpret_cast<float2*>(ws);
    const bool x16 = icx::aligned16(x), y4 = (reinterpret_cast<uintptr_t>(y) & 3u) == 0;
    // Partition: rows in row mode, float4 groups (or single elements) otherwise.  Both
    // launches use the same grid, so block b reads the same slice twice; ~4 float4 per lane.
    size_t units, unit, tail;
    if (opt_rowsum) {
        units = n / row_len;
        unit = row_len;
        tail = 0;
    } else if (x16 && y4 && n >= 4) {  // as in dql_from_parts: every slice holds a float4
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
        if (!qvec)
            hipLaunchKernelGGL((dql_quantize_kernel<false, false>), dim3(G), dim3(kThreads), 0, s, x, units, unit,
                               tail, y, part, G, y_scale, y_zp);
        else if (nt_y)
            hipLaunchKernelGGL((dql_quantize_kernel<true, true>), dim3(G), dim3(kThreads), 0, s, x, units, unit,
                               tail, y, part, G, y_scale, y_zp);
        else
            hipLaunchKernelGGL((dql_quantize_kernel<false, true>), dim3(G), dim3(kThreads), 0, s, x, units, unit,
                               tail, y, part, G, y_scale, y_zp);
        ICX_LAUNCH_CHECK("dql_quantize_kernel");
    }
    return ICX_OK;
}

extern "C" int icx_dynamic_quantize_linear(icx_stream_t stream, const float* x, size_t n,
                                           uint8_t* y, float* y_scale, uint8_t* y_zp,
                                           int32_t* opt_rowsum, size_t row_len, void* ws,
                                           size_t ws_bytes) {
    icx::clear_error();
    return icx::dql_two_launch(reinterpret_cast<hipStream_t>(stream), x, n, y, y_scale, y_zp, opt_rowsum,
                               row_len, ws, ws_bytes, true);
}
