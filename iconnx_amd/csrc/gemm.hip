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
// Tiling: v_mfma_i32_32x32x32_i8 tiles.  128x128 block tiles (4 waves of 64x64, three
// blocks per CU) by default; 64x64 when 128x128 tiles would leave CUs idle; 256x192 (12
// waves) when that gives every CU a tile; 256x256 (8 waves of 128x64) when there are at
// least 512 of them; a persistent producer/consumer kernel for K-heavy shapes with fewer
// tiles than CUs.  Operand tiles reach LDS by LDS DMA (main loops B, B2, C) or through
// registers (main loop A: any K and alignment).  Blocks are remapped so each XCD
// (blockIdx % 8) works on a contiguous, M-grouped range of tiles that shares A/B panels in
// its own L2.
#include <atomic>
#include <mutex>

#include "chain.hpp"
#include "dql_core.hpp"
#include "internal.hpp"
#include "qexchange.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 16;  // bytes per LDS row (padding against bank conflicts)
constexpr int GROUP_M = 8;

enum { OUT_I32 = 0, OUT_F32 = 1 };
// Epilogue chain forms: general per-element operands; column operands, binary ops only;
// column operands with the operand-free erf / save steps (GELU).
enum { CH_GENERAL = 0, CH_COL = 1, CH_COL_EXT = 2 };

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
    uint32_t codes;  // icx::chain_codes(chain)
    icx_chain chain;
    float2* part;    // DQL range partials of the f32 output, one per block, or null
    // Segmented output (seg_n > 0): columns [s*seg_n, (s+1)*seg_n) go to the row-major
    // [M, seg_n] tensor seg[s] instead of C.  seg_n is a multiple of the block tile width,
    // so a tile lies in one segment.
    void* seg[icx::kMaxSegments];
    int seg_n;
    // Quantized output (the GEMM is the producer of a DynamicQuantizeLinear): y as u8, its
    // scale and zero point, the exchange buffer (see qout_epilogue) and the bound of every
    // wait, in polls.
    uint8_t* qy;
    float* q_scale;
    uint8_t* q_zp;
    unsigned* q_sync;
    unsigned long long q_wait;  // exchange wait limit, wall-clock ticks
    unsigned q_poison;  // 0; the fault test hook makes block 0's wait expect tag ^ q_poison
    // Quantized input (the GEMM runs the DynamicQuantizeLinear of its A operand itself): x
    // f32 [M, K]; A (= qy) receives the DQL's y, q_scale / q_zp its scale and zero point,
    // through the same exchange; each block quantizes q_rows rows of its row panel.
    const float* xin;
    int q_rows;
};

// Output of the tile whose first column is n0: base pointer, row stride and the global
// column that is column 0 of that output.
struct OutView {
    float* base;
    int ld;
    int c0;
};
__device__ __forceinline__ OutView out_view(const GemmArgs& g, int n0) {
    if (g.seg_n <= 0) return {reinterpret_cast<float*>(g.C), g.N, 0};
    const int s = n0 / g.seg_n;
    return {reinterpret_cast<float*>(g.seg[s]), g.seg_n, s * g.seg_n};
}

__device__ __forceinline__ int load_zp(const void* p, int is_u8, int idx) {
    if (!p) return 0;
    return is_u8 ? (int)reinterpret_cast<const uint8_t*>(p)[idx]
                 : (int)reinterpret_cast<const int8_t*>(p)[idx];
}

// 16 bytes of row `row` starting at column `k` of a [rows, K] byte matrix.  Branch-free
// for VEC (K % 16 == 0, so K >= 16): the address is clamped into the matrix and `keep`
// records whether the chunk is real, so every load of a K step stays in flight; the shift
// and the zeroing of out-of-range chunks happen in fix16() when the chunk is written to
// LDS, after the MFMAs of the current step.
template <bool VEC>
__device__ __forceinline__ uint4 load16(const int8_t* base, int rows, int K, int row, int k,
                                        uint32_t xr, uint32_t& keep) {
    if (VEC) {
        keep = (row < rows && k < K) ? 0xFFFFFFFFu : 0u;
        const int8_t* p = base + (size_t)min(row, rows - 1) * K + min(k, K - 16);
        return *reinterpret_cast<const uint4*>(p);
    } else {
        keep = 0xFFFFFFFFu;
        uint32_t w[4] = {0, 0, 0, 0};
        if (row < rows) {
            const int8_t* p = base + (size_t)row * K;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (k + j < K) {
                    uint32_t b = (uint8_t)p[k + j] ^ (xr & 0xFFu);
                    w[j >> 2] |= b << (8 * (j & 3));
                }
            }
        }
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <bool VEC>
__device__ __forceinline__ uint4 fix16(uint4 v, uint32_t xr, uint32_t keep) {
    if (!VEC) return v;  // already shifted and zero-filled
    return make_uint4((v.x ^ xr) & keep, (v.y ^ xr) & keep, (v.z ^ xr) & keep, (v.w ^ xr) & keep);
}

// Logical tile of this block: XCD-contiguous, then GROUP_M-grouped.  The hardware places
// workgroup i on XCD i % 8; remapping gives each XCD a contiguous run of tiles, and the
// grouping makes consecutive tiles share A row panels, so panels stay in that XCD's L2.
__device__ __forceinline__ void tile_coords(const GemmArgs& g, int& tm, int& tn) {
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int per_group = GROUP_M * g.tiles_n;
    const int group = bid / per_group;
    const int first_m = group * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int in_group = bid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

// Wave grid WGM x WGN over the BM x BN block tile; each wave owns (BM/WGM) x (BN/WGN).
template <int BM, int BN, int WGM, int WGN>
struct EpiLayout {
    static constexpr int NW = WGM * WGN;
    static constexpr int WN = BN / WGN;
    static constexpr int SROW = WN + 8;  // floats per staged row (4-row offset = 32 banks)
    static constexpr int STAGE_BYTES = NW * 32 * SROW * 4;
    static constexpr int ROWT_OFF = STAGE_BYTES + ICX_MAX_CHAIN * BN * 4;  // after the column operands
    static constexpr int COLT_OFF = ROWT_OFF + BM * 4;                     // after the row terms
    static constexpr int BYTES = COLT_OFF + 2 * BN * 4;                    // + column terms and factors
};

__device__ const uint8_t kZeroByte = 0;
__device__ const float kOneF = 1.0f;

// A load through a global-address-space pointer: a generic (flat) load would also count in
// lgkmcnt, so every later scalar-load wait would wait for it too.
template <typename T>
__device__ __forceinline__ T load_global(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}

// The global operands of a tile's epilogue, held in registers by the wave that stages them:
// both factors of the chain's column operands, the column sums, the zero points and the row
// sums.  The tiled kernels load them before their main loop, so that the loads' latency
// (about 1.7 us at the start of a chip-wide epilogue) hides under it; gemm_epilogue writes
// them to LDS.  Wave w covers columns 64 (w % CG) .. +63 and chain steps OPW (w / CG) ..
// +OPW-1; waves w < BM / 64 cover rows 64 w .. +63.  Every load is unconditional (an absent
// factor or zero point reads a constant), so all of them are in flight at once.
template <int BM, int BN, int NW, bool OPS>
struct EpiOperands {
    static constexpr int CG = (BN + 63) / 64;
    static_assert(NW % CG == 0, "column groups must split over the waves");
    static constexpr int OPW = OPS ? (ICX_MAX_CHAIN + NW / CG - 1) / (NW / CG) : 1;
    static constexpr int RG = (BM + 63) / 64;
    static_assert(RG <= NW, "one row group per wave");
    float f0[OPW], f1[OPW];
    int32_t csum = 0, rsum = 0;
    uint8_t azp = 0, bzp = 0;

    // `wid` must be wave-uniform (readfirstlane): the op fields are then scalar loads of the
    // kernel arguments and the selects below are branch-free, so no load waits for another.
    __device__ __forceinline__ void load(const GemmArgs& g, int m0, int n0, int wid, int lane) {
        const int c = min(n0 + (wid % CG) * 64 + lane, g.N - 1);
        const int og = wid / CG;
        if constexpr (OPS) {
#pragma unroll
            for (int i = 0; i < OPW; ++i) {
                const int k = og * OPW + i;
                const icx_chain_op& op = g.chain.ops[min(k, ICX_MAX_CHAIN - 1)];
                const bool live = k < g.chain.n_ops && icx::op_takes_operand(op.op);
                f0[i] = load_global(live ? op.p0 + (op.kind0 == ICX_BCAST_SCALAR ? 0 : c) : &kOneF);
                f1[i] = load_global((live && op.p1) ? op.p1 + (op.kind1 == ICX_BCAST_SCALAR ? 0 : c) : &kOneF);
            }
        }
        // a zero offset the compiler cannot see through: as a uniform value the activation's
        // zero point would be moved to a scalar register right after its load, a wait for it
        int zero = 0;
        asm volatile("" : "+v"(zero));
        azp = load_global((g.a_zp ? reinterpret_cast<const uint8_t*>(g.a_zp) : &kZeroByte) + zero);
        if (og == 0) {
            csum = load_global(g.colsum + c);
            bzp = load_global(g.b_zp ? reinterpret_cast<const uint8_t*>(g.b_zp) + (g.b_zp_len == 1 ? 0 : c) : &kZeroByte);
        }
        if (g.rowsum_raw && wid < RG) rsum = load_global(g.rowsum_raw + min(m0 + wid * 64 + lane, g.M - 1));
    }

    // The fused DQL + GEMM launch loaded its activation scale and zero point before its
    // blocks had computed them: put the values in (every chain factor read from the scale's
    // address is a scalar operand; the host checks that).
    __device__ __forceinline__ void patch_dql(const GemmArgs& g, int wid, float xs, uint8_t zp) {
        azp = zp;
        if constexpr (OPS) {
            const int og = wid / CG;
#pragma unroll
            for (int i = 0; i < OPW; ++i) {
                const int k = og * OPW + i;
                const icx_chain_op& op = g.chain.ops[min(k, ICX_MAX_CHAIN - 1)];
                const bool live = k < g.chain.n_ops && icx::op_takes_operand(op.op);
                if (live && op.p0 == g.q_scale) f0[i] = xs;
                if (live && op.p1 == g.q_scale) f1[i] = xs;
            }
        }
    }

    // Column terms (the zero-point correction's per-column part and factor), chain operands
    // and row terms of the tile into the epilogue's LDS areas (read after a barrier).
    __device__ __forceinline__ void stage(const GemmArgs& g, int8_t* smem, int stage_bytes, int rowt_off,
                                          int colt_off, int wid, int lane) const {
        const int cl = (wid % CG) * 64 + lane;
        const int og = wid / CG;
        const int a_zp = g.a_zp_u8 ? (int)azp : (int)(int8_t)azp;
        const uint32_t amz = (uint32_t)(g.alpha - a_zp);
        const uint32_t aK = (uint32_t)g.alpha * (uint32_t)g.K;
        if (cl < BN) {
            if constexpr (OPS) {
                float* sop = reinterpret_cast<float*>(smem + stage_bytes);
#pragma unroll
                for (int k = 0; k < ICX_MAX_CHAIN; ++k) {
                    if (k / OPW != og) continue;
                    if (k < g.chain.n_ops && icx::op_takes_operand(g.chain.ops[k].op)) {
                        float a = f0[k % OPW];
                        if (g.chain.ops[k].p1) a = __fmul_rn(a, f1[k % OPW]);
                        sop[k * BN + cl] = icx::div_feeds_erf(g.chain, k) ? __fdiv_rn(1.0f, a) : a;
                    }
                }
            }
            if (og == 0) {
                const int b_zp = g.b_zp_u8 ? (int)bzp : (int)(int8_t)bzp;
                const uint32_t colfac = (uint32_t)(g.beta - b_zp);
                uint32_t* sct = reinterpret_cast<uint32_t*>(smem + colt_off);
                sct[cl] = amz * (uint32_t)csum + (uint32_t)g.K * amz * colfac;
                sct[BN + cl] = colfac;
            }
        }
        if (g.rowsum_raw && wid < RG && wid * 64 + lane < BM)
            reinterpret_cast<uint32_t*>(smem + rowt_off)[wid * 64 + lane] = (uint32_t)rsum - aK;
    }
};

// ---- epilogue ---------------------------------------------------------------------------
// Each wave stages one 32-row slab of its sub-tile at a time through LDS: the MFMA layout
// (lane = column, registers = rows) is written with the zero-point correction and the Cast
// applied, then read back row-major as float4 / int4 so that the chain runs on 4
// consecutive columns per lane with its column operands in LDS, and the global stores are
// 16-byte and contiguous along rows.  `smem` must not be in use by the main loop any more.
template <int BM, int BN, int WGM, int WGN, int OUT, int CH>
using EpiOperandsFor = EpiOperands<BM, BN, WGM * WGN, OUT == OUT_F32 && CH != CH_GENERAL>;

template <int BM, int BN, int WGM, int WGN, int OUT, int CH>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g,
                                              v16i (&acc)[BM / WGM / 32][BN / WGN / 32],
                                              int8_t* smem, int m0, int n0, float& mn, float& mx,
                                              const EpiOperandsFor<BM, BN, WGM, WGN, OUT, CH>& eo) {
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TI = WM / 32, TJ = WN / 32;
    using EL = EpiLayout<BM, BN, WGM, WGN>;
    constexpr int SROW = EL::SROW;
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int lr = lane & 31;

    eo.stage(g, smem, EL::STAGE_BYTES, EL::ROWT_OFF, EL::COLT_OFF, __builtin_amdgcn_readfirstlane(wid), lane);
    const uint32_t* sct = reinterpret_cast<const uint32_t*>(smem + EL::COLT_OFF);
    uint32_t colterm[TJ], colfac[TJ];
    constexpr int LPR = WN / 4;       // lanes per staged row in the read phase
    constexpr int RPI = 64 / LPR;     // rows per read iteration
    const int cc = (lane % LPR) * 4;  // this lane's 4 columns within the wave tile
    const int rsub = lane / LPR;
    const int gcol = n0 + wn * WN + cc;
    const float* sop = reinterpret_cast<const float*>(smem + EL::STAGE_BYTES);
    const OutView ov = out_view(g, n0);
    const bool vec_out = (ov.ld % 4 == 0) && ((reinterpret_cast<uintptr_t>(ov.base) & 15u) == 0);
    const bool rng = OUT == OUT_F32 && g.part != nullptr;  // uniform: track the DQL range
    float* stage = reinterpret_cast<float*>(smem) + wid * 32 * SROW;
    // the tile's row terms, staged once rather than loaded by every lane for every slab
    const uint32_t* srow = reinterpret_cast<const uint32_t*>(smem + EL::ROWT_OFF);

#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int rbase = m0 + wm * WM + i * 32;
        __syncthreads();  // previous slab read back; column operands and row terms written
        if (i == 0) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                colterm[j] = sct[wn * WN + j * 32 + lr];
                colfac[j] = sct[BN + wn * WN + j * 32 + lr];
            }
        }
        uint32_t rterm[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
            rterm[r] = g.rowsum_raw ? srow[wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] : 0u;
        // without row sums (the weight zero point folded away) the row term is 0: a uniform
        // branch drops its 32-bit multiply (a quarter-rate instruction) from every element
        auto stage_slab = [&](bool with_rows) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int lrow = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    uint32_t v = (uint32_t)acc[i][j][r] + colterm[j];
                    if (with_rows) v += colfac[j] * rterm[r];
                    float* dst = &stage[lrow * SROW + j * 32 + lr];
                    if (OUT == OUT_I32) *reinterpret_cast<int32_t*>(dst) = (int32_t)v;
                    else *dst = (float)(int32_t)v;  // Cast INT32 -> FLOAT, round to nearest even
                }
            }
        };
        if (g.rowsum_raw) stage_slab(true);
        else stage_slab(false);
        __syncthreads();
        constexpr int NQ = 32 / RPI;  // float4 values per lane in this slab
        // the erf-GELU chain also keeps a saved copy of every value: run it on half the slab
        // at a time so the values stay in registers at three blocks per CU
        constexpr int QC = (CH == CH_COL_EXT && NQ > 4) ? NQ / 2 : NQ;
#pragma unroll
        for (int h = 0; h < NQ; h += QC) {
            float4 v[QC];
#pragma unroll
            for (int q = 0; q < QC; ++q)
                v[q] = *reinterpret_cast<const float4*>(&stage[((h + q) * RPI + rsub) * SROW + cc]);
            if (OUT == OUT_F32) {
                if constexpr (CH != CH_GENERAL) {
                    icx::run_chain4<CH == CH_COL_EXT ? 2 : 0>(g.codes, g.chain.n_ops, v, [&](int k) {
                        return *reinterpret_cast<const float4*>(&sop[k * BN + wn * WN + cc]);
                    });
                } else {
#pragma unroll
                    for (int q = 0; q < QC; ++q) {
                        const int grow = min(rbase + (h + q) * RPI + rsub, g.M - 1);
                        float* w = reinterpret_cast<float*>(&v[q]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            w[e] = icx::apply_chain(g.chain, w[e], grow, min(gcol + e, g.N - 1), g.N);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < QC; ++q) {
                const int grow = rbase + (h + q) * RPI + rsub;
                if (grow >= g.M || gcol >= g.N) continue;
                const size_t off = (size_t)grow * ov.ld + (gcol - ov.c0);
                if (vec_out && gcol + 3 < g.N) {
                    icx::store_nt(reinterpret_cast<float4*>(ov.base + off), v[q]);
                    if (rng) {
                        icx::range_acc(v[q].x, mn, mx);
                        icx::range_acc(v[q].y, mn, mx);
                        icx::range_acc(v[q].z, mn, mx);
                        icx::range_acc(v[q].w, mn, mx);
                    }
                } else {
                    const float* w = reinterpret_cast<const float*>(&v[q]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gcol + e < g.N) {
                            ov.base[off + e] = w[e];
                            if (rng) icx::range_acc(w[e], mn, mx);
                        }
                }
            }
        }
    }
}

// ---- main loop A: register-staged (any K, any alignment) -------------------------------
// Block tile BM x BN, 4 waves in 2x2, each wave a (BM/2) x (BN/2) sub-tile made of
// TI x TJ v_mfma_i32_32x32x32_i8 tiles; two LDS stages with rows padded by 16 B.
template <int BM, int BN, bool VEC, int OUT, int CH>
__global__ void __launch_bounds__(kThreads) gemm_i8_kernel(GemmArgs g) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int AQ = BM * BK / 16 / kThreads;  // 16-byte chunks per thread per stage
    constexpr int BQ = BN * BK / 16 / kThreads;
    constexpr int TILE_BYTES = 2 * (BM + BN) * LDS_STRIDE;
    constexpr int EPI_BYTES = EpiLayout<BM, BN, 2, 2>::BYTES;
    __shared__ __attribute__((aligned(16)))
        int8_t smem[TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES];
    int8_t (*sA)[BM * LDS_STRIDE] = reinterpret_cast<int8_t (*)[BM * LDS_STRIDE]>(smem);
    int8_t (*sB)[BN * LDS_STRIDE] =
        reinterpret_cast<int8_t (*)[BN * LDS_STRIDE]>(smem + 2 * BM * LDS_STRIDE);

    int tm, tn;
    tile_coords(g, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int lr = lane & 31, lk = (lane >> 5) * 16;
    const int crow = t >> 2, ccol = (t & 3) * 16;  // this thread's chunk: row crow + 64q

    uint4 ra[AQ], rb[BQ];
    uint32_t ka[AQ], kb[BQ];
    auto gload = [&](int k0) {
#pragma unroll
        for (int q = 0; q < AQ; ++q)
            ra[q] = load16<VEC>(g.A, g.M, g.K, m0 + crow + 64 * q, k0 + ccol, g.a_xor, ka[q]);
#pragma unroll
        for (int q = 0; q < BQ; ++q)
            rb[q] = load16<VEC>(g.Bp, g.N, g.K, n0 + crow + 64 * q, k0 + ccol, 0u, kb[q]);
    };
    auto sstore = [&](int st) {
#pragma unroll
        for (int q = 0; q < AQ; ++q)
            *reinterpret_cast<uint4*>(&sA[st][(crow + 64 * q) * LDS_STRIDE + ccol]) =
                fix16<VEC>(ra[q], g.a_xor, ka[q]);
#pragma unroll
        for (int q = 0; q < BQ; ++q)
            *reinterpret_cast<uint4*>(&sB[st][(crow + 64 * q) * LDS_STRIDE + ccol]) =
                fix16<VEC>(rb[q], 0u, kb[q]);
    };

    v16i acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
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
            v4i a[TI], b[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[i] = *reinterpret_cast<const v4i*>(
                    &sA[cur][(wm * WM + i * 32 + lr) * LDS_STRIDE + ks * 32 + lk]);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                b[j] = *reinterpret_cast<const v4i*>(
                    &sB[cur][(wn * WN + j * 32 + lr) * LDS_STRIDE + ks * 32 + lk]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    float mn = 0.0f, mx = 0.0f;
    EpiOperandsFor<BM, BN, 2, 2, OUT, CH> eo;
    eo.load(g, m0, n0, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x & 63);
    gemm_epilogue<BM, BN, 2, 2, OUT, CH>(g, acc, smem, m0, n0, mn, mx, eo);
    if (OUT == OUT_F32 && g.part) icx::block_range_store<kThreads>(mn, mx, g.part);
}

// ---- main loop B: LDS DMA (K % 64 == 0, 16-byte aligned operands) ---------------------
// gfx950's global_load_lds_dwordx4 copies 16 bytes per lane from global memory straight
// into LDS (lane i of a wave lands at M0 + 16 i), so no VGPRs hold tiles in flight and
// NS-1 K steps are kept outstanding.  Each stage holds the A and B tiles as 64-byte rows
// (no padding, so one wave instruction fills 16 whole rows); the 16-byte chunk c of row r
// sits at physical slot c ^ ((r >> 2) & 3), which keeps the MFMA fragment reads (32 rows,
// one chunk each) free of bank conflicts.  The copies are issued from inline assembly so
// the compiler does not serialise every LDS read behind them; completion is tracked with
// explicit vmcnt waits: every K step issues exactly P = (BM + BN) / 64 copies per wave, so
// "stage kt has landed" is "at most P * (NS - 2) copies outstanding".  Rows past M / N
// are clamped onto the last real row: they only feed outputs that are never stored.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gptr), "s"(lds_addr)
                 : "memory", "m0");
}

// The same copy from a wave-uniform base in SGPRs plus a 32-bit per-lane byte offset (the
// saddr form): a copy's source costs one VGPR instead of a 64-bit address, and advancing
// along K is a scalar add on the base.  The host keeps every operand below 4 GiB for it.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_addr)
                 : "memory", "m0");
}

// The same copy with the sc1 (agent-scope coherence) cache bit: it reads what agent-scope
// stores of other CUs wrote, not an older copy of the line in this CU's or XCD's caches.
__device__ __forceinline__ void dma16s_coherent(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_addr)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 128x128 tiles: three blocks per CU (12 waves, <= 168 registers each) so that a chip-full
// of tiles (768 at the DistilBERT FFN shapes) runs in one round; the general per-element
// epilogue keeps the default budget (it would spill).
template <int BM, int BN, int WGM, int WGN, int NS, int OUT, int CH>
__global__ void __launch_bounds__(64 * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(BM == 128 && CH != CH_GENERAL ? 3 : 1)))
gemm_i8_dma_kernel(GemmArgs g) {
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int ROWB = 64;                        // bytes per LDS row (= K step)
    constexpr int STAGE = (BM + BN) * ROWB;
    // Only the first DW waves copy tiles (each 16-row copy is one wave instruction); the
    // other waves go straight from the barrier to their MFMAs, keeping the matrix pipe of
    // every SIMD busy while the copies are issued.
    constexpr int DW = NW >= 8 ? NW / 2 : NW;
    constexpr int PA = BM / 16 / DW, PB = BN / 16 / DW;  // copies per copying wave per stage
    constexpr int P = PA + PB;
    static_assert(PA * 16 * DW == BM && PB * 16 * DW == BN, "tile rows must split over waves");
    constexpr int TILE_BYTES = NS * STAGE;
    constexpr int EPI_BYTES = EpiLayout<BM, BN, WGM, WGN>::BYTES;
    __shared__ __attribute__((aligned(1024)))
        int8_t smem[TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES];

    int tm, tn;
    tile_coords(g, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int lr = lane & 31;
    const bool copier = wid < DW;
    const int cw = copier ? wid : 0;
    // wave-uniform LDS byte offsets of this wave's copies, in scalar registers
    const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds_addr_of(smem) + cw * PA * 16 * ROWB);
    const uint32_t lds_b = __builtin_amdgcn_readfirstlane(lds_addr_of(smem) + BM * ROWB + cw * PB * 16 * ROWB);

    // This lane's source rows / chunks for each of its copies (fixed across K steps), as
    // byte offsets from the operand's base.
    uint32_t offA[PA], offB[PB];
#pragma unroll
    for (int i = 0; i < PA; ++i) {
        const int row = (cw * PA + i) * 16 + (lane >> 2);
        const int kc = (lane & 3) ^ ((row >> 2) & 3);
        offA[i] = (uint32_t)((size_t)min(m0 + row, g.M - 1) * g.K + 16 * kc);
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
        const int row = (cw * PB + i) * 16 + (lane >> 2);
        const int kc = (lane & 3) ^ ((row >> 2) & 3);
        offB[i] = (uint32_t)((size_t)min(n0 + row, g.N - 1) * g.K + 16 * kc);
    }
    auto issue = [&](int buf, int kt) {
        if (!copier) return;
        const int8_t* a = g.A + kt * ROWB;
        const int8_t* b = g.Bp + kt * ROWB;
#pragma unroll
        for (int i = 0; i < PA; ++i) dma16s(a, offA[i], lds_a + buf * STAGE + i * 16 * ROWB);
#pragma unroll
        for (int i = 0; i < PB; ++i) dma16s(b, offB[i], lds_b + buf * STAGE + i * 16 * ROWB);
    };

    v16i acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int KT = g.K / ROWB;
    // the epilogue's operands are requested between the first stage's copies and the next
    // ones: loads complete in issue order, so the stage-0 wait below (which leaves the last
    // stage's copies in flight) also covers them, and the main loop's waits count the same
    // copies as without them
    EpiOperandsFor<BM, BN, WGM, WGN, OUT, CH> eo;
    issue(0, 0);
    eo.load(g, m0, n0, __builtin_amdgcn_readfirstlane(wid), lane);
#pragma unroll
    for (int s = 1; s < NS - 1; ++s) issue(s, min(s, KT - 1));

    // Fragment double buffering: the reads of one 32-wide half step are issued a phase
    // ahead of its MFMAs.  Per K step kt:
    //   read F1 (stage kt, half 1) | MFMAs on F0 (stage kt, half 0)
    //   wait own copies of stage kt+1; barrier (everyone is past stage kt-1); issue the
    //   copies of stage kt+NS-1 into stage kt-1's buffer
    //   read F0 (stage kt+1, half 0) | MFMAs on F1
    const uint32_t axr = g.a_xor;
    v4i fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    auto read_half = [&](int stage, int half, v4i (&fa)[TI], v4i (&fb)[TJ]) {
        const int8_t* sa = smem + stage * STAGE;
        const int8_t* sb = sa + BM * ROWB;
        const int kc = half * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = wm * WM + i * 32 + lr;
            fa[i] = *reinterpret_cast<const v4i*>(sa + row * ROWB + 16 * (kc ^ ((row >> 2) & 3)));
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int row = wn * WN + j * 32 + lr;
            fb[j] = *reinterpret_cast<const v4i*>(sb + row * ROWB + 16 * (kc ^ ((row >> 2) & 3)));
        }
    };
    auto mfma_half = [&](const v4i (&fa)[TI], const v4i (&fb)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const v4i a = fa[i] ^ (int)axr;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, fb[j], acc[i][j], 0, 0, 0);
        }
    };

    wait_vmcnt<P * (NS - 2)>();  // stage 0 has landed
    __syncthreads();
    read_half(0, 0, fa0, fb0);
    // sched_barrier(0) keeps the compiler from sinking the fragment reads below the MFMAs
    // they are meant to overlap.
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt % NS;
        read_half(cur, 1, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<P * (NS - 3 > 0 ? NS - 3 : 0)>();  // this wave's copies of stage kt+1
        __syncthreads();                              // everyone's; stage kt-1 is free
        issue((kt + NS - 1) % NS, min(kt + NS - 1, KT - 1));
        if (kt + 1 < KT) read_half((kt + 1) % NS, 0, fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();
    __syncthreads();  // all copies landed and all fragment reads done: LDS is free
    float mn = 0.0f, mx = 0.0f;
    gemm_epilogue<BM, BN, WGM, WGN, OUT, CH>(g, acc, smem, m0, n0, mn, mx, eo);
    if (OUT == OUT_F32 && g.part) icx::block_range_store<64 * WGM * WGN>(mn, mx, g.part);
}

// ---- quantized output -------------------------------------------------------------------
// For a GEMM whose f32 output is read only by a DynamicQuantizeLinear: the chain runs on the
// accumulators in their MFMA layout (lane = column), every block publishes the (min, max) of
// its tile, waits for all the others' (every block is resident — the host launches no more
// than fit — and each wait is bounded in time, q_wait wall-clock ticks), folds them into the DQL's scale and
// zero point exactly as the DQL launch would (dql_core.hpp) and writes its tile as u8
// through an LDS byte tile with 16-byte row stores.  The f32 output is never written.  No
// row term: the host requires an int8 weight whose zero point was folded away.
//
// The exchange (q_sync, bounded waits, NaN scale on failure) is qexchange.hpp's.
template <int BM, int BN, int WGM, int WGN, int CH>
__device__ __forceinline__ void qout_epilogue(const GemmArgs& g, v16i (&acc)[BM / WGM / 32][BN / WGN / 32],
                                              int8_t* smem, int m0, int n0, const unsigned& tag,
                                              const EpiOperandsFor<BM, BN, WGM, WGN, OUT_F32, CH>& eo) {
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int NT = 64 * WGM * WGN;
    // operand-free chains: only the straight-line erf-GELU (the host checks is_gelu8), whose
    // registers fit the three waves per SIMD
    constexpr int MODE = CH == CH_COL_EXT ? 3 : 0;
    constexpr int QS = BN + 16;                          // bytes per staged u8 row
    constexpr int SOP_BYTES = ICX_MAX_CHAIN * BN * 4;
    constexpr int COLT_OFF = SOP_BYTES + BM * QS;        // column terms after the byte tile
    constexpr int ROWT_OFF = COLT_OFF + 2 * BN * 4;      // (no row terms here: unused)
    static_assert(ROWT_OFF + BM * 4 <= (BM + BN) * 256, "LDS regions fit the tile buffer");
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int lr = lane & 31;
    const float* sop = reinterpret_cast<const float*>(smem);
    uint8_t* qs = reinterpret_cast<uint8_t*>(smem) + SOP_BYTES;
    // chain operands and column terms (the weight zero point is folded away: beta = 0 and no
    // b_zp, so the column term is (alpha - a_zp) * colsum) from the operands loaded before
    // the main loop
    eo.stage(g, smem, 0, ROWT_OFF, COLT_OFF, __builtin_amdgcn_readfirstlane(wid), lane);
    const uint32_t* sct = reinterpret_cast<const uint32_t*>(smem + COLT_OFF);
    __syncthreads();

    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int c = wn * WN + j * 32 + lr;  // column within the tile
        const uint32_t colterm = sct[c];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            float4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[q].x = (float)(int32_t)((uint32_t)acc[i][j][4 * q + 0] + colterm);
                v[q].y = (float)(int32_t)((uint32_t)acc[i][j][4 * q + 1] + colterm);
                v[q].z = (float)(int32_t)((uint32_t)acc[i][j][4 * q + 2] + colterm);
                v[q].w = (float)(int32_t)((uint32_t)acc[i][j][4 * q + 3] + colterm);
            }
            icx::run_chain4<MODE>(g.codes, g.chain.n_ops, v, [&](int k) {
                const float o = sop[k * BN + c];
                return make_float4(o, o, o, o);
            });
            // register 4 q + e holds row 8 q + 4 (lane >> 5) + e of this 32-row slab; only the
            // last row of tiles can reach past M (a uniform test per tile)
            const int rbase = m0 + wm * WM + i * 32 + 4 * (lane >> 5);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float* w = reinterpret_cast<const float*>(&v[q]);
                if (m0 + BM <= g.M) {
                    mn = fminf(mn, fminf(fminf(w[0], w[1]), fminf(w[2], w[3])));
                    mx = fmaxf(mx, fmaxf(fmaxf(w[0], w[1]), fmaxf(w[2], w[3])));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (rbase + 8 * q + e < g.M) icx::range_acc(w[e], mn, mx);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = __float_as_int(w[e]);
            }
        }
    }
    icx::dql::block_minmax<NT>(mn, mx);
    if (t == 0) icx::qx::publish(g.q_sync, tag, mn, mx);
    bool ok;
    const icx::dql::DqlParams p = icx::qx::gather<NT>(g.q_sync, tag, tag ^ g.q_poison, g.q_wait, ok);
    // quantize into the LDS byte tile [BM][QS]
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int c = wn * WN + j * 32 + lr;
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int r0 = wm * WM + i * 32 + 4 * (lane >> 5);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 w = make_float4(__int_as_float(acc[i][j][4 * q + 0]), __int_as_float(acc[i][j][4 * q + 1]),
                                             __int_as_float(acc[i][j][4 * q + 2]), __int_as_float(acc[i][j][4 * q + 3]));
                const uint32_t b4 = ok ? icx::dql::quant4(w, p) : 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) qs[(r0 + 8 * q + e) * QS + c] = (uint8_t)(b4 >> (8 * e));
            }
        }
    }
    __syncthreads();
    constexpr int C16 = BN / 16;
    for (int idx = t; idx < BM * C16; idx += NT) {
        const int r = idx / C16, c16 = idx - r * C16;
        const int grow = m0 + r;
        if (grow < g.M)
            *reinterpret_cast<uint4*>(g.qy + (size_t)grow * g.N + n0 + 16 * c16) =
                *reinterpret_cast<const uint4*>(qs + r * QS + 16 * c16);
    }
    if (t == 0) icx::qx::finish(g.q_sync, ok, p, g.q_scale, g.q_zp);
}

// ---- main loop B2: LDS DMA with 128-byte K rows (256x256 tile, K % 128 == 0) ------------
// The large-shape variant of main loop B.  A stage holds two 64-wide K steps as 128-byte
// LDS rows, so every lane-octet of a copy reads one whole 128-byte line of a row (the
// 64-byte rows of main loop B read half a line per copy, and the copies' throughput from L2
// is what bounds this GEMM).  Two stages of 64 KB (128 KB): the copies of stage kt+2 are
// issued into stage kt's buffer right after the barrier that ends stage kt, so they have one
// stage (four 32-wide MFMA K steps per wave) to land.  Chunk c of row r sits at slot
// c ^ ((r >> 1) & 7): the 16 lanes of a fragment read that share a cycle hit 16 distinct
// 16-byte bank groups.  Waves 0-3 issue the copies (BM / 32 8-row copies of A and BN / 32
// of B per stage each).  Four tiles: 256x256 with 8 waves of 128x64 (shapes with >= 512 such
// tiles); 256x192 with 12 waves of 64x64 — three per SIMD — for shapes that give every CU
// one such tile (the DistilBERT FFN-up: 256 tiles), where it moves 42% fewer bytes from L2
// into LDS than three 128x128 tiles per CU; 128x96 with 12 waves of 32x32 for shapes that
// give every CU one or more of those; and 64x96 with 6 waves of 32x32, two blocks per CU,
// where 128x96 would give about one (the FFN-down and output projection: 512 tiles).
// QIN: the launch also runs the DynamicQuantizeLinear of A from x (GemmArgs::xin).  Before
// its main loop, block (tm, tn) reads its q_rows rows of row panel tm into registers (QV
// float4 per lane), trades (min, max) with every block through the range exchange, quantizes
// its rows into A and publishes them (its tagged panel word); it streams its weight stages
// into LDS meanwhile, waits for the panel words of the other blocks of panel tm, and only
// then copies A.  The panel's rows cross XCDs (each XCD has its own L2): they are written
// with agent-scope stores (the sc1 bit: through to memory), every wave waits for its stores
// to complete before the barrier after which the panel word is written, and A is copied with
// sc1 loads, which do not take a stale line from this CU's or XCD's caches — the ordering an
// agent-scope release / acquire gives atomics, without the fences' passes over the whole L2
// (measured: 3.6 us of a 39 us launch).
constexpr int QV = 4;

template <int BM, int BN, int WGM, int WGN, int OUT, int CH, int QOUT = 0, int QIN = 0>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_i8_dma128_kernel(GemmArgs g) {
    static_assert(!(QOUT && QIN), "one exchange per launch");
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int ROWB = 128;
    constexpr int STAGE = (BM + BN) * ROWB;
    constexpr int DW = 4;
    constexpr int PA = BM / 8 / DW, PB = BN / 8 / DW;
    static_assert(PA * 8 * DW == BM && PB * 8 * DW == BN, "tile rows must split over the copying waves");
    static_assert(PA + PB <= 63, "outstanding copies must fit the 6-bit vmcnt");
    constexpr int TILE_BYTES = 2 * STAGE;
    constexpr int EPI_BYTES = EpiLayout<BM, BN, WGM, WGN>::BYTES;
    __shared__ __attribute__((aligned(1024)))
        int8_t smem[TILE_BYTES > EPI_BYTES ? TILE_BYTES : EPI_BYTES];

    int tm, tn;
    tile_coords(g, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const int lane = t & 63, wid = t >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int lr = lane & 31;
    const bool copier = wid < DW;
    const int cw = copier ? wid : 0;
    const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds_addr_of(smem) + cw * PA * 8 * ROWB);
    const uint32_t lds_b = __builtin_amdgcn_readfirstlane(lds_addr_of(smem) + BM * ROWB + cw * PB * 8 * ROWB);
    // lane l of a copy covers row (l >> 3) of its 8-row group, physical slot l & 7 (byte
    // offsets from the operand's base)
    uint32_t offA[PA], offB[PB];
#pragma unroll
    for (int i = 0; i < PA; ++i) {
        const int row = (cw * PA + i) * 8 + (lane >> 3);
        const int kc = (lane & 7) ^ ((row >> 1) & 7);
        offA[i] = (uint32_t)((size_t)min(m0 + row, g.M - 1) * g.K + 16 * kc);
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
        const int row = (cw * PB + i) * 8 + (lane >> 3);
        const int kc = (lane & 7) ^ ((row >> 1) & 7);
        offB[i] = (uint32_t)((size_t)min(n0 + row, g.N - 1) * g.K + 16 * kc);
    }
    const int KT = g.K / ROWB;
    // the launch number of a quantized-output launch: read by one thread before its first
    // copies (so the stage-0 wait covers it and the main loop hides its latency), shared
    // through LDS at the epilogue
    __shared__ unsigned s_qtag;
    unsigned q_tag0 = 0;
    if (QOUT != 0 && t == 0) q_tag0 = icx::qx::read_tag(g.q_sync);
    auto issue_a = [&](int buf, int kt) {
        if (!copier) return;
        const int8_t* a = g.A + kt * ROWB;
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            if constexpr (QIN != 0) dma16s_coherent(a, offA[i], lds_a + buf * STAGE + i * 8 * ROWB);
            else dma16s(a, offA[i], lds_a + buf * STAGE + i * 8 * ROWB);
        }
    };
    auto issue_b = [&](int buf, int kt) {
        if (!copier) return;
        const int8_t* b = g.Bp + kt * ROWB;
#pragma unroll
        for (int i = 0; i < PB; ++i) dma16s(b, offB[i], lds_b + buf * STAGE + i * 8 * ROWB);
    };
    auto issue = [&](int buf, int kt) {
        issue_a(buf, kt);
        issue_b(buf, kt);
    };

    v16i acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const uint32_t axr = g.a_xor;
    v4i fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    // fragments of 32-wide K step q (0..3) of a stage
    auto read_q = [&](int stage, int q, v4i (&fa)[TI], v4i (&fb)[TJ]) {
        const int8_t* sa = smem + stage * STAGE;
        const int8_t* sb = sa + BM * ROWB;
        const int kc = q * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = wm * WM + i * 32 + lr;
            fa[i] = *reinterpret_cast<const v4i*>(sa + row * ROWB + 16 * (kc ^ ((row >> 1) & 7)));
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int row = wn * WN + j * 32 + lr;
            fb[j] = *reinterpret_cast<const v4i*>(sb + row * ROWB + 16 * (kc ^ ((row >> 1) & 7)));
        }
    };
    auto mfma_q = [&](const v4i (&fa)[TI], const v4i (&fb)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const v4i a = fa[i] ^ (int)axr;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, fb[j], acc[i][j], 0, 0, 0);
        }
    };

    // the epilogue's operands are requested between stage 0's copies and stage 1's: loads
    // complete in issue order, so the stage-0 wait below also covers them, and the main
    // loop's waits count the same copies as without them
    EpiOperandsFor<BM, BN, WGM, WGN, OUT, CH> eo;
    if constexpr (QIN != 0) {
        constexpr int NT = 64 * WGM * WGN;
        __shared__ unsigned s_itag;
        __shared__ int s_late;
        if (t == 0) {
            s_itag = icx::qx::read_tag(g.q_sync);
            s_late = 0;
        }
        const int rows_m = min(BM, g.M - m0);
        const int r0 = min(tn * g.q_rows, rows_m), r1 = min(r0 + g.q_rows, rows_m);
        const int n4 = (r1 - r0) * (g.K / 4);
        const float4* xs4 = reinterpret_cast<const float4*>(g.xin + (size_t)(m0 + r0) * g.K);
        float4 xv[QV];
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const int q = t + u * NT;
            xv[u] = q < n4 ? xs4[q] : make_float4(0.f, 0.f, 0.f, 0.f);  // 0.0 never moves the range
        }
        float qmn = 0.0f, qmx = 0.0f;
#pragma unroll
        for (int u = 0; u < QV; ++u) icx::dql::acc4(xv[u], qmn, qmx);
        icx::dql::block_minmax<NT>(qmn, qmx);  // its barrier also publishes s_itag
        const unsigned tag = s_itag;
        if (t == 0) icx::qx::publish(g.q_sync, tag, qmn, qmx);
        // the weight's first two stages and the epilogue operands stream in during the exchange
        issue_b(0, 0);
        eo.load(g, m0, n0, __builtin_amdgcn_readfirstlane(wid), lane);
        issue_b(1, min(1, KT - 1));
        bool ok;
        const icx::dql::DqlParams p = icx::qx::gather<NT, true>(g.q_sync, tag, tag ^ g.q_poison, g.q_wait, ok);
        uint32_t* ya = reinterpret_cast<uint32_t*>(g.qy + (size_t)(m0 + r0) * g.K);
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const int q = t + u * NT;
            if (q < n4)
                __hip_atomic_store(ya + q, ok ? icx::dql::quant4(xv[u], p) : 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        if (t == 0) icx::qx::finish(g.q_sync, ok, p, g.q_scale, g.q_zp);
        // every wave's rows in memory before the block's panel word says they are there
        wait_vmcnt<0>();
        __syncthreads();
        unsigned* pw = icx::qx::panel(g.q_sync) + tm * g.tiles_n;
        if (t == 0) __hip_atomic_store(pw + tn, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t < g.tiles_n) {
            const unsigned long long t0 = wall_clock64();
            while (__hip_atomic_load(pw + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag) {
                if (wall_clock64() - t0 > g.q_wait) {
                    s_late = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();  // the copies of A (coherent loads) start after every panel word was seen
        const bool good = ok && s_late == 0;
        if (t == 0 && ok && !good)
            __hip_atomic_fetch_add(g.q_sync + icx::kQoutErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        eo.patch_dql(g, __builtin_amdgcn_readfirstlane(wid), good ? (float)p.s : __builtin_nanf(""),
                     (uint8_t)p.zp);
        issue_a(0, 0);
        issue_a(1, min(1, KT - 1));
        wait_vmcnt<PA>();  // stage 0 has landed (the wait before the panel word covered the weight's)
    } else {
        issue(0, 0);
        eo.load(g, m0, n0, __builtin_amdgcn_readfirstlane(wid), lane);
        issue(1, min(1, KT - 1));
        wait_vmcnt<PA + PB>();  // stage 0 has landed
    }
    __syncthreads();
    read_q(0, 0, fa0, fb0);
    // Per stage: the reads of K step q+1 are issued before the MFMAs of step q; between
    // steps 2 and 3 every wave waits for its copies of stage kt+1 and the barrier frees
    // stage kt's buffer (its last fragments are in registers) for the copies of stage kt+2.
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        read_q(cur, 1, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        mfma_q(fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        read_q(cur, 2, fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        mfma_q(fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        read_q(cur, 3, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        mfma_q(fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<0>();   // this wave's copies of stage kt+1
        __syncthreads();   // everyone's; stage kt is fully read
        issue(cur, min(kt + 2, KT - 1));
        if (kt + 1 < KT) read_q(cur ^ 1, 0, fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        mfma_q(fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();
    __syncthreads();  // all copies landed and all fragment reads done: LDS is free
    float mn = 0.0f, mx = 0.0f;
    if constexpr (QOUT != 0) {
        if (t == 0) s_qtag = q_tag0;  // read by every thread after the epilogue's first barrier
        qout_epilogue<BM, BN, WGM, WGN, CH>(g, acc, smem, m0, n0, s_qtag, eo);
        return;
    }
    gemm_epilogue<BM, BN, WGM, WGN, OUT, CH>(g, acc, smem, m0, n0, mn, mx, eo);
    if (OUT == OUT_F32 && g.part) icx::block_range_store<64 * WGM * WGN>(mn, mx, g.part);
}

// ---- main loop C: persistent producer / consumer (K % 64 == 0, column-only epilogue) ----
// One block per CU slot loops over tiles (virtual tile ids blockIdx.x, +gridDim.x, ...,
// mapped XCD-contiguous like tile_coords).  The K steps of all of a block's tiles form
// one flat sequence of S = tiles x KT steps:
//   * one producer wave (the last) issues every LDS DMA copy, NS-1 steps ahead, and is
//     the only wave that waits on vmcnt;
//   * the WGM x WGN consumer waves read fragments and run the MFMAs, and after a tile's
//     last K step convert, correct, chain and store their accumulators straight from
//     registers with non-temporal stores.  Consumers issue no loads the main loop waits
//     for, so those stores drain while the next tile's MFMAs run.
// The per-tile epilogue operands (column sums, per-column zero points, column factors,
// row sums) are loaded by each consumer at the start of the tile and first used after
// its last K step, by which time the previous tile's stores have long left.
// Barrier protocol (every wave executes exactly S + 1 barriers, all at top level):
//   barrier(-1): stage 0 has landed;
//   barrier(s):  stage s+1 has landed, and every consumer is done reading stage s-1, so
//                after it the producer refills stage s-1's buffer with step s+NS-1.
// Steps past the end re-copy the last step into the free buffer so that every step
// issues exactly P copies and the counted vmcnt waits stay exact.
template <int BM, int BN, int WGM, int WGN>
struct StreamLayout {
    static constexpr int NC = WGM * WGN;          // consumer waves
    static constexpr int WN = BN / WGN;
    static constexpr int OPND_BYTES = NC * ICX_MAX_CHAIN * WN * 4;  // per-wave operand rows
};

__device__ __forceinline__ void stream_tile(const GemmArgs& g, int v, int T, int& tm, int& tn) {
    int bid = v;
    if ((T & 7) == 0 && (gridDim.x & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int per_group = GROUP_M * g.tiles_n;
    const int group = bid / per_group;
    const int first_m = group * GROUP_M;
    const int gsz = min(g.tiles_m - first_m, GROUP_M);
    const int in_group = bid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

template <int BM, int BN, int WGM, int WGN, int NP, int NS, int OUT, int CH>
__global__ void __launch_bounds__(64 * (WGM * WGN + NP))
gemm_i8_stream_kernel(GemmArgs g) {
    using SL = StreamLayout<BM, BN, WGM, WGN>;
    constexpr int NC = SL::NC;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int ROWB = 64;
    constexpr int STAGE = (BM + BN) * ROWB;
    constexpr int PA = BM / 16 / NP, PB = BN / 16 / NP, P = PA + PB;  // copies per producer per step
    static_assert(PA * 16 * NP == BM && PB * 16 * NP == BN, "tile rows must split over the producers");
    static_assert(NS >= 3, "the protocol reads stages s and s+1 while s+2.. are in flight");
    static_assert(P * (NS - 2) <= 63, "outstanding copies must fit the 6-bit vmcnt");
    constexpr int MODE = CH == CH_COL_EXT ? 2 : 0;
    __shared__ __attribute__((aligned(1024))) int8_t smem[NS * STAGE + SL::OPND_BYTES];

    const int T = g.tiles_m * g.tiles_n;
    const int G = gridDim.x;
    const int ntiles = (T - (int)blockIdx.x + G - 1) / G;  // >= 1: the host launches G <= T
    const int KT = g.K / ROWB;
    const int S = ntiles * KT;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float rmn = 0.0f, rmx = 0.0f;  // DQL range of the output (consumers; when g.part is given)

    if (wid >= NC) {
        // ------------------------------ producers -----------------------------------------
        // Producer p copies rows [p*BM/NP, (p+1)*BM/NP) of the A tile and the same share of
        // the B tile.  Row pointers are computed once per tile; a step only adds its K offset.
        const int p = __builtin_amdgcn_readfirstlane(wid - NC);
        const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr_of(smem));
        const uint32_t ldsA = lds0 + p * PA * 16 * ROWB, ldsB = lds0 + BM * ROWB + p * PB * 16 * ROWB;
        int rowA[PA], rowB[PB], kcA[PA], kcB[PB];
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            rowA[i] = (p * PA + i) * 16 + (lane >> 2);
            kcA[i] = 16 * ((lane & 3) ^ ((rowA[i] >> 2) & 3));
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            rowB[i] = (p * PB + i) * 16 + (lane >> 2);
            kcB[i] = 16 * ((lane & 3) ^ ((rowB[i] >> 2) & 3));
        }
        uint32_t offA[PA], offB[PB];  // byte offsets from the operands' bases
        auto set_tile = [&](int ordinal) {
            int tm, tn;
            stream_tile(g, (int)blockIdx.x + ordinal * G, T, tm, tn);
#pragma unroll
            for (int i = 0; i < PA; ++i)
                offA[i] = (uint32_t)((size_t)min(tm * BM + rowA[i], g.M - 1) * g.K + kcA[i]);
#pragma unroll
            for (int i = 0; i < PB; ++i)
                offB[i] = (uint32_t)((size_t)min(tn * BN + rowB[i], g.N - 1) * g.K + kcB[i]);
        };
        // Issue state: the step being issued, as (tile ordinal, K step).
        int it = 0, ik = 0, buf = 0;
        set_tile(0);
        auto issue_next = [&]() {
            const uint32_t off = __builtin_amdgcn_readfirstlane(buf * STAGE);
            const int8_t* a = g.A + __builtin_amdgcn_readfirstlane(ik * ROWB);
            const int8_t* b = g.Bp + __builtin_amdgcn_readfirstlane(ik * ROWB);
#pragma unroll
            for (int i = 0; i < PA; ++i)
                dma16s(a, offA[i], __builtin_amdgcn_readfirstlane(ldsA + off + i * 16 * ROWB));
#pragma unroll
            for (int i = 0; i < PB; ++i)
                dma16s(b, offB[i], __builtin_amdgcn_readfirstlane(ldsB + off + i * 16 * ROWB));
            buf = buf + 1 == NS ? 0 : buf + 1;
            // advance to the next step; past the last one keep re-copying it
            if (it * KT + ik + 1 < S) {
                if (++ik == KT) {
                    ik = 0;
                    set_tile(++it);
                }
            }
        };
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) issue_next();
        wait_vmcnt<P * (NS - 2)>();  // stage 0
        __syncthreads();               // barrier(-1)
        for (int s = 0; s < S; ++s) {
            wait_vmcnt<P * (NS - 3)>();  // stage s+1
            __syncthreads();               // barrier(s)
            issue_next();                  // step s+NS-1 into stage s-1's buffer
        }
        wait_vmcnt<0>();  // no copy may still target this block's LDS when it exits
    } else {
    // -------------------------------- consumers --------------------------------------------
    const int wm = wid / WGN, wn = wid % WGN;
    const int lr = lane & 31;
    float* opnd = reinterpret_cast<float*>(smem + NS * STAGE) + wid * ICX_MAX_CHAIN * WN;

    // scalars, loaded before any store is issued
    const int azp = load_zp(g.a_zp, g.a_zp_u8, 0);
    const int bzp_scalar = (g.b_zp && g.b_zp_len == 1) ? load_zp(g.b_zp, g.b_zp_u8, 0) : 0;
    const uint32_t amz = (uint32_t)(g.alpha - azp);
    const uint32_t aK = (uint32_t)g.alpha * (uint32_t)g.K;

    const uint32_t axr = g.a_xor;
    v4i fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    auto read_half = [&](int stage, int half, v4i (&fa)[TI], v4i (&fb)[TJ]) {
        const int8_t* sa = smem + stage * STAGE;
        const int8_t* sb = sa + BM * ROWB;
        const int kc = half * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = wm * WM + i * 32 + lr;
            fa[i] = *reinterpret_cast<const v4i*>(sa + row * ROWB + 16 * (kc ^ ((row >> 2) & 3)));
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int row = wn * WN + j * 32 + lr;
            fb[j] = *reinterpret_cast<const v4i*>(sb + row * ROWB + 16 * (kc ^ ((row >> 2) & 3)));
        }
    };
    v16i acc[TI][TJ];
    auto mfma_half = [&](const v4i (&fa)[TI], const v4i (&fb)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const v4i a = fa[i] ^ (int)axr;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, fb[j], acc[i][j], 0, 0, 0);
        }
    };

    __syncthreads();  // barrier(-1)
    read_half(0, 0, fa0, fb0);
    int cur = 0;  // stage buffer of step s
    int s = 0;
    for (int t = 0; t < ntiles; ++t) {
        int tm, tn;
        stream_tile(g, (int)blockIdx.x + t * G, T, tm, tn);
        const int m0 = tm * BM + wm * WM, n0 = tn * BN + wn * WN;
        // epilogue operands of this tile (first used after the last K step)
        int cs[TJ], bz[TJ];
        float ov[TJ][ICX_MAX_CHAIN];
        int rs[TI];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = min(n0 + j * 32 + lr, g.N - 1);
            cs[j] = g.colsum[col];
            bz[j] = (g.b_zp && g.b_zp_len != 1) ? load_zp(g.b_zp, g.b_zp_u8, col) : bzp_scalar;
            if (OUT == OUT_F32) {
#pragma unroll
                for (int k = 0; k < ICX_MAX_CHAIN; ++k) {
                    ov[j][k] = (k < g.chain.n_ops && icx::op_takes_operand(g.chain.ops[k].op))
                                   ? icx::col_operand(g.chain, k, col) : 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TI; ++i)
            rs[i] = g.rowsum_raw ? g.rowsum_raw[min(m0 + i * 32 + lr, g.M - 1)] : 0;
        // keep those loads here, ahead of the main loop
        asm volatile("" ::: "memory");

#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

        for (int kt = 0; kt < KT; ++kt, ++s) {
            const int nxt = cur + 1 == NS ? 0 : cur + 1;
            read_half(cur, 1, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_half(fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();  // barrier(s)
            if (s + 1 < S) read_half(nxt, 0, fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_half(fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
        }

        // ---- epilogue straight from the accumulators -------------------------------------
        // lane = column (n0 + j*32 + lr); register r of tile (i, j) = row
        // m0 + i*32 + 8*(r>>2) + 4*(lane>>5) + (r&3).
        const OutView ow = out_view(g, tn * BN);
        uint32_t colfac[TJ], colterm[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            colfac[j] = (uint32_t)(g.beta - bz[j]);
            colterm[j] = amz * (uint32_t)cs[j] + (uint32_t)g.K * amz * colfac[j];
            if (OUT == OUT_F32) {
#pragma unroll
                for (int k = 0; k < ICX_MAX_CHAIN; ++k)
                    if (k < g.chain.n_ops) opnd[k * WN + j * 32 + lr] = ov[j][k];
            }
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int rbase = m0 + i * 32 + 4 * (lane >> 5);
            uint32_t rt[16];  // row term of each register's row (row sums are held by lane = row)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                rt[r] = g.rowsum_raw
                            ? (uint32_t)__shfl(rs[i], 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), 64) - aK
                            : 0u;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int col = n0 + j * 32 + lr;
                float4 v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float* w = reinterpret_cast<float*>(&v[q]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * q + e;
                        const uint32_t x = (uint32_t)acc[i][j][r] + colterm[j] + colfac[j] * rt[r];
                        if (OUT == OUT_I32) w[e] = __int_as_float((int32_t)x);
                        else w[e] = (float)(int32_t)x;  // Cast INT32 -> FLOAT (RNE)
                    }
                }
                if (OUT == OUT_F32) {
                    icx::run_chain4<MODE>(g.codes, g.chain.n_ops, v, [&](int k) {
                        const float o = opnd[k * WN + j * 32 + lr];
                        return make_float4(o, o, o, o);
                    });
                }
                if (col < g.N) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float* w = reinterpret_cast<const float*>(&v[q]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int row = rbase + 8 * q + e;
                            if (row < g.M) {
                                __builtin_nontemporal_store(
                                    w[e], ow.base + (size_t)row * ow.ld + (col - ow.c0));
                                if (OUT == OUT_F32 && g.part) icx::range_acc(w[e], rmn, rmx);
                            }
                        }
                    }
                }
            }
        }
    }
    }  // consumers
    if (OUT == OUT_F32 && g.part) icx::block_range_store<64 * (WGM * WGN + NP)>(rmn, rmx, g.part);
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

// Raw row sums of A (bytes as u8 or i8), one wave per row; 16-byte loads summed with the
// 4-way byte dot product against 0x01010101 when rows are 16-byte aligned.
__global__ void __launch_bounds__(kThreads)
rowsum_kernel(const void* __restrict__ A, int is_u8, int M, int K, int vec,
              int32_t* __restrict__ rowsum) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (m >= M) return;
    int s = 0;
    const uint8_t* row = reinterpret_cast<const uint8_t*>(A) + (size_t)m * K;
    if (vec) {
        const uint4* r16 = reinterpret_cast<const uint4*>(row);
        const int n16 = K / 16;
#pragma unroll 4
        for (int i = lane; i < n16; i += 64) {
            const uint4 v = r16[i];
            if (is_u8) {
                s = (int)__builtin_amdgcn_udot4(v.x, 0x01010101u, (uint32_t)s, false);
                s = (int)__builtin_amdgcn_udot4(v.y, 0x01010101u, (uint32_t)s, false);
                s = (int)__builtin_amdgcn_udot4(v.z, 0x01010101u, (uint32_t)s, false);
                s = (int)__builtin_amdgcn_udot4(v.w, 0x01010101u, (uint32_t)s, false);
            } else {
                s = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, s, false);
            }
        }
    } else if (is_u8) {
        for (int k = lane; k < K; k += 64) s += (int)row[k];
    } else {
        for (int k = lane; k < K; k += 64) s += (int)(int8_t)row[k];
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

template <int BM, int BN, bool VEC>
void launch_reg_v(int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(kThreads);
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, VEC, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else if (ch == CH_COL)
        hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, VEC, OUT_F32, CH_COL>), grid, block, 0, s, g);
    else if (ch == CH_COL_EXT)
        hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, VEC, OUT_F32, CH_COL_EXT>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, VEC, OUT_F32, CH_GENERAL>), grid, block, 0, s, g);
}

template <int BM, int BN>
void launch_reg(bool vec, int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    if (vec) launch_reg_v<BM, BN, true>(out_kind, ch, blocks, s, g);
    else launch_reg_v<BM, BN, false>(out_kind, ch, blocks, s, g);
}

template <int BM, int BN, int WGM, int WGN, int NS>
void launch_dma(int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(64 * WGM * WGN);
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_dma_kernel<BM, BN, WGM, WGN, NS, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else if (ch == CH_COL)
        hipLaunchKernelGGL((gemm_i8_dma_kernel<BM, BN, WGM, WGN, NS, OUT_F32, CH_COL>), grid, block, 0, s, g);
    else if (ch == CH_COL_EXT)
        hipLaunchKernelGGL((gemm_i8_dma_kernel<BM, BN, WGM, WGN, NS, OUT_F32, CH_COL_EXT>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_dma_kernel<BM, BN, WGM, WGN, NS, OUT_F32, CH_GENERAL>), grid, block, 0, s, g);
}

// The 256x256 tile is only instantiated for int32 output and binary column chains (its
// register budget has no room for the general or GELU epilogues).  K % 128 == 0 takes the
// 128-byte-row main loop.
template <int WGM, int WGN, int NS>
void launch_dma_big(int out_kind, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(64 * WGM * WGN);
    if (g.K % 128 == 0) {
        if (out_kind == OUT_I32)
            hipLaunchKernelGGL((gemm_i8_dma128_kernel<256, 256, 2, 4, OUT_I32, CH_GENERAL>), grid, dim3(512), 0, s, g);
        else
            hipLaunchKernelGGL((gemm_i8_dma128_kernel<256, 256, 2, 4, OUT_F32, CH_COL>), grid, dim3(512), 0, s, g);
        return;
    }
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_dma_kernel<256, 256, WGM, WGN, NS, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_dma_kernel<256, 256, WGM, WGN, NS, OUT_F32, CH_COL>), grid, block, 0, s, g);
}

// 256x192 tiles, 12 waves (K % 128 == 0, column chains or int32 output).
void launch_dma_mid(int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(768);
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<256, 192, 4, 3, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else if (ch == CH_COL_EXT)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<256, 192, 4, 3, OUT_F32, CH_COL_EXT>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<256, 192, 4, 3, OUT_F32, CH_COL>), grid, block, 0, s, g);
}

// 64x96 tiles (6 waves of 32x32, two blocks per CU) when 128x96 ones give every CU about one:
// two independent pipelines per CU hide some of each other's copy latency (the encoder's
// output projection and FFN-down: 16.83 -> 16.52 us per launch on average).
void launch_dma_narrow64(int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(384);
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<64, 96, 2, 3, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else if (ch == CH_COL_EXT)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<64, 96, 2, 3, OUT_F32, CH_COL_EXT>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<64, 96, 2, 3, OUT_F32, CH_COL>), grid, block, 0, s, g);
}

// 128x96 tiles, 12 waves of 32x32 (K % 128 == 0, column chains or int32 output).
void launch_dma_narrow(int out_kind, int ch, unsigned blocks, hipStream_t s, const GemmArgs& g) {
    const dim3 grid(blocks), block(768);
    if (out_kind == OUT_I32)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<128, 96, 4, 3, OUT_I32, CH_GENERAL>), grid, block, 0, s, g);
    else if (ch == CH_COL_EXT)
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<128, 96, 4, 3, OUT_F32, CH_COL_EXT>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((gemm_i8_dma128_kernel<128, 96, 4, 3, OUT_F32, CH_COL>), grid, block, 0, s, g);
}

// Persistent producer / consumer kernel: grid = min(tiles, resident blocks), resident
// blocks from the occupancy calculator (cached per instantiation and device).

template <int BM, int BN, int WGM, int WGN, int NP, int NS, int OUT, int CH>
int launch_stream_one(unsigned tiles, hipStream_t s, GemmArgs g) {
    auto kern = gemm_i8_stream_kernel<BM, BN, WGM, WGN, NP, NS, OUT, CH>;
    constexpr int threads = 64 * (WGM * WGN + NP);
    static int per_cu[64] = {0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    const int d = (dev >= 0 && dev < 64) ? dev : 0;
    if (!per_cu[d]) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), threads, 0) !=
                hipSuccess || nb <= 0)
            nb = 1;
        per_cu[d] = nb;
    }
    unsigned grid = (unsigned)(per_cu[d] * icx::num_cus());
    if (grid > tiles) grid = tiles;
    if (grid > (unsigned)icx::kMaxRangeParts) g.part = nullptr;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), 0, s, g);
    return g.part ? (int)grid : 0;
}

// Returns the number of range partials written (0: none).
template <int BM, int BN, int WGM, int WGN, int NP, int NS>
int launch_stream(int out_kind, int ch, unsigned tiles, hipStream_t s, const GemmArgs& g) {
    if (out_kind == OUT_I32)
        return launch_stream_one<BM, BN, WGM, WGN, NP, NS, OUT_I32, CH_GENERAL>(tiles, s, g);
    else if (ch == CH_COL_EXT)
        return launch_stream_one<BM, BN, WGM, WGN, NP, NS, OUT_F32, CH_COL_EXT>(tiles, s, g);
    else
        return launch_stream_one<BM, BN, WGM, WGN, NP, NS, OUT_F32, CH_COL>(tiles, s, g);
}

// 256x192 tiles quantizing their own output: every block must be resident at once, so the
// launch is refused (ICX_ERR_UNSUPPORTED, nothing launched) when the occupancy calculator
// says the grid does not fit.
template <int CH>
int launch_qout(unsigned blocks, hipStream_t s, const GemmArgs& g) {
    auto kern = gemm_i8_dma128_kernel<256, 192, 4, 3, OUT_F32, CH, 1>;
    static int per_cu[64] = {0};
    int d = 0;
    ICX_HIP_CHECK(hipGetDevice(&d));
    if (d < 0 || d >= 64) ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: device index %d", d);
    if (!per_cu[d]) {
        int n = 0;
        ICX_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, 768, 0));
        per_cu[d] = n > 0 ? n : -1;
    }
    if (per_cu[d] < 0 || blocks > (unsigned)(per_cu[d] * icx::num_cus()))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: %u blocks exceed the %d resident ones", blocks,
                 per_cu[d] * icx::num_cus());
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(768), 0, s, g);
    ICX_LAUNCH_CHECK("gemm_i8_dma128_kernel (quantized output)");
    return ICX_OK;
}

// Resident blocks per CU of a kernel of `threads` threads (cached per device in *cache).
template <typename Kern>
int resident_per_cu(Kern kern, int threads, int* cache) {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 0;
    if (!cache[d]) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, 0) != hipSuccess) n = 0;
        cache[d] = n > 0 ? n : -1;
    }
    return cache[d] > 0 ? cache[d] : 0;
}

// The quantized-input launch on BM x BN tiles of WGM x WGN waves: ICX_ERR_UNSUPPORTED unless
// every block is resident at once.
template <int BM, int BN, int WGM, int WGN, int CH>
int launch_qin(unsigned blocks, hipStream_t s, const GemmArgs& g) {
    auto kern = gemm_i8_dma128_kernel<BM, BN, WGM, WGN, OUT_F32, CH, 0, 1>;
    static int per_cu[64] = {0};
    const int n = resident_per_cu(kern, 64 * WGM * WGN, per_cu);
    if (n <= 0 || blocks > (unsigned)(n * icx::num_cus()))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: %u blocks exceed the %d resident ones", blocks,
                 n * icx::num_cus());
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WGM * WGN), 0, s, g);
    ICX_LAUNCH_CHECK("gemm_i8_dma128_kernel (quantized input)");
    return ICX_OK;
}

int gemm_common(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype,
                int b_packed, const int32_t* b_colsum, size_t M, size_t K, size_t N,
                const void* a_zp, const void* b_zp, size_t b_zp_len, const int32_t* a_rowsum,
                const icx_chain* chain, void* C, int out_kind, void* ws, size_t ws_bytes,
                const char* who, float2* part = nullptr, int* n_part = nullptr,
                float* const* segs = nullptr, int n_seg = 0) {
    if (n_part) *n_part = 0;
    if (n_seg) {
        if (out_kind != OUT_F32 || n_seg < 1 || n_seg > icx::kMaxSegments || N % n_seg != 0 ||
            (N / n_seg) % 256 != 0 || part)
            ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: %d output segments over N = %zu (segments must be equal, a "
                     "multiple of 256 columns, at most %d, no range partials)", who, n_seg, N, icx::kMaxSegments);
        for (int i = 0; i < n_seg; ++i)
            if (!segs[i]) ICX_FAIL(ICX_ERR_INVALID_ARG, "%s: null output segment %d", who, i);
        C = segs[0];
    }
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
            const int rvec = (K % 16 == 0 && icx::aligned16(A)) ? 1 : 0;
            hipLaunchKernelGGL(rowsum_kernel, dim3((unsigned)icx::cdiv(M, kThreads / 64)),
                               dim3(kThreads), 0, s, A, a_dtype == ICX_U8 ? 1 : 0, (int)M,
                               (int)K, rvec, rs);
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
    g.tiles_m = (int)icx::cdiv(M, 128);
    g.tiles_n = (int)icx::cdiv(N, 128);
    g.a_xor = a_dtype == ICX_U8 ? 0x80808080u : 0u;
    g.alpha = alpha;
    g.beta = beta;
    g.a_zp_u8 = a_dtype == ICX_U8;
    g.b_zp_u8 = b_dtype == ICX_U8;
    g.b_zp_len = (int)(b_zp ? b_zp_len : 1);
    if (chain) g.chain = *chain;
    else g.chain.n_ops = 0;
    g.codes = icx::chain_codes(g.chain);
    g.seg_n = n_seg ? (int)(N / n_seg) : 0;
    for (int i = 0; i < n_seg; ++i) g.seg[i] = segs[i];

    const bool vec = K >= 16 && (K % 16 == 0) && icx::aligned16(A) && icx::aligned16(Bp);
    // (the LDS-DMA main loops address each operand as a base plus 32-bit byte offsets)
    const bool dma = vec && K >= 64 && K % 64 == 0 && (uint64_t)M * K <= 0xffffffffull &&
                     (uint64_t)N * K <= 0xffffffffull;
    const bool colchain = out_kind == OUT_F32 && icx::chain_is_col_only(g.chain);
    const int ch = !colchain ? CH_GENERAL : (icx::chain_mode(g.chain) == 2 ? CH_COL_EXT : CH_COL);
    // 256x256 tiles (128x128 per wave) when there are enough of them to fill the chip;
    // otherwise 128x128 so that every CU gets tiles.  Row / full-tensor chain operands
    // take the general per-element path, kept on the 128x128 tile.
    const bool big = icx::cdiv(M, 256) * icx::cdiv(N, 256) >= 512 && (out_kind == OUT_I32 || ch == CH_COL);
    // K-heavy shapes with fewer 64x64 tiles than CUs: the persistent producer / consumer
    // kernel, whose 8 MFMA waves per tile hide the long K loop better than 4.  (The encoder's
    // FFN-down projection, 4096x3072x768, runs faster as 768 tiles of 64x64.)
    const bool stream = dma && (out_kind == OUT_I32 || ch != CH_GENERAL) && K >= 2048 &&
                        icx::cdiv(M, 64) * icx::cdiv(N, 64) < (size_t)icx::num_cus();
    if (stream) {
        g.tiles_m = (int)icx::cdiv(M, 128);
        g.tiles_n = (int)icx::cdiv(N, 128);
        if (out_kind == OUT_F32) g.part = part;
        const int np = launch_stream<128, 128, 4, 2, 2, 4>(out_kind, ch, (unsigned)(g.tiles_m * g.tiles_n), s, g);
        ICX_LAUNCH_CHECK("gemm_i8_stream_kernel");
        if (n_part) *n_part = np;
        return ICX_OK;
    }
    // 256x192 tiles when they give at least three quarters of the CUs one (and no partial
    // column tile): fewer operand bytes per output than three 128x128 tiles per CU (the
    // encoder's Q/K/V group, 192 tiles: 2.6 us less per forward than 576 of 128x128)
    const bool mid = !big && dma && K % 128 == 0 && N % 192 == 0 && (out_kind == OUT_I32 || ch != CH_GENERAL) &&
                     icx::cdiv(M, 256) * (N / 192) * 4 >= (size_t)icx::num_cus() * 3 &&
                     (n_seg == 0 || (N / n_seg) % 192 == 0);
    // 128x96 tiles (12 waves of 32x32) when those give every CU at least one, for a single
    // output (the encoder's FFN-down 4096x3072x768: 24.3 -> 21.0 us; its output projection
    // 4096x768x768: 10.2 -> 9.1 us; over a Q/K/V group the segmented store ran slower)
    const bool narrow = !big && !mid && dma && K % 128 == 0 && N % 96 == 0 && n_seg == 0 &&
                        (out_kind == OUT_I32 || ch != CH_GENERAL) &&
                        icx::cdiv(M, 128) * (N / 96) >= (size_t)icx::num_cus();
    const bool narrow64 = narrow && icx::cdiv(M, 64) * (N / 96) <= 2 * (size_t)icx::num_cus();
    // 64x64 tiles when 128x128 ones would leave CUs idle (up to six blocks per CU to hide
    // each K step's latency)
    const bool small = dma && !big && !mid && !narrow && icx::cdiv(M, 128) * icx::cdiv(N, 128) < (size_t)icx::num_cus();
    if (big) {
        g.tiles_m = (int)icx::cdiv(M, 256);
        g.tiles_n = (int)icx::cdiv(N, 256);
    } else if (mid) {
        g.tiles_m = (int)icx::cdiv(M, 256);
        g.tiles_n = (int)(N / 192);
    } else if (narrow) {
        g.tiles_m = (int)icx::cdiv(M, narrow64 ? 64 : 128);
        g.tiles_n = (int)(N / 96);
    } else if (small) {
        g.tiles_m = (int)icx::cdiv(M, 64);
        g.tiles_n = (int)icx::cdiv(N, 64);
    }
    const unsigned blocks = (unsigned)(g.tiles_m * g.tiles_n);
    if (out_kind == OUT_F32 && part && blocks <= (unsigned)icx::kMaxRangeParts) g.part = part;
    if (dma) {
        if (big) launch_dma_big<2, 4, 4>(out_kind, blocks, s, g);
        else if (mid) launch_dma_mid(out_kind, ch, blocks, s, g);
        else if (narrow64) launch_dma_narrow64(out_kind, ch, blocks, s, g);
        else if (narrow) launch_dma_narrow(out_kind, ch, blocks, s, g);
        else if (small) launch_dma<64, 64, 2, 2, 3>(out_kind, ch, blocks, s, g);
        else launch_dma<128, 128, 2, 2, 3>(out_kind, ch, blocks, s, g);
    } else {
        if (big) launch_reg<256, 256>(vec, out_kind, ch, blocks, s, g);
        else launch_reg<128, 128>(vec, out_kind, ch, blocks, s, g);
    }
    ICX_LAUNCH_CHECK("gemm_i8_kernel");
    if (n_part && g.part) *n_part = (int)blocks;
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

// ---- icx_matmul_integer_noalloc: the workspace in a file-scope device array ---------------
// For callers that cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc).  The workspace of icx_matmul_integer (the packed weight and its
// column sums when B is not packed, row sums of A when a zero point needs them) lives in
// `scratch`, one copy per GPU, held until the process ends.  Every byte of it that a call
// reads is written earlier in the same call, so nothing needs clearing between calls; calls
// that overlap on one GPU (two streams, two host threads) share the array and race.
static __device__ __align__(256) char scratch[icx::kNoAllocScratchBytes];

namespace {
// Device address of `scratch` on each device (the array's name in host code is a host-side
// stand-in, never a device address).  Looked up once per device, with that device current.
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

int scratch_ptr(void** out) {
    int dev = 0;
    ICX_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) ICX_FAIL(ICX_ERR_UNSUPPORTED, "MatMulInteger (no-alloc): device index %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            ICX_FAIL(ICX_ERR_HIP, "MatMulInteger (no-alloc): hipGetSymbolAddress(scratch) failed: %s",
                     hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return ICX_OK;
}
}  // namespace

extern "C" size_t icx_matmul_integer_noalloc_max_bytes(void) { return icx::kNoAllocScratchBytes; }

extern "C" int icx_matmul_integer_noalloc(icx_stream_t stream, const void* A, int a_dtype,
                                          const void* B, int b_dtype, int b_packed,
                                          const int32_t* b_colsum, size_t M, size_t K, size_t N,
                                          const void* a_zp, const void* b_zp, size_t b_zp_len,
                                          const int32_t* a_rowsum, int32_t* C) {
    icx::clear_error();
    // the same workspace icx_matmul_integer would need, checked before any HIP call
    const size_t need = ws_layout(M, K, N, b_packed).total;
    if (need > icx::kNoAllocScratchBytes)
        ICX_FAIL(ICX_ERR_WORKSPACE,
                 "MatMulInteger (no-alloc): M=%zu K=%zu N=%zu (b_packed=%d) needs %zu bytes of workspace; the "
                 "static scratch holds %zu (pack the weight once with icx_pack_weight, or call icx_matmul_integer)",
                 M, K, N, b_packed, need, icx::kNoAllocScratchBytes);
    void* ws = nullptr;
    if (M && N) {
        const int rc = scratch_ptr(&ws);
        if (rc) return rc;
    }
    return gemm_common(reinterpret_cast<hipStream_t>(stream), A, a_dtype, B, b_dtype, b_packed, b_colsum, M, K, N,
                       a_zp, b_zp, b_zp_len, a_rowsum, nullptr, C, OUT_I32, ws, icx::kNoAllocScratchBytes,
                       "MatMulInteger (no-alloc)");
}

int icx::qlinear_f32(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype, int b_packed,
                     const int32_t* b_colsum, size_t M, size_t K, size_t N, const void* a_zp, const void* b_zp,
                     size_t b_zp_len, const int32_t* a_rowsum, const icx_chain* chain, float* Y, void* ws,
                     size_t ws_bytes, float2* part, int* n_part) {
    return gemm_common(s, A, a_dtype, B, b_dtype, b_packed, b_colsum, M, K, N, a_zp, b_zp, b_zp_len, a_rowsum,
                       chain, Y, OUT_F32, ws, ws_bytes, "QLinear", part, n_part);
}

// icx_debug_qout_fault: > 0 makes every quantized-output launch wait for a tag that no block
// publishes, giving up after that many polls (every block then exits through the failure
// path); 0 is normal operation.
static std::atomic<int> g_qout_fault_spin{0};

extern "C" void icx_debug_qout_fault(int spin) { g_qout_fault_spin.store(spin > 0 ? spin : 0); }

int icx::qout_fault_spin() { return g_qout_fault_spin.load(std::memory_order_relaxed); }

int icx::qlinear_dql(hipStream_t s, const void* A, int a_dtype, const int8_t* Bp, int b_dtype,
                     const int32_t* b_colsum, size_t M, size_t K, size_t N, const void* a_zp,
                     const icx_chain* chain, uint8_t* y, float* y_scale, uint8_t* y_zp, unsigned* sync) {
    if (!A || !Bp || !b_colsum || !y || !y_scale || !y_zp || !sync)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "QLinear+DQL: null pointer");
    if (!icx::is_int8_kind(a_dtype) || b_dtype != ICX_I8)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: needs an Int8 weight (dtypes %d, %d)", a_dtype, b_dtype);
    if (M == 0 || M > 0x7fffffff || K > 0x7fffffff || N > 0x7fffffff || K < 128 || K % 128 != 0 ||
        N % 192 != 0 || (uint64_t)M * K > 0xffffffffull || (uint64_t)N * K > 0xffffffffull ||
        !icx::aligned16(A) || !icx::aligned16(Bp) || !icx::aligned16(y))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: shape %zux%zux%zu or alignment outside the 256x192 kernel",
                 M, K, N);
    GemmArgs g{};
    if (chain) {
        int rc = icx::validate_chain(chain, "QLinear+DQL");
        if (rc) return rc;
        g.chain = *chain;
    } else {
        g.chain.n_ops = 0;
    }
    if (!icx::chain_is_col_only(g.chain))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: the epilogue has row or full-tensor operands");
    const unsigned blocks = (unsigned)(icx::cdiv(M, 256) * (N / 192));
    if (blocks > (unsigned)icx::kQoutMaxBlocks)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: %u tiles exceed %d", blocks, icx::kQoutMaxBlocks);
    g.A = reinterpret_cast<const int8_t*>(A);
    g.Bp = Bp;
    g.colsum = b_colsum;
    g.a_zp = a_zp;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.tiles_m = (int)icx::cdiv(M, 256);
    g.tiles_n = (int)(N / 192);
    g.a_xor = a_dtype == ICX_U8 ? 0x80808080u : 0u;
    g.alpha = a_dtype == ICX_U8 ? 128 : 0;
    g.beta = 0;
    g.a_zp_u8 = a_dtype == ICX_U8;
    g.b_zp_len = 1;
    g.codes = icx::chain_codes(g.chain);
    g.qy = y;
    g.q_scale = y_scale;
    g.q_zp = y_zp;
    g.q_sync = sync;
    g.q_wait = icx::wall_ticks(icx::kExchangeWaitUs);
    g.q_poison = 0;
    if (const int f = icx::qout_fault_spin()) {  // test hook
        g.q_wait = icx::wall_ticks((unsigned)f);
        g.q_poison = 0x80000000u;
    }
    if (icx::chain_mode(g.chain) == 2) {
        if (!icx::is_gelu8(g.codes, g.chain.n_ops))
            ICX_FAIL(ICX_ERR_UNSUPPORTED, "QLinear+DQL: an operand-free chain other than the erf-GELU");
        return launch_qout<CH_COL_EXT>(blocks, s, g);
    }
    return launch_qout<CH_COL>(blocks, s, g);
}

int icx::dql_qlinear(hipStream_t s, const float* x, size_t M, size_t K, uint8_t* y, float* y_scale,
                     uint8_t* y_zp, const int8_t* Bp, int b_dtype, const int32_t* b_colsum, size_t N,
                     const icx_chain* chain, float* Y, unsigned* sync) {
    if (!x || !y || !y_scale || !y_zp || !Bp || !b_colsum || !Y || !sync)
        ICX_FAIL(ICX_ERR_INVALID_ARG, "DQL+QLinear: null pointer");
    if (b_dtype != ICX_I8) ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: needs an Int8 weight (dtype %d)", b_dtype);
    if (M == 0 || M > 0x7fffffff || K > 0x7fffffff || N > 0x7fffffff || K < 128 || K % 128 != 0 ||
        N % 96 != 0 || (uint64_t)M * K > 0xffffffffull || (uint64_t)N * K > 0xffffffffull ||
        !icx::aligned16(x) || !icx::aligned16(y) || !icx::aligned16(Bp))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: shape %zux%zux%zu or alignment outside the kernels", M, K, N);
    // 256x192 tiles (12 waves) where their blocks' rows fit the registers (every block
    // quantizes q_rows rows of its row panel, QV float4 per lane), else 64x96 (6 waves; a
    // batch-1 activation, say)
    bool wide = N % 192 == 0 && icx::cdiv(256, N / 192) * K <= (size_t)QV * 4 * 768;
    if (wide && icx::cdiv(M, 256) * (N / 192) > (size_t)icx::num_cus()) wide = false;  // one block per CU
    const size_t BMv = wide ? 256 : 64, BNv = wide ? 192 : 96, NTv = wide ? 768 : 384;
    const size_t tiles_m = icx::cdiv(M, BMv), tiles_n = N / BNv;
    const size_t blocks = tiles_m * tiles_n;
    if (blocks > (size_t)icx::kQoutMaxBlocks)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: %zu tiles exceed %d", blocks, icx::kQoutMaxBlocks);
    const size_t q_rows = icx::cdiv(BMv, tiles_n);
    if (q_rows * K > (size_t)QV * 4 * NTv)
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: %zu rows of %zu per block exceed the registers", q_rows, K);
    GemmArgs g{};
    if (chain) {
        int rc = icx::validate_chain(chain, "DQL+QLinear");
        if (rc) return rc;
        g.chain = *chain;
    } else {
        g.chain.n_ops = 0;
    }
    if (!icx::chain_is_col_only(g.chain))
        ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: the epilogue has row or full-tensor operands");
    for (int k = 0; k < g.chain.n_ops; ++k) {  // the activation scale is computed in the launch
        const icx_chain_op& op = g.chain.ops[k];
        if ((op.p0 == y_scale && op.kind0 != ICX_BCAST_SCALAR) || (op.p1 == y_scale && op.kind1 != ICX_BCAST_SCALAR))
            ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: the DQL scale is read as a non-scalar operand");
    }
    g.A = reinterpret_cast<const int8_t*>(y);
    g.Bp = Bp;
    g.colsum = b_colsum;
    g.a_zp = y_zp;
    g.C = Y;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.tiles_m = (int)tiles_m;
    g.tiles_n = (int)tiles_n;
    g.a_xor = 0x80808080u;
    g.alpha = 128;
    g.beta = 0;
    g.a_zp_u8 = 1;
    g.b_zp_len = 1;
    g.codes = icx::chain_codes(g.chain);
    g.xin = x;
    g.q_rows = (int)q_rows;
    g.qy = y;
    g.q_scale = y_scale;
    g.q_zp = y_zp;
    g.q_sync = sync;
    g.q_wait = icx::wall_ticks(icx::kExchangeWaitUs);
    g.q_poison = 0;
    if (const int f = icx::qout_fault_spin()) {  // test hook
        g.q_wait = icx::wall_ticks((unsigned)f);
        g.q_poison = 0x80000000u;
    }
    if (icx::chain_mode(g.chain) == 2) {
        if (!icx::is_gelu8(g.codes, g.chain.n_ops))
            ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: an operand-free chain other than the erf-GELU");
        if (!wide) ICX_FAIL(ICX_ERR_UNSUPPORTED, "DQL+QLinear: the erf-GELU chain takes the 256x192 tiles only");
        return launch_qin<256, 192, 4, 3, CH_COL_EXT>((unsigned)blocks, s, g);
    }
    return wide ? launch_qin<256, 192, 4, 3, CH_COL>((unsigned)blocks, s, g)
                : launch_qin<64, 96, 2, 3, CH_COL>((unsigned)blocks, s, g);
}

extern "C" int icx_dql_qlinear_f32(icx_stream_t stream, const float* x, size_t M, size_t K, uint8_t* y,
                                   float* y_scale, uint8_t* y_zp, const void* B, int b_dtype,
                                   const int32_t* b_colsum, size_t N, const icx_chain* chain, float* Y,
                                   void* sync) {
    icx::clear_error();
    return icx::dql_qlinear(reinterpret_cast<hipStream_t>(stream), x, M, K, y, y_scale, y_zp,
                            reinterpret_cast<const int8_t*>(B), b_dtype, b_colsum, N, chain, Y,
                            static_cast<unsigned*>(sync));
}

int icx::qlinear_f32_seg(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype,
                         const int32_t* b_colsum, size_t M, size_t K, size_t N, const void* a_zp,
                         const void* b_zp, size_t b_zp_len, const int32_t* a_rowsum, const icx_chain* chain,
                         float* const* ys, int n_seg, void* ws, size_t ws_bytes) {
    return gemm_common(s, A, a_dtype, B, b_dtype, 1, b_colsum, M, K, N, a_zp, b_zp, b_zp_len, a_rowsum, chain,
                       nullptr, OUT_F32, ws, ws_bytes, "QLinear", nullptr, nullptr, ys, n_seg);
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
