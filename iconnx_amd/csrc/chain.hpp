// Device-side evaluation of an icx_chain: ordered f32 binary ops, one IEEE-754 single
// rounding each (explicit *_rn intrinsics, and the library is built with
// -ffp-contract=off), matching separate ONNX Mul / Add / Sub / Div nodes evaluated one at a
// time (src/operators/{mul,add,div}.rs).
//
// Two evaluation forms:
//  * apply_chain      — general: every operand fetched per element (any broadcast kind);
//  * load_col_operands + run_chain4 (op-major, over chain_codes) — when every factor is a
//    scalar or a [cols] vector (the dequant-scale / bias / per-channel chain case): the
//    operands of one column are fetched once and the per-element work is pure arithmetic.
#pragma once

#include "icx_common.hpp"

#include <cstdint>

namespace icx {

__device__ __forceinline__ float load_bcast(const float* p, int kind, size_t r, size_t c,
                                            size_t cols) {
    switch (kind) {
        case ICX_BCAST_SCALAR: return p[0];
        case ICX_BCAST_COL: return p[c];
        case ICX_BCAST_ROW: return p[r];
        default: return p[r * cols + c];
    }
}

__device__ __forceinline__ bool op_takes_operand(int op) { return op <= ICX_OP_DIV; }

// erf as the reference evaluates it (src/operators/erf.rs:21-31): Abramowitz-Stegun 7.1.26
// in f32, one rounding per polynomial operation.  t = 1/d (d >= 1) is the hardware
// reciprocal refined by one Newton step (two FMAs; the correctly rounded quotient except in
// rare last-bit cases) and exp(-a^2) the hardware exp2 of -a^2 * log2(e), whose relative
// error (~|a^2| * 2^-24) multiplies a term that is below e^-a^2: both stay far below the
// formula's own 1.5e-7 error, at a handful of instructions instead of a correctly rounded
// division and a library expf (the GELU epilogue of the FFN-up projection runs this for
// every output element).
__device__ __forceinline__ float erf_ref(float x) {
    // x.signum() for every non-NaN x (+-1, also for +-0); NaN is returned as is below
    const float sign = copysignf(1.0f, x);
    // |x| >= 10 gives exactly +-1 either way (e^-100 is 0 in f32); the clamp keeps the
    // Newton step finite for |x| = inf.
    const float a = fminf(fabsf(x), 16.0f);
    const float d = __fadd_rn(1.0f, __fmul_rn(0.3275911f, a));
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float t = __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
    float p = __fsub_rn(__fmul_rn(1.0614054f, t), 1.4531521f);
    p = __fadd_rn(__fmul_rn(p, t), 1.4214138f);
    p = __fsub_rn(__fmul_rn(p, t), 0.28449672f);
    p = __fadd_rn(__fmul_rn(p, t), 0.2548296f);
    const float e = __expf(__fmul_rn(-a, a));
    const float y = __fsub_rn(1.0f, __fmul_rn(__fmul_rn(p, t), e));
    return (x != x) ? x : __fmul_rn(sign, y);
}

// erf inside the erf-GELU x * (1 + erf(x / sqrt(2))) / 2 of a GEMM epilogue, of an argument
// given pre-scaled as w = u * sqrt(log2 e) (the column factor 1/sqrt(2) times sqrt(log2 e),
// formed once per operand): the same Abramowitz-Stegun 7.1.26 formula with d = 1 +
// (0.3275911 / sqrt(log2 e)) |w|, the polynomial as four FMAs, t = 1/d the hardware
// reciprocal alone (<= 1 ulp), e^(-u^2) = 2^(-w^2) and 1 - p t e as one FMA; NaN and +-inf
// need no special case (NaN propagates through every step; |w| = inf gives t = 0, e = 0,
// y = +-1).  About 11 instructions per element against erf_ref's 26.  It is within 1e-6 of
// erf_ref — the largest differences lie at |u| < 0.06, from the reciprocal's last bit — and
// there the GELU multiplies erf by x itself: with the rest of the GELU as in the chain, its
// output stays within 4e-7 of the op-by-op reference relative to its largest value, as
// close as with erf_ref (modelled on the CPU with the reciprocal and the exponential off by
// one ulp either way).
constexpr float kSqrtLog2e = 1.20112240878f;       // sqrt(log2 e)
constexpr float kErfP = 0.27273747f;               // 0.3275911 / sqrt(log2 e)
__device__ __forceinline__ float erf_gelu_scaled(float w) {
    const float b = fabsf(w);
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(kErfP, b, 1.0f));
    float p = __builtin_fmaf(1.0614054f, t, -1.4531521f);
    p = __builtin_fmaf(p, t, 1.4214138f);
    p = __builtin_fmaf(p, t, -0.28449672f);
    p = __builtin_fmaf(p, t, 0.2548296f);
    const float e = __builtin_amdgcn_exp2f(__fmul_rn(-b, b));
    return copysignf(__builtin_fmaf(-__fmul_rn(p, t), e, 1.0f), w);
}

__device__ __forceinline__ float chain_operand(const icx_chain_op& op, size_t r, size_t c,
                                               size_t cols) {
    if (!op_takes_operand(op.op)) return 0.0f;
    float a = load_bcast(op.p0, op.kind0, r, c, cols);
    if (op.p1) a = __fmul_rn(a, load_bcast(op.p1, op.kind1, r, c, cols));
    return a;
}

__device__ __forceinline__ float apply_binary(int op, float lhs, float rhs) {
    switch (op) {
        case ICX_OP_ADD: return __fadd_rn(lhs, rhs);
        case ICX_OP_SUB: return __fsub_rn(lhs, rhs);
        case ICX_OP_MUL: return __fmul_rn(lhs, rhs);
        default: return __fdiv_rn(lhs, rhs);
    }
}

__device__ __forceinline__ float apply_one(const icx_chain_op& op, float v, float o) {
    return op.operand_is_lhs ? apply_binary(op.op, o, v) : apply_binary(op.op, v, o);
}

// One step including the operand-free ones; `s` is the saved value.
__device__ __forceinline__ float step_one(const icx_chain_op& op, float v, float o, float& s) {
    switch (op.op) {
        case ICX_OP_ERF: return erf_ref(v);
        case ICX_OP_SAVE: s = v; return v;
        case ICX_OP_MUL_SAVED: return __fmul_rn(s, v);
        default: return apply_one(op, v, o);
    }
}

__device__ __forceinline__ float apply_chain(const icx_chain& ch, float v, size_t r, size_t c,
                                             size_t cols) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < ICX_MAX_CHAIN; ++i)
        if (i < ch.n_ops) v = step_one(ch.ops[i], v, chain_operand(ch.ops[i], r, c, cols), s);
    return v;
}

// Column-only chains: operands of column c (scalar or [cols] factors).
__device__ __forceinline__ float col_factor(const float* p, int kind, size_t c) {
    return kind == ICX_BCAST_SCALAR ? p[0] : p[c];
}

// x / d whose only reader is the next step's Erf (the erf-GELU's x / sqrt(2)).  The op-major
// evaluators (run_chain4 over chain_codes) run it as x * RN(1/d): the quotient then differs
// from the IEEE one by at most one ulp, which moves erf by at most max|erf'(t) t| * 2^-23
// < 4e-8 — inside erf's own tolerance — and saves a correctly rounded division per element.
// The per-element evaluator (apply_chain) keeps the division.
__host__ __device__ inline bool div_feeds_erf(const icx_chain& ch, int k) {
    return k + 1 < ch.n_ops && ch.ops[k].op == ICX_OP_DIV && !ch.ops[k].operand_is_lhs &&
           ch.ops[k + 1].op == ICX_OP_ERF;
}

// Operand of step k at column c as the op-major evaluators consume it: the factor product,
// or its correctly rounded reciprocal for a division that feeds an Erf (see above).
__device__ __forceinline__ float col_operand(const icx_chain& ch, int k, size_t c) {
    const icx_chain_op& op = ch.ops[k];
    float a = col_factor(op.p0, op.kind0, c);
    if (op.p1) a = __fmul_rn(a, col_factor(op.p1, op.kind1, c));
    return div_feeds_erf(ch, k) ? __fdiv_rn(1.0f, a) : a;
}

// The operands of column c for the op-major evaluators (run_chain4 with chain_codes).
__device__ __forceinline__ void load_col_operands(const icx_chain& ch, size_t c,
                                                  float (&o)[ICX_MAX_CHAIN]) {
#pragma unroll
    for (int i = 0; i < ICX_MAX_CHAIN; ++i)
        o[i] = (i < ch.n_ops && op_takes_operand(ch.ops[i].op)) ? col_operand(ch, i, c) : 0.0f;
}


// ---- op-major evaluation over a register block of float4 values ------------------------
// The op codes of a chain packed 4 bits per op: bits [2:0] = ICX_OP_*, bit 3 = operand on
// the left.  One uniform switch per op, then straight-line IEEE ops over every value the
// lane holds — no per-element branching.  `opnd(k)` returns the float4 operand of op k for
// the lane's 4 columns (unused by the operand-free ops).
// A division that feeds an Erf is coded as a multiplication: its staged operand is the
// reciprocal (col_operand).
__host__ __device__ inline uint32_t chain_codes(const icx_chain& ch) {
    uint32_t c = 0;
    for (int i = 0; i < ch.n_ops; ++i) {
        const int op = div_feeds_erf(ch, i) ? ICX_OP_MUL : ch.ops[i].op;
        c |= (uint32_t)((op & 7) | (ch.ops[i].operand_is_lhs ? 8 : 0)) << (4 * i);
    }
    return c;
}

// 0 when every step is a binary op, 2 when an operand-free step (erf / save) occurs.
inline int chain_mode(const icx_chain& ch) {
    for (int i = 0; i < ch.n_ops; ++i)
        if (ch.ops[i].op > ICX_OP_DIV) return 2;
    return 0;
}

#define ICX_EW4(expr)                                   \
    _Pragma("unroll") for (int u = 0; u < NV; ++u) {    \
        { float& x = v[u].x; const float y = o.x; x = (expr); } \
        { float& x = v[u].y; const float y = o.y; x = (expr); } \
        { float& x = v[u].z; const float y = o.z; x = (expr); } \
        { float& x = v[u].w; const float y = o.w; x = (expr); } \
    }

// Operand-free steps over the whole block; `sv` holds the saved values.
#define ICX_EW4S(stmt)                                                  \
    _Pragma("unroll") for (int u = 0; u < NV; ++u) {                    \
        { float& x = v[u].x; float& z = sv[u].x; stmt; }                \
        { float& x = v[u].y; float& z = sv[u].y; stmt; }                \
        { float& x = v[u].z; float& z = sv[u].z; stmt; }                \
        { float& x = v[u].w; float& z = sv[u].w; stmt; }                \
    }

// The op codes of the dequantized erf-GELU of an FFN projection (Mul, Add, Save, Mul, Erf,
// Add, MulSaved, Mul; the operand-side bits ignored) — run as straight-line code below.
__host__ __device__ inline bool is_gelu8(uint32_t codes, int n_ops) {
    return n_ops == 8 && (codes & 0x77777777u) == 0x26042502u;
}

// MODE 0: the four binary ops only (no extra registers, no erf code); MODE 2: also the
// operand-free steps (erf, save, multiply by the saved value); MODE 3: only the straight-line
// erf-GELU (is_gelu8 must hold; for a kernel whose register budget has no room for the
// per-op loop's saved values).  The host picks the mode with chain_mode(), so kernels
// without a GELU-style chain do not pay for it.
template <int MODE, int NV, typename OpndFn>
__device__ __forceinline__ void run_chain4(uint32_t codes, int n_ops, float4 (&v)[NV],
                                           OpndFn opnd) {
    if constexpr (MODE >= 2) {
        // The dequantized erf-GELU of an FFN projection — Mul, Add, Save, Mul (the Div by
        // sqrt(2) as the product with its reciprocal), Erf, Add, Mul by the saved value, Mul —
        // as straight-line code, without the loop's per-op dispatch and the register copies
        // that dispatch costs: the dequant Mul and bias Add as in the loop (one rounding each),
        // then erf_gelu_scaled of x * (c3 sqrt(log2 e)) and x * (erf * c7 + c5 c7) — the
        // last three ops as one FMA and a product — with the two column factors formed once
        // per operand.
        if (MODE == 3 || is_gelu8(codes, n_ops)) {
            const float4 o0 = opnd(0), o1 = opnd(1), o3 = opnd(3), o5 = opnd(5), o7 = opnd(7);
            const float4 w3 = make_float4(__fmul_rn(o3.x, kSqrtLog2e), __fmul_rn(o3.y, kSqrtLog2e),
                                          __fmul_rn(o3.z, kSqrtLog2e), __fmul_rn(o3.w, kSqrtLog2e));
            const float4 h57 = make_float4(__fmul_rn(o5.x, o7.x), __fmul_rn(o5.y, o7.y), __fmul_rn(o5.z, o7.z),
                                           __fmul_rn(o5.w, o7.w));
            auto gelu = [](float x, float a0, float a1, float c3, float c7, float c57) {
                x = __fadd_rn(__fmul_rn(x, a0), a1);
                return __fmul_rn(x, __builtin_fmaf(erf_gelu_scaled(__fmul_rn(x, c3)), c7, c57));
            };
#pragma unroll
            for (int u = 0; u < NV; ++u) {
                v[u].x = gelu(v[u].x, o0.x, o1.x, w3.x, o7.x, h57.x);
                v[u].y = gelu(v[u].y, o0.y, o1.y, w3.y, o7.y, h57.y);
                v[u].z = gelu(v[u].z, o0.z, o1.z, w3.z, o7.z, h57.z);
                v[u].w = gelu(v[u].w, o0.w, o1.w, w3.w, o7.w, h57.w);
            }
            return;
        }
    }
    if constexpr (MODE == 3) return;
    // The dequant (Mul) and bias (Add) that head every quantized linear's chain, straight-line
    // for the same reason; the ops after them, if any, go through the loop.  Binary-only
    // chains (MODE 0) only: in the GELU kernels the extra code costs registers.
    int k0 = 0;
    if (MODE != 0) {
    } else if (n_ops >= 2 && (codes & 0x77u) == 0x02u) {
        const float4 o0 = opnd(0), o1 = opnd(1);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            v[u].x = __fadd_rn(__fmul_rn(v[u].x, o0.x), o1.x);
            v[u].y = __fadd_rn(__fmul_rn(v[u].y, o0.y), o1.y);
            v[u].z = __fadd_rn(__fmul_rn(v[u].z, o0.z), o1.z);
            v[u].w = __fadd_rn(__fmul_rn(v[u].w, o0.w), o1.w);
        }
        if (n_ops == 2) return;
        k0 = 2;
    } else if (n_ops == 1 && (codes & 7u) == ICX_OP_MUL) {  // the dequant alone
        const float4 o0 = opnd(0);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            v[u].x = __fmul_rn(v[u].x, o0.x);
            v[u].y = __fmul_rn(v[u].y, o0.y);
            v[u].z = __fmul_rn(v[u].z, o0.z);
            v[u].w = __fmul_rn(v[u].w, o0.w);
        }
        return;
    }
    float4 sv[MODE == 2 ? NV : 1];
#pragma unroll 1
    for (int k = k0; k < n_ops; ++k) {
        const uint32_t code = (codes >> (4 * k)) & 15u;
        if constexpr (MODE == 2) {
            if ((code & 7u) > ICX_OP_DIV) {
                switch (code & 7u) {
                    case ICX_OP_SAVE: ICX_EW4S(z = x) break;
                    case ICX_OP_MUL_SAVED: ICX_EW4S(x = __fmul_rn(z, x)) break;
                    default: ICX_EW4S(x = erf_ref(x)) break;
                }
                continue;
            }
        }
        const float4 o = opnd(k);
        switch (code) {
            case ICX_OP_ADD: ICX_EW4(__fadd_rn(x, y)) break;
            case ICX_OP_ADD | 8: ICX_EW4(__fadd_rn(y, x)) break;
            case ICX_OP_SUB: ICX_EW4(__fsub_rn(x, y)) break;
            case ICX_OP_SUB | 8: ICX_EW4(__fsub_rn(y, x)) break;
            case ICX_OP_MUL: ICX_EW4(__fmul_rn(x, y)) break;
            case ICX_OP_MUL | 8: ICX_EW4(__fmul_rn(y, x)) break;
            case ICX_OP_DIV: ICX_EW4(__fdiv_rn(x, y)) break;
            default: ICX_EW4(__fdiv_rn(y, x)) break;
        }
    }
}
#undef ICX_EW4
#undef ICX_EW4S

// Host side: true when every operand factor is a scalar or a [cols] vector.
inline bool chain_is_col_only(const icx_chain& ch) {
    for (int i = 0; i < ch.n_ops; ++i) {
        const icx_chain_op& o = ch.ops[i];
        if (o.op > ICX_OP_DIV) continue;
        if (o.kind0 != ICX_BCAST_SCALAR && o.kind0 != ICX_BCAST_COL) return false;
        if (o.p1 && o.kind1 != ICX_BCAST_SCALAR && o.kind1 != ICX_BCAST_COL) return false;
    }
    return true;
}

// Host-side validation shared by every entry point taking a chain.
int validate_chain(const icx_chain* ch, const char* who);

}  // namespace icx
