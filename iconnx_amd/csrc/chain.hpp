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

// MODE 0: the four binary ops only (no extra registers, no erf code); MODE 2: also the
// operand-free steps (erf, save, multiply by the saved value).  The host picks the mode
// with chain_mode(), so kernels without a GELU-style chain do not pay for it.
template <int MODE, int NV, typename OpndFn>
__device__ __forceinline__ void run_chain4(uint32_t codes, int n_ops, float4 (&v)[NV],
                                           OpndFn opnd) {
    if constexpr (MODE == 2) {
        // The dequantized erf-GELU of an FFN projection — Mul, Add, Save, Mul (the Div by
        // sqrt(2) as the product with its reciprocal), Erf, Add, Mul by the saved value, Mul —
        // as straight-line code: the same operations in the same order as the loop below
        // (Add and Mul commute exactly, so the operand-side bit is ignored), without its per-op
        // dispatch and the register copies that dispatch costs (about 2 instructions per
        // element and op against 1).
        if (n_ops == 8 && (codes & 0x77777777u) == 0x26042502u) {
            const float4 o0 = opnd(0), o1 = opnd(1), o3 = opnd(3), o5 = opnd(5), o7 = opnd(7);
            auto gelu = [](float x, float a0, float a1, float a3, float a5, float a7) {
                x = __fadd_rn(__fmul_rn(x, a0), a1);
                const float z = x;
                x = __fadd_rn(erf_ref(__fmul_rn(x, a3)), a5);
                return __fmul_rn(__fmul_rn(z, x), a7);
            };
#pragma unroll
            for (int u = 0; u < NV; ++u) {
                v[u].x = gelu(v[u].x, o0.x, o1.x, o3.x, o5.x, o7.x);
                v[u].y = gelu(v[u].y, o0.y, o1.y, o3.y, o5.y, o7.y);
                v[u].z = gelu(v[u].z, o0.z, o1.z, o3.z, o5.z, o7.z);
                v[u].w = gelu(v[u].w, o0.w, o1.w, o3.w, o5.w, o7.w);
            }
            return;
        }
    }
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
