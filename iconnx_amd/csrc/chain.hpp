// Device-side evaluation of an icx_chain: ordered f32 binary ops, one IEEE-754 single
// rounding each (explicit *_rn intrinsics, and the library is built with
// -ffp-contract=off), matching separate ONNX Mul / Add / Sub / Div nodes evaluated one at a
// time (src/operators/{mul,add,div}.rs).
#pragma once

#include "icx_common.hpp"

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

__device__ __forceinline__ float chain_operand(const icx_chain_op& op, size_t r, size_t c,
                                               size_t cols) {
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

__device__ __forceinline__ float apply_chain(const icx_chain& ch, float v, size_t r, size_t c,
                                             size_t cols) {
    for (int i = 0; i < ch.n_ops; ++i) {
        const icx_chain_op& op = ch.ops[i];
        const float o = chain_operand(op, r, c, cols);
        v = op.operand_is_lhs ? apply_binary(op.op, o, v) : apply_binary(op.op, v, o);
    }
    return v;
}

// Host-side validation shared by every entry point taking a chain.
int validate_chain(const icx_chain* ch, const char* who);

}  // namespace icx
