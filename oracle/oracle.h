/*
 * CPU oracle for the int8 dynamic-quantized linear path — TEST INFRASTRUCTURE ONLY.
 *
 * A single-threaded C restatement of the reference's CPU operators, used as the parity
 * checker for the HIP kernels and as the timed CPU baseline.  Only tests/, the
 * smoke() entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it;
 * the product library (iconnx_amd, libiconnx_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to the
 * ryanoneill/iconnx checkout).  Build: `make -C oracle` (gcc, -ffp-contract=off so each
 * f32/f64 operation rounds exactly once, as in the Rust source).
 */
#ifndef ICONNX_ORACLE_H
#define ICONNX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_ERR_OVERFLOW = 1, /* i32 overflow: the reference panics (checked_mul/checked_add) */
    ORC_ERR_ARG = 2,      /* shape / dtype / zero-point contract violated */
};

enum { ORC_DT_I8 = 0, ORC_DT_U8 = 1, ORC_DT_I32 = 2 };
enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3 };

/* DynamicQuantizeLinear (src/operators/dynamic_quantize_linear.rs:32-112).
 * Writes y[n], the f32 scale and the u8 zero point.  `scale64` (nullable) receives the
 * f64 scale the per-element quantize divides by (0.0 for the constant-input sentinel). */
void orc_dql_u8(const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                double* scale64);

/* MatMulInteger (src/operators/matmul_integer.rs:52-267), rows [row_begin, row_end) of
 * out[M,N] = sum_k (a[m,k]-a_zp) * (b[k,n]-b_zp).  a/b are i8 or u8 (a_dt/b_dt).
 * b_zp_len == 1 is the reference's scalar zero point; b_zp_len == N is the ONNX per-column
 * form the reference rejects (matmul_integer.rs:206-213) — an extension, pinned only by the
 * ONNX definition.  Returns ORC_ERR_OVERFLOW where the reference would panic. */
int orc_matmul_integer_rows(const void* a, int a_dt, const void* b, int b_dt, size_t M,
                            size_t K, size_t N, int32_t a_zp, const int32_t* b_zp,
                            size_t b_zp_len, size_t row_begin, size_t row_end, int32_t* out);

/* Cast INT32 -> FLOAT (src/operators/cast.rs:46-49): `x as f32`, round to nearest even. */
void orc_cast_i32_f32(const int32_t* x, size_t n, float* y);

/* Broadcasting f32 binary op (Add src/operators/add.rs:27-86, Sub, Mul
 * src/operators/mul.rs:26-58, Div src/operators/div.rs:21-77): numpy/ndarray broadcasting,
 * one IEEE-754 single rounding per element.  Ranks <= 8.  out_shape/out_rank receive the
 * broadcast shape.  Returns ORC_ERR_ARG when the shapes do not broadcast. */
int orc_binary_f32(int op, const float* a, const size_t* a_shape, int a_rank, const float* b,
                   const size_t* b_shape, int b_rank, float* out, size_t* out_shape,
                   int* out_rank);

/* DequantizeLinear (src/operators/dequantize_linear.rs:32-180): y = (x as f32 - zp as f32)
 * * scale, per element; the axis coordinate of flat index i is (i / inner) % axis_size
 * (axis_size = 1 for per-tensor).  zp may be NULL (zero). */
void orc_dequantize_linear(const void* x, int x_dt, const float* scale, const void* zp,
                           size_t n, size_t axis_size, size_t inner, float* y);

/* ---- encoder ops (fp32) -------------------------------------------------------------- */

/* Sum of a contiguous f32 slice in the order of ndarray 0.16's `numeric_util::unrolled_fold`
 * (the reference's `sum_axis` / `mean_axis` over a contiguous last axis, Cargo.toml:21):
 * eight partial sums p_j over x[j], x[j+8], ... then acc = 0 + (p0+p4), + (p1+p5),
 * + (p2+p6), + (p3+p7), then the < 8 leftover elements in order. */
float orc_sum_unrolled8(const float* x, size_t n);

/* LayerNormalization over the last axis (src/operators/layer_normalization.rs:25-80):
 * mean = sum/n; c = x - mean; var = sum(c*c)/n; std = sqrt(var + eps);
 * y = (c / std) * scale + bias, every step one f32 rounding.  x, y: [rows, cols]. */
void orc_layer_norm(const float* x, size_t rows, size_t cols, const float* scale,
                    const float* bias, float eps, float* y);

/* Softmax over the last axis (src/operators/softmax.rs:25-40): m = max (NaN-ignoring fold
 * from -inf), e = exp(x - m) (libm expf, as Rust's f32::exp), y = e / sum(e). */
void orc_softmax_last(const float* x, size_t rows, size_t cols, float* y);

/* Erf (src/operators/erf.rs:21-31): Abramowitz-Stegun 7.1.26 in f32 with libm expf. */
void orc_erf(const float* x, size_t n, float* y);

/* Batched f32 MatMul (src/operators/matmul.rs:20-150): c[b] = a[b] @ b[b or 0], a [M,K],
 * b [K,N].  Accumulated in f64 and rounded once: the reference's sgemm summation order
 * (matrixmultiply crate microkernels) is not restated, so parity with it is by tolerance. */
void orc_matmul_f32(const float* a, const float* b, size_t batch, int b_broadcast, size_t M,
                    size_t K, size_t N, float* c);

/* ReduceMean (src/operators/reduce_mean.rs:19-105) of x viewed as [outer, axis_len, inner]
 * over its middle axis: y[outer, inner] = sum / (axis_len as f32).  ndarray 0.16's
 * sum_axis: the least-strided axis (the last one of a standard-layout array, or all of x as
 * one slice for data.mean()) lane by lane with unrolled_fold (sequential == 0, inner must be
 * 1); any other axis as res = 0 + x[.., 0, ..] + x[.., 1, ..] + ... (sequential != 0). */
void orc_reduce_mean(const float* x, size_t outer, size_t axis_len, size_t inner,
                     int sequential, float* y);

/* Pow (src/operators/pow.rs:18-45): y[i] = powf(x[i], e[i]) — Rust's f32::powf is the C
 * library's powf (glibc on Linux); e already broadcast to x's shape by the caller. */
void orc_pow_f32(const float* x, const float* e, size_t n, float* y);

/* Sqrt (src/operators/sqrt.rs:18-30): y = sqrtf(x) (f32::sqrt, correctly rounded). */
void orc_sqrt_f32(const float* x, size_t n, float* y);

/* Transpose (src/operators/transpose.rs:10-40): y = x.permuted_axes(perm) in standard
 * layout; elem bytes 1, 4 or 8; rank <= 8. */
void orc_transpose(const void* x, size_t elem, int rank, const size_t* dims, const int* perm,
                   void* y);

#ifdef __cplusplus
}
#endif
#endif
