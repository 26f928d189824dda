/*
 * CPU oracle for the int8 dynamic-quantized linear path — TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract.  Compiled with -ffp-contract=off: every float/double
 * expression below rounds once per operation, as the Rust source does.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Rust `f64::clamp(qmin, qmax) as u8`: clamp keeps NaN, the saturating cast maps NaN to 0
 * (dynamic_quantize_linear.rs:91, :101). */
static uint8_t clamp_to_u8(double q) {
    if (isnan(q)) return 0;
    if (q < 0.0) q = 0.0;
    if (q > 255.0) q = 255.0;
    return (uint8_t)q;
}

/* f64::round_ties_even: IEEE roundTiesToEven, the default rounding mode of nearbyint. */
static double round_ties_even(double v) { return nearbyint(v); }

void orc_dql_u8(const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                double* scale64) {
    /* dynamic_quantize_linear.rs:56-69 — range starts at 0.0 (so zero is representable),
     * accumulated in f64, NaN skipped. */
    double min_x = 0.0, max_x = 0.0;
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        if (isnan(v)) continue;
        double vd = (double)v;
        if (vd < min_x) min_x = vd;
        if (vd > max_x) max_x = vd;
    }
    const double qmin = 0.0, qmax = 255.0;
    /* :75-84 — constant tensor: scale 0, zero point 0, all y = 0. */
    if (min_x == max_x) {
        memset(y, 0, n);
        *y_scale = 0.0f;
        *y_zp = 0;
        if (scale64) *scale64 = 0.0;
        return;
    }
    /* :89-92 */
    double s = (max_x - min_x) / (qmax - qmin);
    double izp = round_ties_even(qmin - min_x / s);
    uint8_t zp = clamp_to_u8(izp);
    *y_scale = (float)s;
    *y_zp = zp;
    if (scale64) *scale64 = s;
    /* :97-103 — per element, in f64 against the f64 scale. */
    for (size_t i = 0; i < n; ++i) {
        double q = round_ties_even((double)x[i] / s) + (double)zp;
        y[i] = clamp_to_u8(q);
    }
}

static int32_t load_operand(const void* p, int dt, size_t i) {
    return dt == ORC_DT_U8 ? (int32_t)((const uint8_t*)p)[i] : (int32_t)((const int8_t*)p)[i];
}

int orc_matmul_integer_rows(const void* a, int a_dt, const void* b, int b_dt, size_t M,
                            size_t K, size_t N, int32_t a_zp, const int32_t* b_zp,
                            size_t b_zp_len, size_t row_begin, size_t row_end, int32_t* out) {
    if ((a_dt != ORC_DT_I8 && a_dt != ORC_DT_U8) || (b_dt != ORC_DT_I8 && b_dt != ORC_DT_U8))
        return ORC_ERR_ARG;
    if (b_zp_len != 1 && b_zp_len != N) return ORC_ERR_ARG;
    if (row_end > M || row_begin > row_end) return ORC_ERR_ARG;
    /* gemm_i32_into (matmul_integer.rs:239-267): naive row, col, k loop with B read
     * column-strided, operands promoted to i32, checked multiply and add. */
    for (size_t row = row_begin; row < row_end; ++row) {
        for (size_t col = 0; col < N; ++col) {
            const int32_t bz = b_zp[b_zp_len == 1 ? 0 : col];
            int32_t acc = 0;
            for (size_t kk = 0; kk < K; ++kk) {
                int32_t av = load_operand(a, a_dt, row * K + kk) - a_zp;
                int32_t bv = load_operand(b, b_dt, kk * N + col) - bz;
                int32_t prod;
                if (__builtin_mul_overflow(av, bv, &prod)) return ORC_ERR_OVERFLOW;
                if (__builtin_add_overflow(acc, prod, &acc)) return ORC_ERR_OVERFLOW;
            }
            out[row * N + col] = acc;
        }
    }
    return ORC_OK;
}

void orc_cast_i32_f32(const int32_t* x, size_t n, float* y) {
    /* cast.rs:46-49 */
    for (size_t i = 0; i < n; ++i) y[i] = (float)x[i];
}

int orc_binary_f32(int op, const float* a, const size_t* a_shape, int a_rank, const float* b,
                   const size_t* b_shape, int b_rank, float* out, size_t* out_shape,
                   int* out_rank) {
    enum { MAXR = 8 };
    if (a_rank > MAXR || b_rank > MAXR || a_rank < 0 || b_rank < 0) return ORC_ERR_ARG;
    if (op < ORC_ADD || op > ORC_DIV) return ORC_ERR_ARG;
    int r = a_rank > b_rank ? a_rank : b_rank;
    size_t ad[MAXR], bd[MAXR], od[MAXR];
    /* right-align both shapes (add.rs:248-257, div.rs:326-335) */
    for (int i = 0; i < r; ++i) {
        int ia = i - (r - a_rank), ib = i - (r - b_rank);
        ad[i] = ia >= 0 ? a_shape[ia] : 1;
        bd[i] = ib >= 0 ? b_shape[ib] : 1;
        if (ad[i] == bd[i] || bd[i] == 1) od[i] = ad[i];
        else if (ad[i] == 1) od[i] = bd[i];
        else return ORC_ERR_ARG; /* ndarray's broadcast() returns None -> the reference panics */
    }
    size_t as[MAXR], bs[MAXR], total = 1;
    size_t sa = 1, sb = 1;
    for (int i = r - 1; i >= 0; --i) {
        as[i] = ad[i] == 1 ? 0 : sa;
        bs[i] = bd[i] == 1 ? 0 : sb;
        sa *= ad[i];
        sb *= bd[i];
        total *= od[i];
    }
    size_t idx[MAXR];
    memset(idx, 0, sizeof(idx));
    for (size_t flat = 0; flat < total; ++flat) {
        size_t oa = 0, ob = 0;
        for (int i = 0; i < r; ++i) {
            oa += idx[i] * as[i];
            ob += idx[i] * bs[i];
        }
        float x = a[oa], yv = b[ob], z;
        switch (op) {
            case ORC_ADD: z = x + yv; break;
            case ORC_SUB: z = x - yv; break;
            case ORC_MUL: z = x * yv; break;
            default: z = x / yv; break; /* IEEE division (div.rs:345-346) */
        }
        out[flat] = z;
        for (int i = r - 1; i >= 0; --i) {
            if (++idx[i] < od[i]) break;
            idx[i] = 0;
        }
    }
    for (int i = 0; i < r; ++i) out_shape[i] = od[i];
    *out_rank = r;
    return ORC_OK;
}

static float load_as_f32(const void* p, int dt, size_t i) {
    switch (dt) {
        case ORC_DT_I8: return (float)((const int8_t*)p)[i];
        case ORC_DT_U8: return (float)((const uint8_t*)p)[i];
        default: return (float)((const int32_t*)p)[i];
    }
}

void orc_dequantize_linear(const void* x, int x_dt, const float* scale, const void* zp,
                           size_t n, size_t axis_size, size_t inner, float* y) {
    /* dequantize_linear.rs:90-95 (scale per element), :99-155 (zp per element, as f32),
     * :158-174 ((x as f32 - zp as f32) * scale), :185-214 (axis broadcast). */
    for (size_t i = 0; i < n; ++i) {
        size_t ax = axis_size == 1 ? 0 : (i / inner) % axis_size;
        float xi = load_as_f32(x, x_dt, i);
        float zpi = zp ? load_as_f32(zp, x_dt, ax) : 0.0f;
        y[i] = (xi - zpi) * scale[ax];
    }
}

/* ---- encoder ops ----------------------------------------------------------------------- */

float orc_sum_unrolled8(const float* x, size_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) p[j] = p[j] + x[i + j];
    float acc = 0.0f;
    acc = acc + (p[0] + p[4]);
    acc = acc + (p[1] + p[5]);
    acc = acc + (p[2] + p[6]);
    acc = acc + (p[3] + p[7]);
    for (; i < n; ++i) acc = acc + x[i];
    return acc;
}

void orc_layer_norm(const float* x, size_t rows, size_t cols, const float* scale,
                    const float* bias, float eps, float* y) {
    /* layer_normalization.rs:45-77; mean_axis = sum_axis / n with n as f32 */
    float* c = (float*)malloc(cols * sizeof(float));
    float* sq = (float*)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        const float mean = orc_sum_unrolled8(xr, cols) / (float)cols;
        for (size_t j = 0; j < cols; ++j) {
            c[j] = xr[j] - mean;
            sq[j] = c[j] * c[j];
        }
        const float var = orc_sum_unrolled8(sq, cols) / (float)cols;
        const float sd = sqrtf(var + eps);
        for (size_t j = 0; j < cols; ++j) {
            const float nrm = c[j] / sd;
            y[r * cols + j] = nrm * scale[j] + bias[j];
        }
    }
    free(c);
    free(sq);
}

void orc_softmax_last(const float* x, size_t rows, size_t cols, float* y) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        float m = -INFINITY;
        for (size_t j = 0; j < cols; ++j) m = fmaxf(m, xr[j]); /* f32::max ignores NaN */
        for (size_t j = 0; j < cols; ++j) yr[j] = expf(xr[j] - m);
        const float s = orc_sum_unrolled8(yr, cols);
        for (size_t j = 0; j < cols; ++j) yr[j] = yr[j] / s;
    }
}

void orc_reduce_mean(const float* x, size_t outer, size_t axis_len, size_t inner,
                     int sequential, float* y) {
    /* reduce_mean.rs:64-72: data.mean() = sum() / n, data.mean_axis(Axis(a)) = sum_axis / n,
     * n converted by A::from_usize (one rounding above 2^24); ndarray 0.16 sum_axis walks the
     * min-stride axis lane by lane with unrolled_fold, any other by adding sub-views into a
     * zero array in axis order. */
    const float fn = (float)axis_len;
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < inner; ++i) {
            float acc;
            if (!sequential) {
                acc = orc_sum_unrolled8(x + o * axis_len, axis_len);
            } else {
                acc = 0.0f;
                for (size_t a = 0; a < axis_len; ++a) acc = acc + x[(o * axis_len + a) * inner + i];
            }
            y[o * inner + i] = acc / fn;
        }
}

void orc_pow_f32(const float* x, const float* e, size_t n, float* y) {
    /* pow.rs:27-35: b.powf(e) per element of the broadcast exponent */
    for (size_t i = 0; i < n; ++i) y[i] = powf(x[i], e[i]);
}

void orc_sqrt_f32(const float* x, size_t n, float* y) {
    /* sqrt.rs:26-29: x.sqrt() */
    for (size_t i = 0; i < n; ++i) y[i] = sqrtf(x[i]);
}

static float erf1(float x) {
    /* erf.rs:21-31: sign * (1 - poly(t) * t * exp(-a*a)), t = 1 / (1 + 0.3275911 a) */
    const float sign = isnan(x) ? x : (x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : copysignf(1.0f, x)));
    const float a = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float poly = ((((1.0614054f * t - 1.4531521f) * t) + 1.4214138f) * t - 0.28449672f) * t
                       + 0.2548296f;
    const float y = 1.0f - poly * t * expf(-a * a);
    return sign * y;
}

void orc_erf(const float* x, size_t n, float* y) {
    for (size_t i = 0; i < n; ++i) y[i] = erf1(x[i]);
}

void orc_matmul_f32(const float* a, const float* b, size_t batch, int b_broadcast, size_t M,
                    size_t K, size_t N, float* c) {
    for (size_t bi = 0; bi < batch; ++bi) {
        const float* ab = a + bi * M * K;
        const float* bb = b + (b_broadcast ? 0 : bi * K * N);
        float* cb = c + bi * M * N;
        for (size_t m = 0; m < M; ++m)
            for (size_t n = 0; n < N; ++n) {
                double s = 0.0;
                for (size_t k = 0; k < K; ++k) s += (double)ab[m * K + k] * (double)bb[k * N + n];
                cb[m * N + n] = (float)s;
            }
    }
}

void orc_transpose(const void* x, size_t elem, int rank, const size_t* dims, const int* perm,
                   void* y) {
    size_t n = 1, in_stride[8], out_dims[8];
    for (int d = 0; d < rank; ++d) n *= dims[d];
    size_t st = 1;
    for (int d = rank - 1; d >= 0; --d) {
        in_stride[d] = st;
        st *= dims[d];
    }
    for (int d = 0; d < rank; ++d) out_dims[d] = dims[perm[d]];
    for (size_t o = 0; o < n; ++o) {
        size_t rem = o, src = 0;
        for (int d = rank - 1; d >= 0; --d) {
            const size_t idx = rem % out_dims[d];
            rem /= out_dims[d];
            src += idx * in_stride[perm[d]];
        }
        memcpy((char*)y + o * elem, (const char*)x + src * elem, elem);
    }
}
