"""Pins of the oracle's ReduceMean, Pow and Sqrt, and of the node-by-node LayerNorm they
compose (an export below opset 17 writes LayerNorm as ReduceMean -> Sub -> Pow(2) ->
ReduceMean -> Add(eps) -> Sqrt -> Div -> Mul -> Add; the reference runs those nodes one by
one, src/graph_executor.rs:356-432).

What pins each function:
  * ReduceMean (src/operators/reduce_mean.rs:19-105) — the eight ONNX 1.18
    ``test_reduce_mean_*`` goldens the reference vendors (numpy's mean: values within f32
    rounding; the reference's own rank-0 result of the full reduction is reshaped to the
    golden's [1, 1, 1]); hand-derived known answers that only the right summation order gives
    (ndarray 0.16: unrolled_fold over the contiguous last axis, plain order otherwise); a
    float64 brute force.
  * Pow (src/operators/pow.rs:18-45, f32::powf = the C library's powf) — the four float
    ``test_pow*`` goldens; within one ulp of the correctly rounded square for exponent 2, and
    equal to it for all but a small fraction of inputs (glibc's powf is not correctly rounded).
  * Sqrt (src/operators/sqrt.rs:18-30) — the two ``test_sqrt*`` goldens, and numpy's
    correctly rounded float32 sqrt bit for bit.
  * The decomposed LayerNorm with the square (Mul(c, c)) is the fused LayerNormalization
    oracle (itself pinned by the ONNX LayerNormalization goldens) bit for bit; with powf it is
    within 1e-6 of it.
"""
import numpy as np
import pytest

import oracle
from tests.golden_util import bits, tensor

REDUCE_MEAN = [
    "test_reduce_mean_default_axes_keepdims_example", "test_reduce_mean_default_axes_keepdims_random",
    "test_reduce_mean_do_not_keepdims_example", "test_reduce_mean_do_not_keepdims_random",
    "test_reduce_mean_keepdims_example", "test_reduce_mean_keepdims_random",
    "test_reduce_mean_negative_axes_keepdims_example", "test_reduce_mean_negative_axes_keepdims_random",
]


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def ulps(a, b):
    """|a - b| in units in the last place of float32 (same-sign finite values)."""
    ia = bits(a).astype(np.int64)
    ib = bits(b).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("case", REDUCE_MEAN)
def test_reduce_mean_goldens(goldens, case):
    c = goldens[case]
    x, axes = tensor(c["inputs"][0]), tensor(c["inputs"][1])
    keep = c["attributes"].get("keepdims", 1) == 1
    y = oracle.reduce_mean(x, list(axes.reshape(-1)), keepdims=keep)
    want = tensor(c["outputs"][0])
    if axes.size == 0:
        assert y.shape == ()  # the reference's full reduction is rank 0; ONNX keeps [1]*rank
        y = y.reshape(want.shape)
    assert y.shape == want.shape, case
    assert rel_err(y, want) < 2e-7, case


def test_reduce_mean_order_known_answers():
    # [2^24, 1 x 15]: the true sum is 2^24 + 15.  ndarray's unrolled_fold over a contiguous
    # lane: p0 = 2^24 + 1 -> 2^24 (tie to even), p1..p7 = 1 + 1 = 2, then
    # 0 + (p0 + p4) + (p1 + p5) + (p2 + p6) + (p3 + p7) = 2^24 + 14 exactly; / 16 = 2^20 + 0.875.
    # Added in order (a middle axis, res = 0 + x0 + x1 + ...) every +1 rounds back to 2^24:
    # 2^24 / 16 = 2^20.
    v = np.array([2.0 ** 24] + [1.0] * 15, np.float32)
    assert oracle.reduce_mean(v.reshape(1, 16), [-1])[0, 0] == np.float32(2 ** 20 + 0.875)
    assert oracle.reduce_mean(v.reshape(1, 16, 1), [1])[0, 0, 0] == np.float32(2 ** 20)
    assert oracle.reduce_mean(v.reshape(2, 8), None) == np.float32(2 ** 20 + 0.875)  # data.mean()
    assert oracle.reduce_mean(v.reshape(4, 4), [-1], keepdims=False).shape == (4,)
    # a trailing size-1 axis does not make the reduced axis the contiguous one: plain order
    assert oracle.reduce_mean(v.reshape(1, 16, 1), [-2])[0, 0, 0] == np.float32(2 ** 20)


@pytest.mark.parametrize("shape,axis", [((7, 768), -1), ((3, 5, 13), 1), ((4, 9), 0),
                                        ((2, 3, 4, 5), 2), ((1000,), 0)])
def test_reduce_mean_against_float64(shape, axis):
    x = np.random.default_rng(7).standard_normal(shape).astype(np.float32)
    y = oracle.reduce_mean(x, [axis])
    want = x.astype(np.float64).mean(axis=axis, keepdims=True)
    assert np.max(np.abs(y - want)) < 1e-6 * max(1.0, np.max(np.abs(x)))


@pytest.mark.parametrize("case", ["test_pow", "test_pow_bcast_array", "test_pow_bcast_scalar",
                                  "test_pow_example"])
def test_pow_goldens(goldens, case):
    c = goldens[case]
    x, e = (tensor(t) for t in c["inputs"])
    y = oracle.pow(x, e)
    want = tensor(c["outputs"][0])
    assert y.shape == want.shape
    assert int(np.max(ulps(y, want))) <= 1, case
    if case != "test_pow":  # small integer powers: exact
        assert np.array_equal(bits(y), bits(want)), case


def test_pow_two_is_the_square_within_one_ulp():
    x = np.random.default_rng(11).standard_normal(2_000_000).astype(np.float32)
    got = oracle.pow(x, np.float32(2.0))
    exact = (x.astype(np.float64) ** 2).astype(np.float32)  # x^2 exact in f64, rounded once
    d = ulps(got, exact)
    assert int(d.max()) <= 1
    frac = float(np.mean(d != 0))
    # glibc's powf misrounds a small fraction (0.07 % of [1, 2) exhaustively on glibc 2.35)
    assert frac < 5e-3, frac
    # special values of C99 Annex F that the reference's f32::powf inherits
    sp = oracle.pow(np.array([-2.0, 0.0, -0.0, np.inf, -np.inf, np.nan, 1.0], np.float32),
                    np.array([3.0, -1.0, 2.0, 2.0, 2.0, 0.0, np.nan], np.float32))
    assert sp[0] == -8.0 and sp[1] == np.inf and bits(sp[2]) == bits(np.float32(0.0))
    assert sp[3] == np.inf and sp[4] == np.inf and sp[5] == 1.0 and sp[6] == 1.0


def test_pow_rejects_an_exponent_that_does_not_broadcast():
    with pytest.raises(oracle.OracleError):
        oracle.pow(np.ones((2, 3), np.float32), np.ones((4,), np.float32))


@pytest.mark.parametrize("case", ["test_sqrt", "test_sqrt_example"])
def test_sqrt_goldens(goldens, case):
    c = goldens[case]
    x = tensor(c["inputs"][0])
    assert np.array_equal(bits(oracle.sqrt(x)), bits(tensor(c["outputs"][0])))


def test_sqrt_is_numpys_correctly_rounded_sqrt():
    x = np.abs(np.random.default_rng(5).standard_normal(100_000)).astype(np.float32) * 1e3
    x[:4] = [0.0, 1.0, 2.0, np.inf]
    assert np.array_equal(bits(oracle.sqrt(x)), bits(np.sqrt(x)))
    assert np.isnan(oracle.sqrt(np.array([-1.0], np.float32))[0])


@pytest.mark.parametrize("rows,cols", [(64, 768), (33, 100), (5, 7), (16, 1024)])
def test_decomposed_layer_norm_with_the_square_is_layer_normalization(rows, cols):
    rng = np.random.default_rng(rows * cols)
    x = (rng.standard_normal((rows, cols)) * 3 + 0.5).astype(np.float32)
    g = rng.uniform(0.9, 1.1, cols).astype(np.float32)
    b = (0.02 * rng.standard_normal(cols)).astype(np.float32)
    for eps in (1e-12, 1e-5):
        fused = oracle.layer_norm(x, g, b, eps=np.float32(eps))
        dec = oracle.layer_norm_decomposed(x, g, b, eps, square=True)
        assert np.array_equal(bits(dec), bits(fused)), eps
        # with the reference's powf: within 1e-6 (a last-bit difference in a few squares)
        assert rel_err(oracle.layer_norm_decomposed(x, g, b, eps), fused) < 1e-6
    # no affine tail: the fused norm with gamma 1 and beta -0 (which change no bit)
    plain = oracle.layer_norm_decomposed(x, None, None, 1e-5, square=True)
    ident = oracle.layer_norm(x, np.ones(cols, np.float32), np.full(cols, -0.0, np.float32),
                              eps=np.float32(1e-5))
    assert np.array_equal(bits(plain), bits(ident))
    # the residual Add in front is the Add node
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    assert np.array_equal(bits(oracle.layer_norm_decomposed(x, g, b, 1e-5, residual=r, square=True)),
                          bits(oracle.layer_norm(oracle.add(x, r), g, b, eps=np.float32(1e-5))))
