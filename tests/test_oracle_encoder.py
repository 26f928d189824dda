"""Pins of the oracle's encoder ops (LayerNormalization, Softmax, Erf, f32 MatMul, Transpose)
— the fp32 ops the DistilBERT-shaped encoder needs around the quantized linears.

Sources of truth, in order of strength:
  * the ONNX 1.18 node goldens the reference vendors (tests/golden/onnx_node_goldens.json);
    they were produced by numpy, whose summation order differs from the reference's
    ndarray, so fp32 reductions are compared within a stated tolerance;
  * the reference's own unit-test literals for Erf (src/operators/erf.rs tests);
  * float64 brute force and invariants (row sums, symmetry, shift behaviour).
The exact f32 summation order of ndarray 0.16 (`unrolled_fold`, a dependency absent from
the reference checkout) is restated, not imported; tests below check the restatement's
internal consistency and its agreement with float64 sums.
"""
import itertools
import math

import numpy as np
import pytest

import oracle
from tests.golden_util import bits, tensor

ENC_GOLDENS = [
    "test_layer_normalization_2d_axis1", "test_layer_normalization_2d_axis_negative_1",
    "test_layer_normalization_3d_axis2_epsilon",
    "test_layer_normalization_3d_axis_negative_1_epsilon",
    "test_layer_normalization_4d_axis3", "test_layer_normalization_4d_axis_negative_1",
]


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.mark.parametrize("case", ENC_GOLDENS)
def test_layer_norm_goldens(goldens, case):
    c = goldens[case]
    x, scale, bias = (tensor(t) for t in c["inputs"])
    eps = c["attributes"].get("epsilon", 1e-5)
    y = oracle.layer_norm(x, scale, bias, eps=eps)
    want = tensor(c["outputs"][0])
    assert rel_err(y, want) < 2e-6, case


@pytest.mark.parametrize("case", ["test_softmax_example", "test_softmax_axis_2",
                                  "test_softmax_default_axis", "test_softmax_negative_axis",
                                  "test_softmax_large_number"])
def test_softmax_goldens(goldens, case):
    c = goldens[case]
    x = tensor(c["inputs"][0])
    y = oracle.softmax(x, axis=c["attributes"].get("axis", -1))
    assert rel_err(y, tensor(c["outputs"][0])) < 1e-6, case


def test_erf_golden(goldens):
    c = goldens["test_erf"]
    x = tensor(c["inputs"][0])
    # Abramowitz-Stegun 7.1.26 has |error| <= 1.5e-7; evaluated in f32 (as the reference
    # does) a few roundings near 1 add up to ~3e-7 more.  The golden is the exact erf.
    assert float(np.max(np.abs(oracle.erf(x) - tensor(c["outputs"][0])))) < 6e-7


@pytest.mark.parametrize("case", ["test_matmul_2d", "test_matmul_3d", "test_matmul_4d"])
def test_matmul_goldens(goldens, case):
    c = goldens[case]
    a, b = (tensor(t) for t in c["inputs"])
    assert rel_err(oracle.matmul_f32(a, b), tensor(c["outputs"][0])) < 1e-6


@pytest.mark.parametrize("case", ["test_transpose_default"] +
                         ["test_transpose_all_permutations_%d" % i for i in range(6)])
def test_transpose_goldens_exact(goldens, case):
    c = goldens[case]
    x = tensor(c["inputs"][0])
    y = oracle.transpose(x, c["attributes"].get("perm"))
    assert np.array_equal(bits(y), bits(tensor(c["outputs"][0])))


# ---- Erf: the reference's unit-test literals (src/operators/erf.rs tests) ----------------
def test_erf_reference_literals():
    e = lambda v: float(oracle.erf(np.array([v], np.float32))[0])
    assert e(0.0) == 0.0
    assert abs(e(1.0) - 0.8427008) < 1e-6 and abs(e(-1.0) + 0.8427008) < 1e-6
    assert e(math.inf) == 1.0 and e(-math.inf) == -1.0
    assert math.isnan(e(math.nan))
    assert abs(e(0.5) - 0.5204999) < 2e-7 and abs(e(-0.5) + 0.5204999) < 2e-7
    assert abs(e(2.5) - 0.9995931) < 2e-7 and abs(e(-2.5) + 0.9995931) < 2e-7


def test_erf_grid_properties():
    """The reference's grid tests (odd symmetry, bounds) plus the A&S error bound against
    the float64 erf on [-6, 6] step 0.001."""
    g = (-6.0 + np.arange(12001, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    y = oracle.erf(g)
    assert float(np.max(np.abs(oracle.erf(-g) + y))) < 1e-6
    assert float(np.max(np.abs(y))) <= 1.0 + 1e-6
    exact = np.array([math.erf(float(v)) for v in g])
    assert float(np.max(np.abs(y - exact))) < 6e-7


# ---- summation order (ndarray unrolled_fold restatement) ---------------------------------
def _unrolled8_py(x):
    x = np.asarray(x, np.float32)
    p = [np.float32(0)] * 8
    n8 = len(x) // 8 * 8
    for i in range(0, n8, 8):
        for j in range(8):
            p[j] = np.float32(p[j] + x[i + j])
    acc = np.float32(0)
    for a, b in ((0, 4), (1, 5), (2, 6), (3, 7)):
        acc = np.float32(acc + np.float32(p[a] + p[b]))
    for v in x[n8:]:
        acc = np.float32(acc + v)
    return acc


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 15, 64, 100, 768, 3073])
def test_sum_unrolled8_order(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * np.float32(1e3)
    assert np.array_equal(bits(oracle.sum_unrolled8(x)), bits(_unrolled8_py(x)))
    if n:
        assert abs(float(oracle.sum_unrolled8(x)) - float(np.sum(x, dtype=np.float64))) < 1e-3 * n
    # an order-sensitive input: a sequential sum loses the unit terms, the 8-way one keeps
    # the ones accumulated away from the large partial
    y = np.array([2.0 ** 24] + [1.0] * 15, np.float32)
    assert float(oracle.sum_unrolled8(y)) == 2.0 ** 24 + 14.0


def test_layer_norm_matches_float64_and_normalises():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((64, 768)) * 3 + 1).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, 768).astype(np.float32)
    bias = rng.standard_normal(768).astype(np.float32)
    y = oracle.layer_norm(x, scale, bias, eps=1e-12)
    xd = x.astype(np.float64)
    m = xd.mean(-1, keepdims=True)
    v = ((xd - m) ** 2).mean(-1, keepdims=True)
    want = (xd - m) / np.sqrt(v + 1e-12) * scale + bias
    assert rel_err(y, want) < 1e-5
    z = oracle.layer_norm(x, np.ones(768, np.float32), np.zeros(768, np.float32))
    assert float(np.max(np.abs(z.mean(-1)))) < 1e-5
    assert float(np.max(np.abs(z.astype(np.float64).var(-1) - 1.0))) < 1e-3


def test_softmax_rows_sum_to_one_and_handle_extremes():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((32, 128)) * 4).astype(np.float32)
    y = oracle.softmax(x)
    assert float(np.max(np.abs(y.astype(np.float64).sum(-1) - 1.0))) < 1e-6
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(-1, keepdims=True))
    assert rel_err(y, e / e.sum(-1, keepdims=True)) < 1e-6
    big = np.array([[1e4, 1e4 - 1, -np.inf, 0.0]], np.float32)
    yb = oracle.softmax(big)
    assert yb[0, 2] == 0.0 and abs(float(yb.sum()) - 1.0) < 1e-6


def test_matmul_batch_rules_and_float64():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((3, 5, 7)).astype(np.float32)
    b = rng.standard_normal((7, 4)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_err(oracle.matmul_f32(a, b), want) < 1e-6
    b3 = rng.standard_normal((3, 7, 4)).astype(np.float32)
    assert rel_err(oracle.matmul_f32(a, b3), a.astype(np.float64) @ b3) < 1e-6
    a2 = rng.standard_normal((5, 7)).astype(np.float32)
    assert rel_err(oracle.matmul_f32(a2, b3), a2.astype(np.float64) @ b3) < 1e-6
    with pytest.raises(oracle.OracleError):
        oracle.matmul_f32(a, rng.standard_normal((2, 7, 4)).astype(np.float32))


def test_transpose_all_rank4_permutations_exact():
    x = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    for perm in itertools.permutations(range(4)):
        assert np.array_equal(oracle.transpose(x, perm), x.transpose(perm))
    u = np.arange(24, dtype=np.uint8).reshape(2, 3, 4)
    assert np.array_equal(oracle.transpose(u, (1, 2, 0)), u.transpose(1, 2, 0))
