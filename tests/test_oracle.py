"""Pin the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so a plausible slip in the restatement fails it:
  * f32 instead of f64 DQL arithmetic -> the reference literals [-1,0,1] -> zp 128 and
    [0,2,4] -> y[1] = 128 fail (both are f64-only results);
  * truncation instead of round-half-to-even -> the same literals fail;
  * a range that does not include 0 -> the max/min-adjusted ONNX goldens fail;
  * a dropped zero-point term or a transposed operand in MatMulInteger -> the ONNX golden
    (a_zp = 12) and the int64 brute force fail;
  * a fused multiply-add or a swapped Div operand -> the bit-exact *_bcast goldens fail.
"""
import math

import numpy as np
import pytest

import oracle
from tests.golden_util import NP, bits, tensor


# --------------------------------------------------------------------------------------
# DynamicQuantizeLinear
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["test_dynamicquantizelinear_max_adjusted",
                                  "test_dynamicquantizelinear_min_adjusted"])
def test_dql_onnx_goldens_exact(goldens, case):
    g = goldens[case]
    x = tensor(g["inputs"][0])
    y, s, zp = oracle.dynamic_quantize_linear(x)
    ey, es, ezp = (tensor(t) for t in g["outputs"])
    assert y.shape == ey.shape
    np.testing.assert_array_equal(y, ey)
    assert bits(s) == bits(es)
    assert zp == ezp


def test_dql_onnx_golden_known_f64_divergence(goldens):
    """test_dynamicquantizelinear: scale and zp match the ONNX golden; y matches except
    y[3], where x/scale = -127.5 exactly in f64 (reference: RNE -> -128 -> y = 25) but
    -127.49999 in f32 (the golden's 26).  The reference's f64 semantics are the contract."""
    g = goldens["test_dynamicquantizelinear"]
    x = tensor(g["inputs"][0])
    y, s, zp = oracle.dynamic_quantize_linear(x)
    ey, es, ezp = (tensor(t) for t in g["outputs"])
    assert bits(s) == bits(es) and zp == ezp
    diff = np.nonzero(y != ey)[0].tolist()
    assert diff == [3] and int(y[3]) == 25 and int(ey[3]) == 26
    # the golden is what f32 arithmetic produces: x / scale_f32 rounded in f32
    q32 = np.rint(x.astype(np.float32) / es.astype(np.float32)).astype(np.float32) + np.float32(zp)
    assert int(np.clip(q32, 0, 255)[3]) == 26


def test_dql_reference_literals(literals):
    for lit in literals["dql"]:
        if "x" not in lit:
            continue
        x = np.array(lit["x"], np.float32).reshape(lit["shape"])
        y, s, zp = oracle.dynamic_quantize_linear(x)
        if "y" in lit:
            assert y.tolist() == lit["y"], lit["cite"]
        if "zp" in lit:
            assert int(zp) == lit["zp"], lit["cite"]
        if "scale" in lit:
            assert float(s) == lit["scale"], lit["cite"]
        if "scale_approx" in lit:
            assert abs(float(s) - lit["scale_approx"]) < lit["scale_tol"], lit["cite"]


def test_dql_shape_preserved(literals):
    lit = literals["dql"][3]
    x = (np.arange(lit["count"], dtype=np.float32) * np.float32(lit["x_range_times"])).reshape(
        lit["shape"])
    y, s, zp = oracle.dynamic_quantize_linear(x)
    assert y.shape == tuple(lit["shape"]) and s.shape == () and zp.shape == ()


def _py_dql(xs):
    """Independent pure-Python restatement (Python floats are IEEE f64; round() on a float
    is round-half-to-even) used as a brute-force check on small inputs."""
    mn, mx = 0.0, 0.0
    for v in xs:
        if math.isnan(v):
            continue
        mn, mx = min(mn, v), max(mx, v)
    if mn == mx:
        return [0] * len(xs), 0.0, 0
    s = (mx - mn) / 255.0
    zp = int(min(max(round(0.0 - mn / s), 0), 255))
    ys = []
    for v in xs:
        q = v / s
        if math.isnan(q):
            ys.append(0)
            continue
        q = float(round(q)) if math.isfinite(q) else q
        ys.append(int(min(max(q + zp, 0.0), 255.0)))
    return ys, s, zp


def test_dql_bruteforce_against_python_f64():
    rng = np.random.default_rng(1234)
    for trial in range(300):
        n = int(rng.integers(1, 64))
        kind = trial % 4
        if kind == 0:
            x = rng.standard_normal(n).astype(np.float32)
        elif kind == 1:  # many exact ties: small integers / 2^k
            x = (rng.integers(-64, 64, n) / 4.0).astype(np.float32)
        elif kind == 2:  # skewed positive
            x = (rng.random(n) * 7 + 0.5).astype(np.float32)
        else:  # with NaN / signed zero
            x = rng.standard_normal(n).astype(np.float32)
            x[rng.integers(0, n)] = np.nan
            x[rng.integers(0, n)] = -0.0
        y, s, zp, s64 = oracle.dynamic_quantize_linear(x, return_scale64=True)
        ey, es, ezp = _py_dql([float(v) for v in x])
        assert y.tolist() == ey, (trial, x)
        assert s64 == es and int(zp) == ezp
        assert bits(s) == bits(np.float32(es))


def test_dql_invariants():
    rng = np.random.default_rng(7)
    x = np.sort(rng.standard_normal(4096).astype(np.float32) * 3 + 0.5)
    x = np.concatenate([x, np.zeros(1, np.float32)])
    y, s, zp = oracle.dynamic_quantize_linear(x)
    assert 0 <= int(zp) <= 255 and float(s) > 0
    assert int(y[-1]) == int(zp)  # zero is exactly representable
    ys = y[:-1].astype(np.int64)
    assert np.all(np.diff(ys) >= 0)  # monotone in x
    assert ys[0] == 0 and ys[-1] == 255  # the extremes map to the end points
    # all-NaN input has an empty range -> the constant-input sentinel
    yn, sn, zpn = oracle.dynamic_quantize_linear(np.full(5, np.nan, np.float32))
    assert yn.tolist() == [0] * 5 and float(sn) == 0.0 and int(zpn) == 0
    # NaN elements quantize to 0
    yx, _, _ = oracle.dynamic_quantize_linear(np.array([1.0, np.nan, -2.0], np.float32))
    assert int(yx[1]) == 0


def test_dql_rejects_non_float():
    with pytest.raises(oracle.OracleError):
        oracle.dynamic_quantize_linear(np.array([1, 2, 3], np.int32))


# --------------------------------------------------------------------------------------
# MatMulInteger
# --------------------------------------------------------------------------------------
def test_mmi_onnx_golden(goldens):
    g = goldens["test_matmulinteger"]
    a, b, azp, bzp = (tensor(t) for t in g["inputs"])
    out = oracle.matmul_integer(a, b, azp, bzp)
    np.testing.assert_array_equal(out, tensor(g["outputs"][0]))


def test_mmi_reference_literals(literals):
    for lit in literals["matmul_integer"]:
        if "a" in lit:
            a = np.array(lit["a"], NP[lit["a_dtype"]]).reshape(lit["a_shape"])
            b = np.array(lit["b"], NP[lit["b_dtype"]]).reshape(lit["b_shape"])
        else:
            a = np.full(lit["a_shape"], lit["fill_a"], NP[lit["a_dtype"]])
            b = np.full(lit["b_shape"], lit["fill_b"], NP[lit["b_dtype"]])
        azp = bzp = None
        if "a_zp" in lit:
            azp = np.array(lit["a_zp"], NP[lit["a_dtype"]]).reshape(lit["zp_shape"])
            bzp = np.array(lit["b_zp"], NP[lit["b_dtype"]]).reshape(lit["zp_shape"])
        out = oracle.matmul_integer(a, b, azp, bzp)
        if "out" in lit:
            assert out.reshape(-1).tolist() == lit["out"], lit["cite"]
        else:
            assert np.all(out == lit["fill_out"]), lit["cite"]


def test_mmi_rejects_like_reference(literals):
    for lit in literals["matmul_integer_rejects"]:
        a = np.ones(lit["a_shape"], NP[lit["a_dtype"]])
        b = np.ones(lit["b_shape"], NP[lit["b_dtype"]])
        azp = None
        if "a_zp" in lit:
            azp = np.array(lit["a_zp"], NP[lit["a_zp_dtype"]])
        with pytest.raises(oracle.OracleError):
            oracle.matmul_integer(a, b, azp)


@pytest.mark.parametrize("adt,bdt", [(np.uint8, np.int8), (np.int8, np.int8),
                                     (np.int8, np.uint8), (np.uint8, np.uint8)])
def test_mmi_bruteforce_int64(adt, bdt):
    rng = np.random.default_rng(42)
    for _ in range(12):
        M, K, N = (int(v) for v in rng.integers(1, 40, 3))
        a = rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1, (M, K)).astype(adt)
        b = rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1, (K, N)).astype(bdt)
        azp = np.array(rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1), adt)
        bzp = np.array(rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1), bdt)
        out = oracle.matmul_integer(a, b, azp, bzp)
        ref = (a.astype(np.int64) - int(azp)) @ (b.astype(np.int64) - int(bzp))
        np.testing.assert_array_equal(out, ref)


def test_mmi_per_column_zero_point_closed_form():
    """ONNX per-column b_zero_point (not supported by the reference): pinned by the
    expansion sum_k (a-az)(b-bz_n) = S_ab - bz_n*Ra - az*Cb_n + K*az*bz_n."""
    rng = np.random.default_rng(3)
    M, K, N = 17, 45, 23
    a = rng.integers(0, 256, (M, K)).astype(np.uint8)
    b = rng.integers(-127, 128, (K, N)).astype(np.int8)
    azp = np.uint8(131)
    bzp = rng.integers(-8, 9, N).astype(np.int8)
    out = oracle.matmul_integer(a, b, azp, bzp, per_column_b_zp=True)
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    closed = (a64 @ b64 - np.outer(a64.sum(1), bzp.astype(np.int64))
              - int(azp) * b64.sum(0)[None, :] + K * int(azp) * bzp.astype(np.int64)[None, :])
    np.testing.assert_array_equal(out, closed)
    with pytest.raises(oracle.OracleError):  # the reference's scalar-only contract
        oracle.matmul_integer(a, b, azp, bzp)


def test_mmi_overflow_is_an_error():
    """The reference's checked i32 arithmetic panics on overflow (matmul_integer.rs:255-262)."""
    K_ok, K_bad = 33025, 33100  # 255 * -255 * K crosses -2^31 between these
    for K, bad in ((K_ok, False), (K_bad, True)):
        a = np.full((1, K), 255, np.uint8)
        b = np.full((K, 1), -128, np.int8)
        bzp = np.array(127, np.int8)
        if bad:
            with pytest.raises(oracle.OracleError):
                oracle.matmul_integer(a, b, None, bzp)
        else:
            assert int(oracle.matmul_integer(a, b, None, bzp)[0, 0]) == 255 * -255 * K


# --------------------------------------------------------------------------------------
# Cast / Mul / Add / Div
# --------------------------------------------------------------------------------------
def test_cast_i32_f32_rounding():
    x = np.array([0, 1, -7, 2**24, 2**24 + 1, 2**24 + 3, -(2**31), 2**31 - 1, 67108865],
                 np.int32)
    y = oracle.cast_i32_f32(x)
    expect = [0.0, 1.0, -7.0, 16777216.0, 16777216.0, 16777220.0, -2147483648.0,
              2147483648.0, 67108864.0]
    assert y.tolist() == expect


@pytest.mark.parametrize("case,fn", [("test_mul", oracle.mul), ("test_mul_bcast", oracle.mul),
                                     ("test_add", oracle.add), ("test_add_bcast", oracle.add),
                                     ("test_div", oracle.div), ("test_div_bcast", oracle.div)])
def test_binary_onnx_goldens_bit_exact(goldens, case, fn):
    g = goldens[case]
    a, b = (tensor(t) for t in g["inputs"])
    out = fn(a, b)
    np.testing.assert_array_equal(bits(out), bits(tensor(g["outputs"][0])))


def test_div_reference_literals(literals):
    for lit in literals["div"]:
        out = oracle.div(np.array(lit["a"], np.float32), np.array(lit["b"], np.float32))
        for o, e in zip(out.tolist(), lit["expect"]):
            if e == "nan":
                assert math.isnan(o)
            elif e == "inf":
                assert o == math.inf
            else:
                assert abs(o - e) < 1e-6


def test_binary_broadcast_orders_and_errors():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 7)).astype(np.float32)
    c = (rng.random(7) + 0.5).astype(np.float32)
    s = np.float32(0.37)
    with np.errstate(all="ignore"):
        for fn, npf in ((oracle.mul, np.multiply), (oracle.add, np.add),
                        (oracle.div, np.divide), (oracle.sub, np.subtract)):
            np.testing.assert_array_equal(bits(fn(x, c)), bits(npf(x, c)))
            np.testing.assert_array_equal(bits(fn(c, x)), bits(npf(c, x)))
            np.testing.assert_array_equal(bits(fn(x, s)), bits(npf(x, s)))
            np.testing.assert_array_equal(bits(fn(x[:, None, :], c[None, :, None][:, :1])),
                                          bits(npf(x[:, None, :], c[None, :, None][:, :1])))
    with pytest.raises(oracle.OracleError):
        oracle.add(x, np.ones(5, np.float32))


# --------------------------------------------------------------------------------------
# DequantizeLinear
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["test_dequantizelinear", "test_dequantizelinear_axis"])
def test_dequantize_onnx_goldens(goldens, case):
    g = goldens[case]
    x, s, zp = (tensor(t) for t in g["inputs"])
    out = oracle.dequantize_linear(x, s, zp, axis=g["attributes"].get("axis", 1))
    np.testing.assert_array_equal(bits(out), bits(tensor(g["outputs"][0])))


def test_dequantize_reference_literals(literals):
    for lit in literals["dequantize_linear"]:
        x = np.array(lit["x"], NP[lit["x_dtype"]]).reshape(lit["x_shape"])
        s = np.array(lit["scale"], np.float32).reshape(lit["scale_shape"])
        zp = None
        if "zp" in lit:
            zp = np.array(lit["zp"], NP[lit["x_dtype"]]).reshape(lit["scale_shape"])
        out = oracle.dequantize_linear(x, s, zp, axis=lit.get("axis", 1)).reshape(-1)
        if lit["tol"] is None:
            assert out.tolist() == lit["y"], lit["cite"]
        else:
            assert np.max(np.abs(out - np.array(lit["y"]))) < lit["tol"], lit["cite"]
    for lit in literals["dequantize_linear_rejects"]:
        x = np.array(lit["x"], NP[lit["x_dtype"]]).reshape(lit["x_shape"])
        s = np.array(lit["scale"], np.float32).reshape(lit["scale_shape"])
        zp = np.array(lit["zp"], NP[lit["zp_dtype"]]).reshape(lit["zp_shape"])
        with pytest.raises(oracle.OracleError):
            oracle.dequantize_linear(x, s, zp)


def test_dequantize_is_cast_then_sub_then_mul():
    """(x as f32 - zp as f32) * scale: two f32 roundings, not an i64 subtract (the
    reference GPU kernel's form) — visible only when |x| > 2^24."""
    x = np.array([2**24 + 1, 2**25 + 3, -5], np.int32)
    zp = np.array(1, np.int32)
    out = oracle.dequantize_linear(x, np.array(1.0, np.float32), zp)
    expect = ((x.astype(np.float32) - np.float32(1)) * np.float32(1)).tolist()
    assert out.tolist() == expect
    # (2^24+1 -> 2^24 as f32) - 1 = 2^24 - 1; the i64 form would give (2^24+1-1) = 2^24
    assert out[0] == np.float32(2**24 - 1)
    assert np.float32(np.int64(2**24 + 1) - 1) == np.float32(2**24)


def test_qlinear_graph_close_to_float64():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 8, 32)).astype(np.float32)
    w = rng.integers(-127, 128, (32, 16)).astype(np.int8)
    bias = (rng.standard_normal(16) * 0.02).astype(np.float32)
    out = oracle.qlinear_graph(x, w, np.array(0, np.int8), np.array(0.02, np.float32), bias)
    xq, xs, xzp = out["xq"], float(out["x_scale"]), int(out["x_zp"])
    ref = ((xq.astype(np.float64) - xzp) @ w.astype(np.float64)) * xs * 0.02 + bias
    np.testing.assert_allclose(out["linear"], ref, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------------------
# Gather
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["test_gather_0", "test_gather_1", "test_gather_2d_indices",
                                  "test_gather_negative_indices"])
def test_gather_onnx_goldens(goldens, case):
    g = goldens[case]
    data, idx = (tensor(t) for t in g["inputs"])
    out = oracle.gather(data, idx, axis=(g["attributes"] or {}).get("axis", 0))
    want = tensor(g["outputs"][0])
    assert out.shape == want.shape and out.dtype == want.dtype
    np.testing.assert_array_equal(bits(out), bits(want))


def test_gather_bruteforce_negative_and_clamped_indices():
    """Element by element in pure Python: out[pre, idx, post] = data[pre, k(idx), post] with
    k = i + len when negative, then clamped into the axis (the GPU kernels' rule)."""
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, (3, 5, 4)).astype(np.uint8)
    for axis in (0, 1, 2, -1):
        ax = axis % 3
        n = data.shape[ax]
        idx = np.array([[0, n - 1, -1], [-n, n + 2, -n - 3]], np.int64)
        out = oracle.gather(data, idx, axis=axis)
        assert out.dtype == np.uint8
        assert out.shape == data.shape[:ax] + idx.shape + data.shape[ax + 1:]
        for o in np.ndindex(out.shape):
            i = idx[o[ax:ax + 2]]
            k = i + n if i < 0 else i
            k = min(max(k, 0), n - 1)
            src = o[:ax] + (k,) + o[ax + 2:]
            assert out[o] == data[src], (axis, o)


def test_gather_identity_and_reversal():
    x = np.arange(2 * 7 * 3, dtype=np.float32).reshape(2, 7, 3)
    np.testing.assert_array_equal(oracle.gather(x, np.arange(7), axis=1), x)
    np.testing.assert_array_equal(oracle.gather(x, np.arange(-1, -8, -1), axis=1), np.flip(x, axis=1))
    assert oracle.gather(x, np.array(3, np.int64), axis=1).shape == (2, 3)
