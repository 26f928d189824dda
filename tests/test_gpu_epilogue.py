"""GPU parity: the fused quantized linear (MatMulInteger + Cast + dequant Mul + bias Add +
Mul/Add/Div/Mul chain in the GEMM store), the standalone fused chain, Cast and
DequantizeLinear — against the oracle run op by op in graph order.

The north star's bar for the fp32 outputs is max-abs error <= 1e-5 relative to the output
magnitude; every op here rounds once in IEEE single precision exactly like the separate
reference nodes, so the tests assert the stronger bit-exact equality and report the
relative error when it fails.
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import configs, ops
from iconnx_amd._lib import IconnxError
from tests.golden_util import bits, tensor

pytestmark = pytest.mark.gpu
REL_TOL = 1e-5  # north-star tolerance for dequantized fp32 outputs


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def assert_f32_equal(got, want, what):
    if np.array_equal(bits(got), bits(want)):
        return
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)))) / scale
    n = int(np.count_nonzero(bits(got) != bits(want)))
    assert err <= REL_TOL, "%s: %d elements differ, max rel err %.3g" % (what, n, err)
    pytest.fail("%s: %d elements differ in the last bits (max rel err %.3g <= tol)"
                % (what, n, err))


def run_linear_config(cfg, sample_rows):
    d = configs.make(cfg)
    x = d["x"].reshape(-1, d["x"].shape[-1])
    M, K = x.shape
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    w = ops.PackedWeight(dev(d["w"]))
    epi = [("Mul", (xs, dev(d["w_scale"])), False), ("Add", dev(d["bias"]), False)]
    epi += [(op, dev(c), False) for op, c in d["chain"]]
    y = ops.gpu_qlinear(xq, w, xzp, dev(d["w_zp"]), epilogue=epi, a_rowsum=rs)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    chain = [(op, c, False) for op, c in d["chain"]]
    for r0, r1 in sample_rows(M):
        ref = oracle.qlinear_graph(x[:, :], d["w"], d["w_zp"], d["w_scale"], d["bias"], chain,
                                   rows=(r0, r1))
        assert_f32_equal(y[r0:r1], ref["y"][r0:r1], "%s rows %d:%d" % (cfg, r0, r1))
    return y


def test_cfg1_single_linear_all_rows():
    run_linear_config("cfg1", lambda M: [(0, M)])


def full_epilogue_check(cfg):
    """The fused quantized linear of a config on every output element.  The int32
    accumulators come from the GEMM without epilogue (every element of which
    tests/test_gpu_mmi.py checks against an exact float64 product; here sampled rows against
    the oracle), the DQL outputs are checked whole against the oracle, and the oracle's
    Cast -> Mul(x_scale * w_scale) -> Add(bias) -> chain, run over all of them, must equal the
    fused output bit for bit."""
    d = configs.make(cfg)
    x = d["x"].reshape(-1, d["x"].shape[-1])
    M, K = x.shape
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    w = ops.PackedWeight(dev(d["w"]))
    epi = [("Mul", (xs, dev(d["w_scale"])), False), ("Add", dev(d["bias"]), False)]
    epi += [(op, dev(c), False) for op, c in d["chain"]]
    y = ops.gpu_qlinear(xq, w, xzp, dev(d["w_zp"]), epilogue=epi, a_rowsum=rs)
    acc = ops.gpu_matmul_integer(xq, w, xzp, dev(d["w_zp"]), a_rowsum=rs)
    torch.cuda.synchronize()
    xq_h, xs_h, xzp_h = xq.cpu().numpy(), xs.cpu().numpy(), xzp.cpu().numpy()
    yq, ys, yz = oracle.dynamic_quantize_linear(x)
    assert np.array_equal(xq_h, yq) and bits(xs_h) == bits(np.float32(ys)) and int(xzp_h) == int(yz)
    acc = acc.cpu().numpy()
    per_col = np.asarray(d["w_zp"]).ndim == 1 and np.asarray(d["w_zp"]).size > 1
    for r0 in (0, M // 2 + 1, M - 2):
        want = oracle.matmul_integer(xq_h[r0:r0 + 2], d["w"], xzp_h, d["w_zp"], per_column_b_zp=per_col)
        assert np.array_equal(acc[r0:r0 + 2], want), "%s accumulators rows %d:%d" % (cfg, r0, r0 + 2)
    want = oracle.add(oracle.mul(oracle.cast_i32_f32(acc), oracle.mul(xs_h, d["w_scale"])), d["bias"])
    del acc
    for op, c in d["chain"]:
        want = {"Mul": oracle.mul, "Add": oracle.add, "Div": oracle.div, "Sub": oracle.sub}[op](want, c)
    assert_f32_equal(y.cpu().numpy(), want, "%s fused epilogue, every element" % cfg)


def test_cfg2_ffn_up_with_chain():
    run_linear_config("cfg2", lambda M: [(0, 40), (M // 2, M // 2 + 8), (M - 24, M)])
    full_epilogue_check("cfg2")


def test_cfg4_per_channel():
    run_linear_config("cfg4", lambda M: [(0, 16), (M // 3, M // 3 + 8), (M - 16, M)])
    full_epilogue_check("cfg4")


def test_cfg5a_fused_dequant_full_size():
    d = configs.make("cfg5a")
    a, b = d["a"], d["b"]
    w = ops.PackedWeight(dev(b))
    epi = [("Mul", (dev(d["a_scale"]), dev(d["b_scale"])), False)]
    y = ops.gpu_qlinear(dev(a), w, dev(d["a_zp"]), dev(d["b_zp"]), epilogue=epi)
    acc = ops.gpu_matmul_integer(dev(a), w, dev(d["a_zp"]), dev(d["b_zp"]))
    torch.cuda.synchronize()
    acc = acc.cpu().numpy()
    # accumulators: row sample vs the oracle
    for r in (0, 4097, 16383):
        want = oracle.matmul_integer(a[r:r + 1], b, d["a_zp"], d["b_zp"])
        assert np.array_equal(acc[r:r + 1], want)
    # epilogue over every element: Cast -> Mul(a_scale * b_scale), via the oracle ops
    s = oracle.mul(d["a_scale"], d["b_scale"])
    want = oracle.mul(oracle.cast_i32_f32(acc), s)
    assert_f32_equal(y.cpu().numpy(), want, "cfg5a epilogue")


def test_chain_cfg5b_full_size():
    d = configs.make("cfg5b")
    x = d["x"]
    y = ops.gpu_fused_chain(dev(x), [(op, dev(c), False) for op, c in d["chain"]])
    torch.cuda.synchronize()
    want = x
    for op, c in d["chain"]:
        want = {"Mul": oracle.mul, "Add": oracle.add, "Div": oracle.div}[op](want, c)
    assert_f32_equal(y.cpu().numpy(), want, "cfg5b chain")


def test_chain_operand_kinds_and_order():
    rng = np.random.default_rng(2)
    rows, cols = 37, 45  # not a multiple of 4: scalar kernel
    for rows, cols in ((37, 45), (64, 256)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        col = (rng.random(cols) + 0.5).astype(np.float32)
        row = (rng.random((rows, 1)) + 0.5).astype(np.float32)
        full = (rng.random((rows, cols)) + 0.5).astype(np.float32)
        s = np.array(1.75, np.float32)
        chain = [("Div", col, True), ("Sub", row, False), ("Mul", full, False),
                 ("Add", s, True), ("Div", (s, col), False), ("Sub", full, True)]
        y = ops.gpu_fused_chain(dev(x), [(op, tuple(dev(t) for t in c) if isinstance(c, tuple)
                                          else dev(c), lhs) for op, c, lhs in chain])
        want = x
        for op, c, lhs in chain:
            c = oracle.mul(*c) if isinstance(c, tuple) else c
            f = {"Mul": oracle.mul, "Add": oracle.add, "Div": oracle.div, "Sub": oracle.sub}[op]
            want = f(c, want) if lhs else f(want, c)
        assert_f32_equal(y.cpu().numpy(), want, "chain %dx%d" % (rows, cols))


def test_fused_pattern_wrappers(goldens):
    """MulAdd / AddMul / SubMul / DivMul: same-shape and [last-dim] broadcast, and the
    ONNX *_bcast goldens through the single-op binary path."""
    rng = np.random.default_rng(8)
    a = rng.standard_normal((3, 4, 5)).astype(np.float32)
    b = (rng.random(5) + 0.5).astype(np.float32)
    c = rng.standard_normal(5).astype(np.float32)
    cases = [(ops.gpu_fused_mul_add, lambda: oracle.add(oracle.mul(a, b), c)),
             (ops.gpu_fused_add_mul, lambda: oracle.mul(oracle.add(a, b), c)),
             (ops.gpu_fused_sub_mul, lambda: oracle.mul(oracle.sub(a, b), c)),
             (ops.gpu_fused_div_mul, lambda: oracle.mul(oracle.div(a, b), c))]
    for fn, ref in cases:
        assert_f32_equal(fn(dev(a), dev(b), dev(c)).cpu().numpy(), ref(), fn.__name__)
        bf, cf = np.broadcast_to(b, a.shape).copy(), np.broadcast_to(c, a.shape).copy()
        assert_f32_equal(fn(dev(a), dev(bf), dev(cf)).cpu().numpy(), ref(), fn.__name__ + " same")
    for case, name in (("test_mul_bcast", "Mul"), ("test_add_bcast", "Add"),
                       ("test_div_bcast", "Div"), ("test_mul", "Mul"), ("test_div", "Div")):
        g = goldens[case]
        x0, x1 = (tensor(t) for t in g["inputs"])
        got = ops.gpu_binary(name, dev(x0), dev(x1)).cpu().numpy()
        assert_f32_equal(got, tensor(g["outputs"][0]), case)


def test_div_ieee_special_values():
    a = np.array([0.0, 0.0, 1.0, 6.0, -8.0, 10.0], np.float32)
    b = np.array([0.0, 1e-12, 0.0, 2.0, 4.0, -5.0], np.float32)
    got = ops.gpu_binary("Div", dev(a), dev(b)).cpu().numpy()
    assert np.isnan(got[0]) and got[1] == 0.0 and got[2] == np.inf
    assert got[3:].tolist() == [3.0, -2.0, -2.0]


def test_cast_i32_f32():
    x = np.array([0, 1, -7, 2**24 + 1, 2**24 + 3, -(2**31), 2**31 - 1, 67108865], np.int32)
    rng = np.random.default_rng(1)
    x = np.concatenate([x, rng.integers(-2**31, 2**31 - 1, 100000).astype(np.int32)])
    got = ops.gpu_cast_i32_f32(dev(x)).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(oracle.cast_i32_f32(x)))


@pytest.mark.parametrize("case", ["test_dequantizelinear", "test_dequantizelinear_axis"])
def test_dequantize_goldens(goldens, case):
    g = goldens[case]
    x, s, zp = (tensor(t) for t in g["inputs"])
    got = ops.gpu_dequantize_linear(dev(x), dev(s), dev(zp), axis=g["attributes"].get("axis", 1))
    np.testing.assert_array_equal(bits(got.cpu().numpy()), bits(tensor(g["outputs"][0])))


def test_dequantize_reference_literals(literals):
    from tests.golden_util import NP
    for lit in literals["dequantize_linear"]:
        x = np.array(lit["x"], NP[lit["x_dtype"]]).reshape(lit["x_shape"])
        s = np.array(lit["scale"], np.float32).reshape(lit["scale_shape"])
        zp = np.array(lit["zp"], NP[lit["x_dtype"]]).reshape(lit["scale_shape"]) if "zp" in lit else None
        axis = lit.get("axis", 1)
        got = ops.gpu_dequantize_linear(dev(x), dev(s), None if zp is None else dev(zp), axis)
        want = oracle.dequantize_linear(x, s, zp, axis)
        np.testing.assert_array_equal(bits(got.cpu().numpy()), bits(want))
    for lit in literals["dequantize_linear_rejects"]:
        x = np.array(lit["x"], NP[lit["x_dtype"]]).reshape(lit["x_shape"])
        s = np.array(lit["scale"], np.float32).reshape(lit["scale_shape"])
        zp = np.array(lit["zp"], NP[lit["zp_dtype"]]).reshape(lit["zp_shape"])
        with pytest.raises(IconnxError):
            ops.gpu_dequantize_linear(dev(x), dev(s), dev(zp))


def test_dequantize_i32_large_values_follow_cpu_semantics():
    x = np.array([2**24 + 1, 2**25 + 3, -5, 123456789], np.int32)
    zp = np.array(1, np.int32)
    s = np.array(0.5, np.float32)
    got = ops.gpu_dequantize_linear(dev(x), dev(s), dev(zp)).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(oracle.dequantize_linear(x, s, zp)))


def test_ffn_down_shape_fused_epilogue():
    """FFN-down shape (K = 3072; 256 tiles of 128x96) with the dequant scale, bias and a
    Sub/Div/Mul chain with an operand on the left, bit-exact vs the oracle's op-by-op graph;
    per-channel scale and zero point included."""
    rng = np.random.default_rng(31)
    M, K, N = 4096, 3072, 768
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    w_zp = rng.integers(-8, 9, N).astype(np.int8)
    w_scale = rng.uniform(0.005, 0.03, N).astype(np.float32)
    bias = (0.02 * rng.standard_normal(N)).astype(np.float32)
    c = [rng.uniform(0.5, 2.0, N).astype(np.float32) for _ in range(3)]
    chain = [("Sub", c[0], True), ("Div", c[1], False), ("Mul", c[2], False)]
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    pw = ops.PackedWeight(dev(w))
    epi = [("Mul", (xs, dev(w_scale)), False), ("Add", dev(bias), False)]
    epi += [(op, dev(v), lhs) for op, v, lhs in chain]
    y = ops.gpu_qlinear(xq, pw, xzp, dev(w_zp), epilogue=epi, a_rowsum=rs)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    for r0, r1 in [(0, 24), (2048, 2056), (M - 16, M)]:
        ref = oracle.qlinear_graph(x, w, w_zp, w_scale, bias, chain, rows=(r0, r1))
        assert_f32_equal(y[r0:r1], ref["y"][r0:r1], "rows %d:%d" % (r0, r1))


def test_division_edge_values():
    """The GEMM epilogues divide by a column operand d with the correctly rounded IEEE
    division (__fdiv_rn), whatever the operands.  cfg2's shape (one 256x192 tile per CU) with
    a Mul before the Div that makes the numerators of chosen columns exactly +-0, subnormal,
    tiny, huge, inf or NaN, and divisors that are 0, tiny, huge, negative or have an all-ones
    significand: bit-exact against the oracle's op-by-op graph on every sampled row."""
    rng = np.random.default_rng(41)
    M, K, N = 4096, 768, 3072
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    w_scale = np.float32(0.01)
    bias = (0.05 * rng.standard_normal(N)).astype(np.float32)
    m = rng.uniform(0.5, 2.0, N).astype(np.float32)
    specials = [0.0, -0.0, 1e-40, -3e-39, 1e-35, 1e-19, 1e19, 1e30, -1e30, np.inf, -np.inf, np.nan]
    for i, v in enumerate(specials):  # every special numerator in a few columns of several tiles
        m[[7 + i, 200 + 3 * i, 1500 + i, N - 1 - i]] = v
    d = rng.uniform(0.25, 4.0, N).astype(np.float32)
    d[::5] *= -1.0
    d[11::97] = np.float32(1.9999999)  # all-ones significand
    d[3::211] = np.float32(-1.9999999)
    # out-of-range divisors in three column tiles only: the other tiles keep the fast path
    d[[400, 2000, 2001, 2900]] = np.array([0.0, 1e-30, -1e25, 5e-19], np.float32)
    chain = [("Mul", m, False), ("Div", d, False), ("Add", bias, False), ("Div", d[::-1].copy(), False)]
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    pw = ops.PackedWeight(dev(w))
    epi = [("Mul", (xs, dev(np.array(w_scale))), False), ("Add", dev(bias), False)]
    epi += [(op, dev(v), lhs) for op, v, lhs in chain]
    y = ops.gpu_qlinear(xq, pw, xzp, None, epilogue=epi, a_rowsum=rs)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    with np.errstate(all="ignore"):
        for r0, r1 in [(0, 40), (1024, 1040), (2040, 2056), (M - 40, M)]:
            ref = oracle.qlinear_graph(x, w, np.array(0, np.int8), np.array(w_scale), bias, chain,
                                       rows=(r0, r1))
            got, want = y[r0:r1], ref["y"][r0:r1]
            bad = int(np.count_nonzero(bits(got) != bits(want)))
            assert bad == 0, "rows %d:%d: %d of %d differ" % (r0, r1, bad, want.size)


def test_persistent_kernel_gelu_epilogue():
    """The operand-free erf / save steps through the persistent kernel (K = 2048)."""
    rng = np.random.default_rng(37)
    M, K, N = 256, 2048, 384
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    w_scale, bias = np.float32(0.01), (0.02 * rng.standard_normal(N)).astype(np.float32)
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    pw = ops.PackedWeight(dev(w))
    c0, c1, c2 = (dev(np.array(v, np.float32)) for v in (1.4142135, 1.0, 0.5))
    epi = [("Mul", (xs, dev(np.array(w_scale))), False), ("Add", dev(bias), False),
           ("Save", None, False), ("Div", c0, False), ("Erf", None, False), ("Add", c1, False),
           ("MulSaved", None, False), ("Mul", c2, False)]
    y = ops.gpu_qlinear(xq, pw, xzp, None, epilogue=epi, a_rowsum=rs)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    t = oracle.qlinear_graph(x, w, np.array(0, np.int8), np.array(w_scale), bias)["linear"]
    want = oracle.mul(oracle.mul(t, oracle.add(oracle.erf(oracle.div(t, np.float32(1.4142135))),
                                               np.float32(1.0))), np.float32(0.5))
    err = float(np.max(np.abs(y.astype(np.float64) - want)) / np.max(np.abs(want)))
    assert err < 1e-6, err


# One shape per tile configuration of the fused GEMM (gemm.hip picks the tile from the shape):
# 256x256 on 128-byte K rows and on 64-byte K rows, 256x192, 128x96, 64x96, 128x128, 64x64,
# and the register-staged kernel (K not a multiple of 16).
TILE_SHAPES = [
    ("256x256", 8192, 256, 4096),
    ("256x256 64-byte rows", 8192, 192, 4096),
    ("256x192", 4096, 256, 3072),
    ("128x96", 8192, 256, 768),
    ("64x96", 4096, 256, 768),
    ("128x128", 2048, 128, 2048),
    ("64x64", 128, 256, 768),
    ("register-staged", 300, 100, 512),
]


@pytest.mark.parametrize("name,M,K,N", TILE_SHAPES, ids=[s[0] for s in TILE_SHAPES])
@pytest.mark.parametrize("w_kind", ["i8", "u8 per-channel zp"])
def test_full_length_chain_every_tile(name, M, K, N, w_kind):
    """The longest epilogue the chain descriptor holds (ICX_MAX_CHAIN = 8 steps: dequant Mul,
    bias Add and six more), with per-column and scalar operands on both sides, IEEE
    divisions, and products of two factors in its last steps, on every tile configuration:
    each kernel loads the operands of its tile's columns before its main loop, spread over
    its waves (column groups x chain steps), so every step position and column group is
    exercised.  Bit-exact against the oracle run op by op, on sampled rows."""
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if w_kind == "i8":
        w = rng.integers(-127, 128, (K, N)).astype(np.int8)
        w_zp = np.array(0, np.int8)
    else:
        w = rng.integers(0, 256, (K, N)).astype(np.uint8)
        w_zp = rng.integers(120, 136, N).astype(np.uint8)
    w_scale = (0.01 + 0.01 * rng.random(N)).astype(np.float32)
    bias = (0.05 * rng.standard_normal(N)).astype(np.float32)
    col = [(0.5 + rng.random(N)).astype(np.float32) for _ in range(5)]
    s1, s2, s3 = (np.array(v, np.float32) for v in (1.25, 0.75, 3.0))
    chain = [("Mul", col[0], False), ("Sub", s1, True), ("Div", col[1], False),
             ("Add", col[2], True), ("Mul", (s2, col[3]), False), ("Div", (col[4], s3), True)]
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=K)
    epi = [("Mul", (xs, dev(w_scale)), False), ("Add", dev(bias), False)]
    epi += [(op, tuple(dev(t) for t in c) if isinstance(c, tuple) else dev(c), lhs) for op, c, lhs in chain]
    y = ops.gpu_qlinear(xq, ops.PackedWeight(dev(w)), xzp, dev(w_zp), epilogue=epi, a_rowsum=rs)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    ochain = [(op, oracle.mul(*c) if isinstance(c, tuple) else c, lhs) for op, c, lhs in chain]
    for r0, r1 in ((0, 8), (M // 2 - 3, M // 2 + 5), (M - 8, M)):
        ref = oracle.qlinear_graph(x, w, w_zp, w_scale, bias, ochain, rows=(r0, r1))
        assert_f32_equal(y[r0:r1], ref["y"][r0:r1], "%s %s rows %d:%d" % (name, w_kind, r0, r1))
