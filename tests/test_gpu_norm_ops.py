"""GPU: ReduceMean, Pow, Sqrt and the node-by-node LayerNorm they make up (an export below
opset 17 writes LayerNorm as ReduceMean -> Sub -> Pow(2) -> ReduceMean -> Add(eps) -> Sqrt ->
Div -> Mul(gamma) -> Add(beta); the reference's DistilBERT-INT8 does), against the oracle.

* ReduceMean and Sqrt: bit-exact (ndarray's summation order, one f32 division; correctly
  rounded sqrt).
* Pow: exponent 2 is the correctly rounded square, bit-exact against the oracle's square
  and within one ulp of the oracle's glibc powf (which misrounds ~0.07 % of squares); other
  exponents use the device powf, compared within two ulps.
* The DecomposedLayerNorm head (one LayerNorm launch) and the same nodes run one by one:
  bit-exact against the oracle with the square (Mul(c, c)), and within the north-star 1e-5
  (relative to the output magnitude) of the oracle with the reference's powf, at the encoder's
  full [32, 128, 768].
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import graphs, ops
from iconnx_amd.executor import GpuGraphExecutor
from iconnx_amd.onnx import ModelWriter, OnnxParser
from tests.golden_util import bits

pytestmark = pytest.mark.gpu
TOL = 1e-5  # north star: within 1e-5 relative to the output magnitude


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


def ulp_diff(a, b):
    return np.abs(bits(a).astype(np.int64) - bits(b).astype(np.int64))


@pytest.mark.parametrize("shape,axis", [((4096, 768), -1), ((33, 7), -1), ((5, 8), 1), ((3, 100), -1),
                                        ((2, 4096), -1), ((7, 13, 5), 1), ((6, 9, 4), 0),
                                        ((3, 5, 2, 4), 2), ((1, 16, 1), 1)])
def test_reduce_mean_bit_exact(shape, axis):
    x = (np.random.default_rng(len(shape) * 100 + shape[-1]).standard_normal(shape) * 2 + 0.3).astype(np.float32)
    for keep in (True, False):
        got = ops.gpu_reduce_mean(dev(x), [axis], keepdims=keep).cpu().numpy()
        want = oracle.reduce_mean(x, [axis], keepdims=keep)
        assert got.shape == want.shape
        assert np.array_equal(bits(got), bits(want)), (shape, axis, keep)


def test_reduce_mean_every_element_and_the_order():
    x = np.random.default_rng(3).standard_normal((64, 1000)).astype(np.float32)
    got = ops.gpu_reduce_mean(dev(x), None).cpu().numpy()
    assert got.shape == (1, 1)
    assert bits(got.reshape(())) == bits(oracle.reduce_mean(x, None))
    # the order-sensitive known answers (unrolled over the last axis, in order over another)
    v = np.array([2.0 ** 24] + [1.0] * 15, np.float32)
    assert ops.gpu_reduce_mean(dev(v.reshape(1, 16)), [-1]).item() == 2 ** 20 + 0.875
    assert ops.gpu_reduce_mean(dev(v.reshape(1, 16, 1)), [1]).item() == 2 ** 20
    assert ops.gpu_reduce_mean_axis(dev(v)).shape == (1,)


def test_pow_square_and_general_exponents():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((512, 768)) * 3).astype(np.float32)
    x[0, :6] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30]
    sq = ops.gpu_pow(dev(x), dev(np.float32(2.0))).cpu().numpy()
    assert np.array_equal(bits(sq), bits(oracle.mul(x, x)))  # the correctly rounded square
    ref = oracle.pow(x, np.float32(2.0))  # the reference's glibc powf
    fin = np.isfinite(ref)
    d = ulp_diff(sq[fin], ref[fin])
    assert int(d.max()) <= 1 and float(np.mean(d != 0)) < 5e-3
    # other exponents: a scalar, one per column, one per row (keepdims [rows, 1])
    ax = np.abs(x[1:]) + np.float32(0.5)
    for e in (np.float32(3.0), np.float32(0.5), np.float32(-1.5),
              rng.uniform(-2, 3, 768).astype(np.float32),
              rng.uniform(-2, 3, (511, 1)).astype(np.float32)):
        got = ops.gpu_pow(dev(ax), dev(e)).cpu().numpy()
        want = oracle.pow(ax, e)
        assert int(ulp_diff(got, want).max()) <= 2, np.shape(e)


def test_sqrt_bit_exact():
    x = (np.abs(np.random.default_rng(4).standard_normal(1 << 20)) * 1e3).astype(np.float32)
    x[:5] = [0.0, -0.0, 1.0, np.inf, 2.0]
    got = ops.gpu_sqrt(dev(x)).cpu().numpy()
    assert np.array_equal(bits(got), bits(oracle.sqrt(x)))
    assert np.isnan(ops.gpu_sqrt(dev(np.array([-1.0], np.float32))).item())


def ln_inputs(B=32, S=128, H=768, seed=1):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((B, S, H)) * 2).astype(np.float32)
    b = rng.standard_normal((B, S, H)).astype(np.float32)
    g = rng.uniform(0.9, 1.1, H).astype(np.float32)
    beta = (0.02 * rng.standard_normal(H)).astype(np.float32)
    return a, b, g, beta


def decomposed_graph(H, residual, affine, g, beta, eps, outputs=None, **kw):
    ex = GpuGraphExecutor()
    ex.add_input("a", [None, None, H])
    if residual:
        ex.add_input("b", [None, None, H])
    y = graphs.add_layer_norm_decomposed(ex, "a", "b" if residual else None, g if affine else None,
                                         beta if affine else None, eps, "ln", **kw)
    for o in outputs or [y]:
        ex.add_output(o)
    return ex, y


def check_against_oracle(got, a, b, g, beta, eps):
    sq = oracle.layer_norm_decomposed(a, g, beta, eps, residual=b, square=True)
    assert np.array_equal(bits(got), bits(sq))
    ref = oracle.layer_norm_decomposed(a, g, beta, eps, residual=b)  # the reference's powf
    assert rel_err(got, ref) < TOL
    return int(np.sum(bits(got) != bits(ref)))


@pytest.mark.parametrize("residual,affine,H", [(True, True, 768), (False, True, 768), (True, False, 768),
                                               (True, True, 1024), (True, True, 100), (False, False, 7)])
def test_decomposed_layer_norm_head(residual, affine, H):
    B, S = (32, 128) if H in (768, 1024) else (3, 50)
    a, b, g, beta = ln_inputs(B, S, H, seed=H)
    eps = 1e-12
    ex, y = decomposed_graph(H, residual, affine, g, beta, eps)
    entries, _ = ex.plan()
    live = [e for e in entries if e.kind != "Skip"]
    assert len(live) == 1 and live[0].pattern == "DecomposedLayerNorm"
    feeds = {"a": dev(a)}
    if residual:
        feeds["b"] = dev(b)
    got = ex.run(feeds, [y])[y]
    check_against_oracle(got, a, b if residual else None, g if affine else None,
                         beta if affine else None, eps)
    # the same arithmetic as the LayerNormalization operator
    ln = ops.gpu_layer_norm(dev(a), dev(g) if affine else None, dev(beta) if affine else None, eps,
                            residual=dev(b) if residual else None).cpu().numpy()
    assert np.array_equal(bits(got), bits(ln))


def test_decomposed_layer_norm_node_by_node():
    a, b, g, beta = ln_inputs(4, 128, 768, seed=5)
    eps = 1e-5
    ex, y = decomposed_graph(768, True, True, g, beta, eps, outputs=["ln.out", "ln.c", "ln.sq"])
    entries, _ = ex.plan()
    assert not any(e.pattern == "DecomposedLayerNorm" for e in entries)
    out = ex.run({"a": dev(a), "b": dev(b)}, ["ln.out", "ln.c", "ln.sq"])
    check_against_oracle(out["ln.out"], a, b, g, beta, eps)
    c = oracle.sub(oracle.add(a, b), oracle.reduce_mean(oracle.add(a, b), [-1]))
    assert np.array_equal(bits(out["ln.c"]), bits(c))
    assert int(ulp_diff(out["ln.sq"], oracle.pow(c, np.float32(2.0))).max()) <= 1


@pytest.mark.parametrize("axes_attr", [False, True])
def test_decomposed_layer_norm_from_an_onnx_file_with_constant_nodes(axes_attr, tmp_path):
    a, b, g, beta = ln_inputs(8, 128, 768, seed=11)
    w = ModelWriter(opset=13 if axes_attr else 18)
    w.add_input("a", [None, None, 768])
    w.add_input("b", [None, None, 768])
    y = graphs.add_layer_norm_decomposed(w, "a", "b", g, beta, 1e-12, "ln", axes_attr=axes_attr,
                                         constants=True)
    w.add_output(y)
    path = str(tmp_path / "ln.onnx")
    w.save(path)
    m = OnnxParser.parse_file(path)
    assert "Constant" in m.list_unique_operators()
    ex = GpuGraphExecutor.from_model(m)
    entries, _ = ex.plan()
    assert [e.pattern for e in entries if e.kind != "Skip"] == ["DecomposedLayerNorm"]
    got = ex.run({"a": a, "b": b}, [y])[y]
    check_against_oracle(got, a, b, g, beta, 1e-12)


def test_encoder_with_decomposed_layer_norms_equals_the_fused_encoder():
    """The full cfg3 encoder (6 layers, b32 s128) written with node-by-node LayerNorms runs
    bit-identically to the one with LayerNormalization nodes — including the DQLs that take
    their range from the norm kernel — and has the same number of launches."""
    x = graphs.encoder_input(32, 128)
    outs = []
    for ln in ("fused", "decomposed"):
        ex = GpuGraphExecutor()
        out, _, _ = graphs.encoder_graph(ex, layer_norm=ln)
        ex.add_output(out)
        outs.append(ex.run({"x": dev(x)}, [out])[out])
        entries, _ = ex.plan()
        if ln == "decomposed":
            assert sum(e.kind == "FusedHead" and e.pattern == "DecomposedLayerNorm" for e in entries) == 12
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
