"""GPU parity of the encoder's fp32 ops against the oracle.

LayerNormalization follows the reference's reduction order exactly and is compared bit for
bit; Softmax, Erf and the attention use the device exp (and the attention MFMA its own
summation order), so they are compared within a stated tolerance relative to the output
magnitude (the north star's 1e-5 bar for fp32 outputs, tighter where the op allows).
Transpose is exact.
"""
import itertools

import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import ops
from iconnx_amd._lib import IconnxError
from tests.golden_util import bits, tensor

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


@pytest.mark.parametrize("rows,cols", [(4096, 768), (4109, 768), (4100, 768), (3, 768), (97, 1024), (33, 3072), (5, 13), (64, 5)])
def test_layer_norm_bit_exact(rows, cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    y = host(ops.gpu_layer_norm(dev(x), dev(g), dev(b), eps=1e-12))
    assert np.array_equal(bits(y), bits(oracle.layer_norm(x, g, b, eps=1e-12)))
    y2 = host(ops.gpu_layer_norm(dev(x), dev(g), dev(b), eps=1e-5, residual=dev(r)))
    want = oracle.layer_norm(oracle.add(x, r), g, b, eps=1e-5)
    assert np.array_equal(bits(y2), bits(want))


@pytest.mark.parametrize("case", ["test_layer_normalization_3d_axis_negative_1_epsilon",
                                  "test_layer_normalization_4d_axis3"])
def test_layer_norm_goldens(goldens, case):
    c = goldens[case]
    x, g, b = (tensor(t) for t in c["inputs"])
    eps = c["attributes"].get("epsilon", 1e-5)
    y = host(ops.gpu_layer_norm(dev(x), dev(g), dev(b), eps=eps))
    assert np.array_equal(bits(y), bits(oracle.layer_norm(x, g, b, eps=eps)))
    assert rel_err(y, tensor(c["outputs"][0])) < 2e-6


@pytest.mark.parametrize("rows,cols", [(4096, 128), (7, 1000), (33, 5)])
def test_softmax_close(rows, cols):
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    y = host(ops.gpu_softmax(dev(x)))
    want = oracle.softmax(x)
    assert rel_err(y, want) < 2e-6
    assert float(np.mean(bits(y) == bits(want))) > 0.9  # mostly bit-identical


def test_erf_and_gelu_chain_close():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((512, 3072)) * 2).astype(np.float32)
    x[0, :6] = [0.0, -0.0, np.inf, -np.inf, 6.0, -6.0]
    e = host(ops.gpu_erf(dev(x)))
    assert float(np.max(np.abs(e - oracle.erf(x)))) < 2e-7
    assert e[0, 0] == 0.0 and e[0, 2] == 1.0 and e[0, 3] == -1.0
    # x * 0.5 * (1 + erf(x / sqrt 2)) as the exported graph evaluates it, node by node
    x = x[1:]  # finite inputs only (GELU(-inf) is NaN)
    c0, c1, c2 = np.float32(1.4142135), np.float32(1.0), np.float32(0.5)
    gelu = [("Save", None, False), ("Div", dev(np.array(c0)), False), ("Erf", None, False),
            ("Add", dev(np.array(c1)), False), ("MulSaved", None, False),
            ("Mul", dev(np.array(c2)), False)]
    y = host(ops.gpu_fused_chain(dev(x), gelu))
    want = oracle.mul(oracle.mul(x, oracle.add(oracle.erf(oracle.div(x, c0)), c1)), c2)
    assert rel_err(y, want) < 1e-6


def test_qlinear_with_gelu_epilogue():
    """FFN-up with the erf-GELU folded into the GEMM store; integer part exact, fp32 close."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((256, 768)).astype(np.float32)
    w = rng.integers(-127, 128, (768, 3072)).astype(np.int8)
    w_scale, bias = np.float32(0.01), (0.02 * rng.standard_normal(3072)).astype(np.float32)
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=768)
    pw = ops.PackedWeight(dev(w))
    c0, c1, c2 = (dev(np.array(v, np.float32)) for v in (1.4142135, 1.0, 0.5))
    epi = [("Mul", (xs, dev(np.array(w_scale))), False), ("Add", dev(bias), False),
           ("Save", None, False), ("Div", c0, False), ("Erf", None, False), ("Add", c1, False),
           ("MulSaved", None, False), ("Mul", c2, False)]
    y = host(ops.gpu_qlinear(xq, pw, xzp, None, epilogue=epi, a_rowsum=rs))
    ref = oracle.qlinear_graph(x, w, np.array(0, np.int8), np.array(w_scale), bias)
    t = ref["linear"]
    want = oracle.mul(oracle.mul(t, oracle.add(oracle.erf(oracle.div(t, np.float32(1.4142135))),
                                               np.float32(1.0))), np.float32(0.5))
    assert rel_err(y, want) < 1e-6


def test_gelu_epilogue_straight_line_matches_the_chain_loop():
    """The 8-op dequant + erf-GELU epilogue runs as straight-line code with the epilogue's
    erf (erf_gelu_scaled: FMA polynomial, hardware reciprocal) and its last three ops as
    one FMA and a product; the same ops through the per-op loop (the dequant and bias in the
    GEMM store, then the 6-op GELU chain as a separate launch, with the reference-order erf)
    agree within 5e-7 of the output's largest value, and both match the oracle within 1e-6 —
    the GELU multiplies erf by x where the two erf forms differ most (|x| < 0.06)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((512, 768)).astype(np.float32)
    w = rng.integers(-127, 128, (768, 3072)).astype(np.int8)
    w_scale, bias = np.float32(0.01), (0.02 * rng.standard_normal(3072)).astype(np.float32)
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=768)
    pw = ops.PackedWeight(dev(w))
    c0, c1, c2 = (dev(np.array(v, np.float32)) for v in (1.4142135, 1.0, 0.5))
    lin = [("Mul", (xs, dev(np.array(w_scale))), False), ("Add", dev(bias), False)]
    gelu = [("Save", None, False), ("Div", c0, False), ("Erf", None, False), ("Add", c1, False),
            ("MulSaved", None, False), ("Mul", c2, False)]
    y8 = host(ops.gpu_qlinear(xq, pw, xzp, None, epilogue=lin + gelu, a_rowsum=rs))
    t = ops.gpu_qlinear(xq, pw, xzp, None, epilogue=lin, a_rowsum=rs)
    y2 = host(ops.gpu_fused_chain(t, gelu))
    assert rel_err(y8, y2) < 5e-7
    th = host(t)
    want = oracle.mul(oracle.mul(th, oracle.add(oracle.erf(oracle.div(th, np.float32(1.4142135))),
                                                np.float32(1.0))), np.float32(0.5))
    assert rel_err(y8, want) < 1e-6 and rel_err(y2, want) < 1e-6


def test_qlinear_with_gelu_epilogue_narrow_tile():
    """The erf-GELU epilogue on the 128x96 tile (4096 x 768 x 768: 256 tiles)."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((4096, 768)).astype(np.float32)
    w = rng.integers(-127, 128, (768, 768)).astype(np.int8)
    w_scale, bias = np.float32(0.01), (0.02 * rng.standard_normal(768)).astype(np.float32)
    xq, xs, xzp, rs = ops.gpu_dynamic_quantize_linear(dev(x), rowsum_row_len=768)
    pw = ops.PackedWeight(dev(w))
    c0, c1, c2 = (dev(np.array(v, np.float32)) for v in (1.4142135, 1.0, 0.5))
    epi = [("Mul", (xs, dev(np.array(w_scale))), False), ("Add", dev(bias), False),
           ("Save", None, False), ("Div", c0, False), ("Erf", None, False), ("Add", c1, False),
           ("MulSaved", None, False), ("Mul", c2, False)]
    y = host(ops.gpu_qlinear(xq, pw, xzp, None, epilogue=epi, a_rowsum=rs))
    t = oracle.qlinear_graph(x, w, np.array(0, np.int8), np.array(w_scale), bias)["linear"]
    want = oracle.mul(oracle.mul(t, oracle.add(oracle.erf(oracle.div(t, np.float32(1.4142135))),
                                               np.float32(1.0))), np.float32(0.5))
    assert rel_err(y, want) < 1e-6


def test_transpose_exact():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    for perm in itertools.permutations(range(4)):
        assert np.array_equal(host(ops.gpu_transpose(dev(x), perm)), x.transpose(perm))
    u = rng.integers(0, 256, (32, 128, 12, 64)).astype(np.uint8)
    assert np.array_equal(host(ops.gpu_transpose(dev(u), (0, 2, 1, 3))), u.transpose(0, 2, 1, 3))
    with pytest.raises(IconnxError):
        ops.gpu_transpose(dev(x), (0, 0, 1, 2))


@pytest.mark.parametrize("shape_a,shape_b", [((3, 4), (4, 3)), ((384, 128, 64), (384, 64, 128)),
                                             ((2, 100, 77), (77, 33)), ((5, 65, 129), (5, 129, 67))])
def test_matmul_f32_close(shape_a, shape_b):
    rng = np.random.default_rng(len(shape_a))
    a = rng.standard_normal(shape_a).astype(np.float32)
    b = rng.standard_normal(shape_b).astype(np.float32)
    assert rel_err(host(ops.gpu_matmul_f32(dev(a), dev(b))), oracle.matmul_f32(a, b)) < 1e-5


def attention_oracle(q, k, v, H, scale, scale_q):
    """The decomposed BERT attention subgraph, op by op through the oracle."""
    B, S, HD = q.shape
    D = HD // H
    split = lambda t: oracle.transpose(t.reshape(B, S, H, D), (0, 2, 1, 3))
    qh, kh, vh = split(q), split(k), split(v)
    if scale_q:
        qh = oracle.div(qh, np.float32(scale))
    kt = oracle.transpose(kh, (0, 1, 3, 2))
    s = oracle.matmul_f32(qh.reshape(B * H, S, D), kt.reshape(B * H, D, S)).reshape(B, H, S, S)
    if not scale_q:
        s = oracle.div(s, np.float32(scale))
    p = oracle.softmax(s)
    ctx = oracle.matmul_f32(p.reshape(B * H, S, S), vh.reshape(B * H, S, D)).reshape(B, H, S, D)
    return oracle.transpose(ctx, (0, 2, 1, 3)).reshape(B, S, HD)


@pytest.mark.parametrize("B,S,H,scale_q", [(4, 128, 12, False), (2, 50, 3, True), (32, 128, 12, False)])
def test_fused_attention_close(B, S, H, scale_q):
    rng = np.random.default_rng(S + H)
    q, k, v = (rng.standard_normal((B, S, H * 64)).astype(np.float32) for _ in range(3))
    out = host(ops.gpu_attention(dev(q), dev(k), dev(v), H, 8.0, scale_div=True, scale_q=scale_q))
    assert rel_err(out, attention_oracle(q, k, v, H, 8.0, scale_q)) < 1e-5


@pytest.mark.parametrize("B,S,H,scale,scale_q", [(3, 97, 5, 3.0, False), (1, 128, 8, 0.7, True)])
def test_fused_attention_other_scales_and_grids(B, S, H, scale, scale_q):
    """A scale that is not a power of two (the correctly rounded division path), a query
    split whose block count is not a multiple of 16 (plain pairing of the two halves), and
    one that is (the XCD-local pairing) with an odd sequence length."""
    rng = np.random.default_rng(B * 1000 + S)
    q, k, v = (rng.standard_normal((B, S, H * 64)).astype(np.float32) for _ in range(3))
    out = host(ops.gpu_attention(dev(q), dev(k), dev(v), H, scale, scale_div=True, scale_q=scale_q))
    assert rel_err(out, attention_oracle(q, k, v, H, scale, scale_q)) < 1e-5


@pytest.mark.parametrize("B,S,H,scale_q", [(2, 129, 3, False), (2, 384, 12, True), (1, 512, 16, False),
                                           (3, 1000, 2, True)])
def test_fused_attention_long_sequences(B, S, H, scale_q):
    """Past 128 keys: 128-key chunks with a running softmax (attention_long_kernel), 64
    queries per block; (batch, head) counts that fill whole groups of 8 (the XCD-local block
    order) and that do not."""
    rng = np.random.default_rng(S * 7 + H)
    q, k, v = (rng.standard_normal((B, S, H * 64)).astype(np.float32) for _ in range(3))
    out = host(ops.gpu_attention(dev(q), dev(k), dev(v), H, 8.0, scale_div=True, scale_q=scale_q))
    assert rel_err(out, attention_oracle(q, k, v, H, 8.0, scale_q)) < 1e-5


def test_attention_rejects_unsupported_shapes():
    q = torch.zeros((1, 10, 32), device="cuda")  # head size 32
    with pytest.raises(IconnxError, match="unsupported"):
        ops.gpu_attention(q, q, q, 1, 8.0)
    q = torch.zeros((1, 8193, 64), device="cuda")  # past the longest sequence
    with pytest.raises(IconnxError, match="unsupported"):
        ops.gpu_attention(q, q, q, 1, 8.0)
