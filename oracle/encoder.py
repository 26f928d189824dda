"""The DistilBERT-shaped encoder restated op by op through the oracle — TEST
INFRASTRUCTURE ONLY (the checker for tests/ and the CPU baseline of bench.py).

Each function follows the node pattern that iconnx_amd.graphs builds and that the reference
executes node by node (src/graph_executor.rs:356-432): DynamicQuantizeLinear, MatMulInteger,
Cast, Mul (x_scale * w_scale, then the dequant), Add (bias), the erf-GELU (Div, Erf, Add,
Mul, Mul), the attention (Reshape, Transpose, Div, MatMul, [the padding mask,] Softmax,
MatMul, Transpose, Reshape) and LayerNormalization(Add(.)).
"""
import numpy as np

from . import (add, cast_i32_f32, div, dynamic_quantize_linear, erf, layer_norm, matmul_f32,
               matmul_integer, mul, softmax, transpose)


def dequant_linear(xq, xs, xzp, p, rows=None, gelu=False):
    """Linear from an already quantized input: MatMulInteger -> Cast -> Mul(x_scale *
    w_scale) -> Add(bias) [-> GELU], rows [r0, r1) of the flattened input (all if None)."""
    x2 = xq.reshape(-1, xq.shape[-1])
    per_col = np.size(p["w_zp"]) > 1  # a per-column weight zero point (the extension's form)
    acc = matmul_integer(x2, p["w"], xzp, p["w_zp"], per_column_b_zp=per_col, rows=rows)
    if rows is not None:
        acc = acc[rows[0]:rows[1]]
    y = add(mul(cast_i32_f32(acc), mul(xs, p["w_scale"])), p["bias"])
    return gelu_ref(y) if gelu else y


def gelu_ref(t):
    d = div(t, np.float32(1.4142135381698608))
    return mul(mul(t, add(erf(d), np.float32(1.0))), np.float32(0.5))


def attention_ref(q, k, v, heads, scale=8.0, scale_q=True, mask=None, cond=None):
    """The exported self-attention subgraph over [B, S, H*D] tensors; ``mask`` (Int64 [B, S],
    0 = padding) adds the export's masked_fill: Where(Expand(Reshape(Equal(mask, 0),
    [B, 1, 1, S]), scores' shape), finfo(f32).min, scores) before the Softmax; ``cond`` (Bool,
    broadcasting over [B, H, S, S]) is that Where's condition given directly."""
    B, S, HD = q.shape
    D = HD // heads
    split = lambda t: transpose(np.ascontiguousarray(t).reshape(B, S, heads, D), (0, 2, 1, 3))  # noqa: E731
    qh, kh, vh = split(q), split(k), split(v)
    if scale_q:
        qh = div(qh, np.float32(scale))
    kt = transpose(kh, (0, 1, 3, 2))
    s = matmul_f32(qh.reshape(B * heads, S, D), kt.reshape(B * heads, D, S)).reshape(B, heads, S, S)
    if not scale_q:
        s = div(s, np.float32(scale))
    if mask is not None or cond is not None:
        from . import layout
        if cond is None:
            m4 = layout.equal(np.asarray(mask, np.int64), np.array(0, np.int64)).reshape(B, 1, 1, S)
            cond = layout.expand(m4, s.shape)
        s = layout.where(cond, np.float32(np.finfo(np.float32).min), s)
    pr = softmax(s)
    ctx = matmul_f32(pr.reshape(B * heads, S, S), vh.reshape(B * heads, S, D)).reshape(B, heads, S, D)
    return transpose(ctx, (0, 2, 1, 3)).reshape(B, S, HD)


def add_layer_norm_ref(a, b, p, eps):
    return layer_norm(add(a, b), p["scale"], p["bias"], eps=eps)


def layer_ref(x, params, heads, eps):
    """One full layer; returns every intermediate the graph names."""
    xq, xs, xzp = dynamic_quantize_linear(x)
    out = {"xq": xq}
    for n in ("q", "k", "v"):
        out[n] = dequant_linear(xq, xs, xzp, params[n]).reshape(x.shape[:-1] + (-1,))
    out["ctx"] = attention_ref(out["q"], out["k"], out["v"], heads, np.sqrt(x.shape[-1] // heads))
    cq, cs, cz = dynamic_quantize_linear(out["ctx"])
    out["o"] = dequant_linear(cq, cs, cz, params["o"]).reshape(x.shape)
    out["x1"] = add_layer_norm_ref(out["o"], x, params["ln1"], eps)
    hq, hs, hz = dynamic_quantize_linear(out["x1"])
    out["h"] = dequant_linear(hq, hs, hz, params["ff1"], gelu=True).reshape(x.shape[:-1] + (-1,))
    fq, fs, fz = dynamic_quantize_linear(out["h"])
    out["f"] = dequant_linear(fq, fs, fz, params["ff2"]).reshape(x.shape)
    out["out"] = add_layer_norm_ref(out["f"], out["x1"], params["ln2"], eps)
    return out
