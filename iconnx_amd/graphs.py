"""Builders for the quantized-linear subgraphs the synthetic configs run through
GpuGraphExecutor.

The node pattern is the one ONNX Runtime's dynamic quantization emits for a Linear /
MatMul, and the one the reference executes node by node (src/graph_executor.rs:356-432;
src/cuda/executor/layout.rs:978-1095, 1254-1271; elementwise.rs:54-200):

    DynamicQuantizeLinear(x)                -> x_q u8, x_scale f32 [], x_zp u8 []
    Mul(x_scale, w_scale)                   -> scale
    MatMulInteger(x_q, W, x_zp, w_zp)       -> acc i32
    Cast(acc, to=FLOAT)                     -> acc_f
    Mul(acc_f, scale)                       -> y0
    Add(y0, bias)                           -> y1
    [Mul / Add / Sub / Div (y, constant)]*  -> y
"""
import numpy as np

from . import configs


def add_dynamic_quantize(ex, x, prefix):
    """DynamicQuantizeLinear node; returns (x_q, x_scale, x_zp) tensor names.  Several
    linears may share one (the Q / K / V projections of an attention block do)."""
    outs = [prefix + ".x_q", prefix + ".x_scale", prefix + ".x_zp"]
    ex.add_node(prefix + ".dql", "DynamicQuantizeLinear", [x], outs)
    return tuple(outs)


def add_quantized_linear(ex, x, w, w_zp, w_scale, bias, chain=(), prefix="ql", dql=None):
    """Add one quantized linear (+ chain) reading tensor ``x``; returns the output name.

    ``w`` int8/uint8 [K, N]; ``w_zp`` scalar or [N] (None: absent input); ``w_scale``
    scalar or [N]; ``bias`` [N] or None; ``chain`` items are (op, constant) or
    (op, constant, constant_is_lhs).  ``dql`` reuses an existing quantization of x."""
    xq, xs, xzp = dql if dql is not None else add_dynamic_quantize(ex, x, prefix)
    p = prefix
    ex.add_initializer(p + ".W", np.asarray(w))
    ex.add_initializer(p + ".w_scale", np.asarray(w_scale, np.float32))
    mm_in = [xq, p + ".W", xzp]
    if w_zp is not None:
        ex.add_initializer(p + ".w_zp", np.asarray(w_zp))
        mm_in.append(p + ".w_zp")
    ex.add_node(p + ".scale", "Mul", [xs, p + ".w_scale"], [p + ".scale"])
    ex.add_node(p + ".mmi", "MatMulInteger", mm_in, [p + ".acc"])
    ex.add_node(p + ".cast", "Cast", [p + ".acc"], [p + ".acc_f"], {"to": 1})
    ex.add_node(p + ".dequant", "Mul", [p + ".acc_f", p + ".scale"], [p + ".linear0"])
    y = p + ".linear0"
    if bias is not None:
        ex.add_initializer(p + ".bias", np.asarray(bias, np.float32))
        ex.add_node(p + ".bias_add", "Add", [y, p + ".bias"], [p + ".linear"])
        y = p + ".linear"
    for i, item in enumerate(chain):
        op, const = item[0], item[1]
        lhs = bool(item[2]) if len(item) > 2 else False
        cname = "%s.c%d" % (p, i)
        ex.add_initializer(cname, np.asarray(const, np.float32))
        out = "%s.chain%d" % (p, i)
        ex.add_node("%s.%s%d" % (p, op.lower(), i), op, [cname, y] if lhs else [y, cname], [out])
        y = out
    return y


def config_graph(ex, cfg, x_name="x", x_shape=None):
    """The linear configs (cfg1 / cfg2 / cfg4) as a graph on executor ``ex``; returns
    (output name, host data dict).  The input is declared with its batch and sequence
    dims dynamic unless ``x_shape`` is given."""
    d = configs.make(cfg)
    shape = x_shape if x_shape is not None else [None, None, d["x"].shape[-1]]
    ex.add_input(x_name, shape)
    w_zp = d["w_zp"]
    y = add_quantized_linear(ex, x_name, d["w"], w_zp, d["w_scale"], d["bias"], d["chain"],
                             prefix=cfg)
    return y, d
