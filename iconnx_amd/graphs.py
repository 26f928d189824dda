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
from .synth import seeded_normal, seeded_uniform


def add_dynamic_quantize(ex, x, prefix):
    """DynamicQuantizeLinear node; returns (x_q, x_scale, x_zp) tensor names.  Several
    linears may share one (the Q / K / V projections of an attention block do)."""
    outs = [prefix + ".x_q", prefix + ".x_scale", prefix + ".x_zp"]
    ex.add_node(prefix + ".dql", "DynamicQuantizeLinear", [x], outs)
    return tuple(outs)


def add_gelu(ex, x, prefix):
    """x * 0.5 * (1 + erf(x / sqrt 2)) as PyTorch exports it: Div, Erf, Add, Mul(x, .),
    Mul(., 0.5).  Returns the output name."""
    p = prefix
    for name, val in (("sqrt2", 1.4142135381698608), ("one", 1.0), ("half", 0.5)):
        ex.add_initializer("%s.%s" % (p, name), np.array(val, np.float32))
    ex.add_node(p + ".div", "Div", [x, p + ".sqrt2"], [p + ".d"])
    ex.add_node(p + ".erf", "Erf", [p + ".d"], [p + ".e"])
    ex.add_node(p + ".add1", "Add", [p + ".e", p + ".one"], [p + ".a"])
    ex.add_node(p + ".mulx", "Mul", [x, p + ".a"], [p + ".m"])
    ex.add_node(p + ".mulhalf", "Mul", [p + ".m", p + ".half"], [p + ".gelu"])
    return p + ".gelu"


def add_quantized_linear(ex, x, w, w_zp, w_scale, bias, chain=(), prefix="ql", dql=None,
                         gelu=False):
    """Add one quantized linear (+ chain) reading tensor ``x``; returns the output name.

    ``w`` int8/uint8 [K, N]; ``w_zp`` scalar or [N] (None: absent input); ``w_scale``
    scalar or [N]; ``bias`` [N] or None; ``chain`` items are (op, constant) or
    (op, constant, constant_is_lhs); ``gelu`` appends an erf-GELU.  ``dql`` reuses an
    existing quantization of x."""
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
    if gelu:
        y = add_gelu(ex, y, p + ".gelu")
    return y


def add_dequantize_linear_head(ex, a, a_zp, w, scale, zp, bias, axis=1, prefix="dq"):
    """MatMulInteger(a, W, a_zp) -> DequantizeLinear(acc, scale, zp, axis) [-> Add(bias)]:
    the form of a quantized linear whose graph dequantizes the int32 accumulator with a
    DequantizeLinear instead of Cast + Mul.  ``a_zp`` a tensor name or None; ``zp`` an Int32
    scalar / [N] or None; ``scale`` scalar or [N].  Returns the output name."""
    p = prefix
    ex.add_initializer(p + ".W", np.asarray(w))
    ex.add_initializer(p + ".scale", np.asarray(scale, np.float32))
    mm_in = [a, p + ".W"] + ([a_zp] if a_zp is not None else [])
    ex.add_node(p + ".mmi", "MatMulInteger", mm_in, [p + ".acc"])
    dq_in = [p + ".acc", p + ".scale"]
    if zp is not None:
        ex.add_initializer(p + ".zp", np.asarray(zp, np.int32))
        dq_in.append(p + ".zp")
    ex.add_node(p + ".dequant", "DequantizeLinear", dq_in, [p + ".linear0"], {"axis": axis})
    y = p + ".linear0"
    if bias is not None:
        ex.add_initializer(p + ".bias", np.asarray(bias, np.float32))
        ex.add_node(p + ".bias_add", "Add", [y, p + ".bias"], [p + ".linear"])
        y = p + ".linear"
    return y


def add_quantized_embedding(ex, ids, table, scale, zp, prefix="emb"):
    """DistilBERT-INT8's embedding front end: Gather(UInt8 table [vocab, hidden], ids) ->
    DequantizeLinear(., scale, zp) -> f32 [..., hidden].  Returns the output name."""
    p = prefix
    ex.add_initializer(p + ".table", np.asarray(table, np.uint8))
    ex.add_initializer(p + ".scale", np.asarray(scale, np.float32))
    ex.add_initializer(p + ".zp", np.asarray(zp, np.uint8))
    ex.add_node(p + ".gather", "Gather", [p + ".table", ids], [p + ".q"], {"axis": 0})
    ex.add_node(p + ".dequant", "DequantizeLinear", [p + ".q", p + ".scale", p + ".zp"], [p + ".out"])
    return p + ".out"


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


# ---------------------------------------------------------------------------------------
# DistilBERT-shaped encoder: 6 layers, hidden 768, 12 heads of 64,
# FFN 3072, random-init weights, every linear quantized dynamically.
# ---------------------------------------------------------------------------------------
ENCODER = dict(layers=6, hidden=768, heads=12, ffn=3072, batch=32, seq=128, eps=1e-12)


def encoder_layer_params(layer, hidden=768, ffn=3072, seed=3000):
    """Seeded random-init weights of one layer: int8 weights uniform in [-127, 127] with a
    per-tensor scale of 5e-4 (std ~0.036 = 1/sqrt(768)) and zero point 0, biases and
    LayerNorm shifts ~ N(0, 0.02), LayerNorm gains ~ U(0.9, 1.1)."""
    base = seed + 100 * layer
    p = {}
    shapes = {"q": (hidden, hidden), "k": (hidden, hidden), "v": (hidden, hidden),
              "o": (hidden, hidden), "ff1": (hidden, ffn), "ff2": (ffn, hidden)}
    for i, (name, (K, N)) in enumerate(shapes.items()):
        p[name] = dict(w=configs.weight_i8(K, N, base + 10 * i),
                       w_zp=np.array(0, np.int8), w_scale=np.array(5e-4, np.float32),
                       bias=(0.02 * seeded_normal(N, base + 10 * i + 1).astype(np.float64)).astype(np.float32))
    for i, name in enumerate(("ln1", "ln2")):
        p[name] = dict(scale=seeded_uniform(hidden, base + 80 + 2 * i, 0.9, 1.1),
                       bias=(0.02 * seeded_normal(hidden, base + 81 + 2 * i).astype(np.float64)).astype(np.float32))
    return p


def add_self_attention(ex, q, k, v, heads, head_dim, prefix):
    """The exported BERT attention subgraph over [B, S, H*D] tensors q, k, v (DistilBERT
    scales q by 1/sqrt(D) before the product).  Returns the [B, S, H*D] context name."""
    p = prefix
    ex.add_initializer(p + ".split", np.array([0, 0, heads, head_dim], np.int64))
    ex.add_initializer(p + ".merge", np.array([0, 0, heads * head_dim], np.int64))
    ex.add_initializer(p + ".sqrt_d", np.array(np.sqrt(head_dim), np.float32))
    for t, perm in ((q, [0, 2, 1, 3]), (k, [0, 2, 3, 1]), (v, [0, 2, 1, 3])):
        tag = {q: "q", k: "k", v: "v"}[t]
        ex.add_node("%s.reshape_%s" % (p, tag), "Reshape", [t, p + ".split"], ["%s.%s4" % (p, tag)])
        ex.add_node("%s.transpose_%s" % (p, tag), "Transpose", ["%s.%s4" % (p, tag)],
                    ["%s.%st" % (p, tag)], {"perm": perm})
    ex.add_node(p + ".scale_q", "Div", [p + ".qt", p + ".sqrt_d"], [p + ".qs"])
    ex.add_node(p + ".scores", "MatMul", [p + ".qs", p + ".kt"], [p + ".s"])
    ex.add_node(p + ".softmax", "Softmax", [p + ".s"], [p + ".p"], {"axis": -1})
    ex.add_node(p + ".context", "MatMul", [p + ".p", p + ".vt"], [p + ".c"])
    ex.add_node(p + ".transpose_c", "Transpose", [p + ".c"], [p + ".ct"], {"perm": [0, 2, 1, 3]})
    ex.add_node(p + ".reshape_c", "Reshape", [p + ".ct", p + ".merge"], [p + ".ctx"])
    return p + ".ctx"


def add_layer_norm(ex, x, residual, scale, bias, eps, prefix):
    """LayerNormalization(Add(x, residual)); returns the output name."""
    p = prefix
    ex.add_initializer(p + ".gamma", np.asarray(scale, np.float32))
    ex.add_initializer(p + ".beta", np.asarray(bias, np.float32))
    ex.add_node(p + ".residual", "Add", [x, residual], [p + ".sum"])
    ex.add_node(p + ".norm", "LayerNormalization", [p + ".sum", p + ".gamma", p + ".beta"],
                [p + ".out"], {"axis": -1, "epsilon": float(eps)})
    return p + ".out"


def add_layer_norm_decomposed(ex, x, residual, scale, bias, eps, prefix, axes_attr=False,
                              constants=False):
    """The LayerNorm an export below opset 17 writes node by node (PyTorch's exporter; the
    reference's DistilBERT-INT8): [Add(x, residual) ->] ReduceMean -> Sub -> Pow(., 2) ->
    ReduceMean -> Add(., eps) -> Sqrt -> Div [-> Mul(., gamma)] [-> Add(., beta)].
    ``axes_attr``: the means' axes as an attribute (opsets before 18) instead of an Int64
    input; ``constants``: the exponent, epsilon and axes as Constant nodes (for a ModelWriter,
    whose file ``from_model`` reads back); ``scale`` / ``bias`` None: no Mul / Add.  Returns
    the output name."""
    p = prefix
    if residual is not None:
        ex.add_node(p + ".residual", "Add", [x, residual], [p + ".sum"])
        x = p + ".sum"

    def const(name, arr):
        if constants:
            ex.add_node(name + ".const", "Constant", [], [name], {"value": arr})
        else:
            ex.add_initializer(name, arr)

    const(p + ".two", np.array(2.0, np.float32))
    const(p + ".eps", np.array(eps, np.float32))
    attrs = {"keepdims": 1}
    if axes_attr:
        attrs["axes"] = [-1]
        mean_in = lambda t: [t]  # noqa: E731
    else:
        const(p + ".axes", np.array([-1], np.int64))
        mean_in = lambda t: [t, p + ".axes"]  # noqa: E731
    ex.add_node(p + ".mean", "ReduceMean", mean_in(x), [p + ".mu"], attrs)
    ex.add_node(p + ".sub", "Sub", [x, p + ".mu"], [p + ".c"])
    ex.add_node(p + ".pow", "Pow", [p + ".c", p + ".two"], [p + ".sq"])
    ex.add_node(p + ".var", "ReduceMean", mean_in(p + ".sq"), [p + ".v"], attrs)
    ex.add_node(p + ".add_eps", "Add", [p + ".v", p + ".eps"], [p + ".ve"])
    ex.add_node(p + ".sqrt", "Sqrt", [p + ".ve"], [p + ".sd"])
    ex.add_node(p + ".div", "Div", [p + ".c", p + ".sd"], [p + ".n"])
    y = p + ".n"
    if scale is not None:
        ex.add_initializer(p + ".gamma", np.asarray(scale, np.float32))
        ex.add_node(p + ".mul_gamma", "Mul", [y, p + ".gamma"], [p + ".scaled"])
        y = p + ".scaled"
    if bias is not None:
        ex.add_initializer(p + ".beta", np.asarray(bias, np.float32))
        ex.add_node(p + ".add_beta", "Add", [y, p + ".beta"], [p + ".out"])
        y = p + ".out"
    return y


def add_encoder_layer(ex, x, params, heads, eps, prefix, layer_norm="fused", **ln_kw):
    """One post-LN transformer layer; returns a dict of the layer's tensor names.
    ``layer_norm``: "fused" (LayerNormalization nodes) or "decomposed" (the node-by-node form
    of add_layer_norm_decomposed, with ``ln_kw`` passed to it)."""
    p = prefix
    norm = add_layer_norm if layer_norm == "fused" else (
        lambda *a: add_layer_norm_decomposed(ex, *a[1:], **ln_kw))
    hidden = params["q"]["w"].shape[0]
    lin = lambda name, inp, **kw: add_quantized_linear(
        ex, inp, params[name]["w"], params[name]["w_zp"], params[name]["w_scale"],
        params[name]["bias"], prefix="%s.%s" % (p, name), **kw)
    dql = add_dynamic_quantize(ex, x, p + ".qkv")
    q, k, v = (lin(n, x, dql=dql) for n in ("q", "k", "v"))
    ctx = add_self_attention(ex, q, k, v, heads, hidden // heads, p + ".attn")
    o = lin("o", ctx)
    x1 = norm(ex, o, x, params["ln1"]["scale"], params["ln1"]["bias"], eps, p + ".ln1")
    h = lin("ff1", x1, gelu=True)
    f = lin("ff2", h)
    x2 = norm(ex, f, x1, params["ln2"]["scale"], params["ln2"]["bias"], eps, p + ".ln2")
    return dict(x=x, xq=dql[0], q=q, k=k, v=v, ctx=ctx, o=o, x1=x1, h=h, f=f, out=x2)


def encoder_graph(ex, layers=6, heads=12, hidden=768, ffn=3072, eps=1e-12, x_name="x",
                  x_shape=None, seed=3000, layer_norm="fused", **ln_kw):
    """The DistilBERT-shaped encoder on executor ``ex``; ``layer_norm`` = "decomposed" writes
    every LayerNorm node by node (ReduceMean / Sub / Pow / Sqrt / Div ...) as an export below
    opset 17 does.  Returns (output name, per-layer tensor names, per-layer params)."""
    ex.add_input(x_name, x_shape if x_shape is not None else [None, None, hidden])
    x, names, params = x_name, [], []
    for l in range(layers):
        prm = encoder_layer_params(l, hidden, ffn, seed)
        t = add_encoder_layer(ex, x, prm, heads, eps, "L%d" % l, layer_norm, **ln_kw)
        names.append(t)
        params.append(prm)
        x = t["out"]
    return x, names, params


# ---------------------------------------------------------------------------------------
# The same encoder as an exported DistilBERT-INT8 writes it (torch.onnx of Hugging Face's
# DistilBertModel, opset 13-16, then ONNX Runtime's dynamic quantization — the form whose op
# list the reference's INT8 design names, docs/superpowers/specs/2026-04-25-ws4-int8-
# quantization-design.md:171): Int64 input_ids / attention_mask; the UINT8 word table through
# Gather + DequantizeLinear, position ids sliced from a [1, 512] constant up to the sequence
# length; every reshape target assembled at run time from Shape / Gather / Unsqueeze / Concat;
# the key transposed twice; the padding mask as Equal / Reshape / Expand / Where(finfo.min)
# on the scores; LayerNorms node by node (ReduceMean / Sub / Pow / Sqrt / Div / Mul / Add).
# ---------------------------------------------------------------------------------------
F32_MIN = np.float32(np.finfo(np.float32).min)


def add_self_attention_export(ex, x, q, k, v, mask, heads, head_dim, prefix, cond=None):
    """MultiHeadSelfAttention over [B, S, H*D] projections q, k, v of ``x`` with the Int64
    padding mask ``mask`` [B, S] (0 = padding), as exported; ``cond`` (a Bool tensor name)
    replaces the mask's Equal / Reshape / Expand as the Where's condition.  Returns the
    context name."""
    p = prefix
    cst = lambda n, a: ex.add_initializer("%s.%s" % (p, n), np.asarray(a))  # noqa: E731
    cst("i0", np.array(0, np.int64))
    cst("i1", np.array(1, np.int64))
    cst("ax0", np.array([0], np.int64))
    cst("m1", np.array([-1], np.int64))
    cst("one", np.array([1], np.int64))
    cst("nh", np.array([heads], np.int64))
    cst("dh", np.array([head_dim], np.int64))
    cst("hid", np.array([heads * head_dim], np.int64))
    cst("zero", np.array(0, np.int64))
    cst("sqrt_d", np.array(np.sqrt(head_dim), np.float32))
    cst("fmin", F32_MIN)
    ext = {x, q, k, v, mask, cond}

    def n(name, op, ins, outs, attrs=None):  # names local to this block get the prefix
        ex.add_node("%s.%s" % (p, name), op, [i if i in ext else "%s.%s" % (p, i) for i in ins],
                    ["%s.%s" % (p, o) for o in outs], attrs)
    # bs = x.size(0), k_length = x.size(1)
    n("shape_x", "Shape", [x], ["xs"])
    n("bs", "Gather", ["xs", "i0"], ["bs"], {"axis": 0})
    n("klen", "Gather", ["xs", "i1"], ["klen"], {"axis": 0})
    n("bs_u", "Unsqueeze", ["bs", "ax0"], ["bs_u"])
    n("klen_u", "Unsqueeze", ["klen", "ax0"], ["klen_u"])
    n("split", "Concat", ["bs_u", "m1", "nh", "dh"], ["split"], {"axis": 0})
    for t, tag in ((q, "q"), (k, "k"), (v, "v")):  # x.view(bs, -1, H, D).transpose(1, 2)
        n("view_" + tag, "Reshape", [t, "split"], [tag + "4"])
        n("tr_" + tag, "Transpose", [tag + "4"], [tag + "t"], {"perm": [0, 2, 1, 3]})
    n("scale_q", "Div", ["qt", "sqrt_d"], ["qs"])
    n("tr_k2", "Transpose", ["kt"], ["kT"], {"perm": [0, 1, 3, 2]})
    n("scores", "MatMul", ["qs", "kT"], ["s"])
    # mask = (mask == 0).view(bs, 1, 1, k_length).expand_as(scores)
    if cond is None:
        n("mask_eq", "Equal", [mask, "zero"], ["meq"])
        n("mask_shape", "Concat", ["bs_u", "one", "one", "klen_u"], ["mshape"], {"axis": 0})
        n("mask_view", "Reshape", ["meq", "mshape"], ["m4"])
        n("shape_s", "Shape", ["s"], ["ss"])
        n("mask_expand", "Expand", ["m4", "ss"], ["mx"])
    n("masked_fill", "Where", [cond if cond is not None else "mx", "fmin", "s"], ["sm"])
    n("softmax", "Softmax", ["sm"], ["pr"], {"axis": -1})
    n("context", "MatMul", ["pr", "vt"], ["c"])
    n("tr_c", "Transpose", ["c"], ["ct"], {"perm": [0, 2, 1, 3]})
    n("merge", "Concat", ["bs_u", "m1", "hid"], ["merge"], {"axis": 0})
    n("unshape", "Reshape", ["ct", "merge"], ["ctx"])
    return p + ".ctx"


def add_embeddings_export(ex, ids, word_table, scale, zp, pos_table, ln, eps, prefix):
    """DistilBERT's Embeddings: Gather(UInt8 word table, input_ids) -> DequantizeLinear, plus
    Gather(position table, position_ids[:, :seq_len]) (a Slice of a [1, max_pos] Int64
    constant), then a LayerNorm node by node.  Returns the output name."""
    p = prefix
    we = add_quantized_embedding(ex, ids, word_table, scale, zp, p + ".word")
    ex.add_initializer(p + ".position_ids", np.arange(pos_table.shape[0], dtype=np.int64).reshape(1, -1))
    ex.add_initializer(p + ".pos_table", np.asarray(pos_table, np.float32))
    ex.add_initializer(p + ".i1", np.array(1, np.int64))
    ex.add_initializer(p + ".z", np.array([0], np.int64))
    ex.add_initializer(p + ".ax1", np.array([1], np.int64))
    ex.add_node(p + ".shape_ids", "Shape", [ids], [p + ".ids_shape"])
    ex.add_node(p + ".seq_len", "Gather", [p + ".ids_shape", p + ".i1"], [p + ".slen"], {"axis": 0})
    ex.add_node(p + ".seq_len_u", "Unsqueeze", [p + ".slen", p + ".z"], [p + ".slen_u"])
    ex.add_node(p + ".pos_slice", "Slice", [p + ".position_ids", p + ".z", p + ".slen_u", p + ".ax1"], [p + ".pid"])
    ex.add_node(p + ".pos_gather", "Gather", [p + ".pos_table", p + ".pid"], [p + ".pemb"], {"axis": 0})
    ex.add_node(p + ".sum", "Add", [we, p + ".pemb"], [p + ".e"])
    return add_layer_norm_decomposed(ex, p + ".e", None, ln["scale"], ln["bias"], eps, p + ".ln")


def export_encoder_graph(ex, layers=6, heads=12, hidden=768, ffn=3072, eps=1e-12, vocab=30522,
                         max_pos=512, seed=3000, per_channel=False, opset17_norm=False):
    """DistilBERT-INT8 as exported (see above) on executor or writer ``ex``: inputs
    ``input_ids`` and ``attention_mask`` (Int64 [B, S]).  The layers carry the weights of
    encoder_graph's; the embedding tables are seeded too.  ``per_channel``: every weight
    with a seeded per-column scale [N] and an Int8 zero point [N] of zeros (ONNX Runtime's
    per_channel quantization of symmetric int8 weights); ``opset17_norm``: the layers'
    LayerNorms as LayerNormalization nodes (an export at opset 17 or later).  Returns (output
    name, names dict with the embedding output and per-layer tensor names, per-layer params,
    embedding params)."""
    ex.add_input("input_ids", [None, None], 7)
    ex.add_input("attention_mask", [None, None], 7)
    emb = dict(word=seeded_uniform(vocab * hidden, seed - 7, 0.0, 255.0).astype(np.uint8).reshape(vocab, hidden),
               scale=np.float32(0.004), zp=np.uint8(128),
               pos=(0.02 * seeded_normal(max_pos * hidden, seed - 6).astype(np.float64)).astype(np.float32)
               .reshape(max_pos, hidden),
               ln=dict(scale=seeded_uniform(hidden, seed - 5, 0.9, 1.1),
                       bias=(0.02 * seeded_normal(hidden, seed - 4).astype(np.float64)).astype(np.float32)))
    x = add_embeddings_export(ex, "input_ids", emb["word"], emb["scale"], emb["zp"], emb["pos"], emb["ln"], eps,
                              "emb")
    names, params = dict(emb=x, layers=[]), []
    for l in range(layers):
        prm = encoder_layer_params(l, hidden, ffn, seed)
        if per_channel:
            for i, nm in enumerate(("q", "k", "v", "o", "ff1", "ff2")):
                N = prm[nm]["w"].shape[1]
                prm[nm]["w_scale"] = seeded_uniform(N, seed + 100 * l + 50 + i, 3e-4, 7e-4)
                prm[nm]["w_zp"] = np.zeros(N, np.int8)
        p = "L%d" % l
        lin = lambda name, inp, **kw: add_quantized_linear(  # noqa: E731
            ex, inp, prm[name]["w"], prm[name]["w_zp"], prm[name]["w_scale"], prm[name]["bias"],
            prefix="%s.%s" % (p, name), **kw)
        norm = (lambda a, r, prm_ln, tag: add_layer_norm(ex, a, r, prm_ln["scale"], prm_ln["bias"], eps, tag)) \
            if opset17_norm else \
            (lambda a, r, prm_ln, tag: add_layer_norm_decomposed(ex, a, r, prm_ln["scale"], prm_ln["bias"], eps, tag))
        dql = add_dynamic_quantize(ex, x, p + ".qkv")
        q, k, v = (lin(nm, x, dql=dql) for nm in ("q", "k", "v"))
        ctx = add_self_attention_export(ex, x, q, k, v, "attention_mask", heads, hidden // heads, p + ".attn")
        o = lin("o", ctx)
        x1 = norm(o, x, prm["ln1"], p + ".ln1")
        h = lin("ff1", x1, gelu=True)
        f = lin("ff2", h)
        x2 = norm(f, x1, prm["ln2"], p + ".ln2")
        names["layers"].append(dict(x=x, xq=dql[0], q=q, k=k, v=v, ctx=ctx, o=o, x1=x1, h=h, f=f, out=x2))
        params.append(prm)
        x = x2
    return x, names, params, emb


def export_inputs(batch=32, seq=128, vocab=30522, seed=2998):
    """Seeded input_ids (uniform over the vocabulary) and an attention mask whose rows keep a
    seeded number of leading tokens (the rest is padding, 0)."""
    ids = (seeded_uniform(batch * seq, seed, 0.0, float(vocab)).astype(np.int64) % vocab).reshape(batch, seq)
    lens = 1 + (seeded_uniform(batch, seed + 1, 0.0, float(seq)).astype(np.int64) % seq)
    lens[0] = seq  # one unpadded row
    mask = (np.arange(seq)[None, :] < lens[:, None]).astype(np.int64)
    return ids, mask


def encoder_input(batch=32, seq=128, hidden=768, seed=2999):
    """Input embeddings ~ N(0, 1), [batch, seq, hidden] float32."""
    return seeded_normal(batch * seq * hidden, seed).reshape(batch, seq, hidden)


def write_model(path, build, *args, **kwargs):
    """Serialise a graph built by one of the builders above into an .onnx file:
    ``build(writer, *args, **kwargs)`` records the nodes (e.g. ``config_graph`` with a config
    name, or ``encoder_graph``) and its first return value is the graph output.  Returns the
    builder's return value."""
    from .onnx import ModelWriter

    w = ModelWriter()
    ret = build(w, *args, **kwargs)
    out = ret[0] if isinstance(ret, tuple) else ret
    w.add_output(out)
    w.save(path)
    return ret
