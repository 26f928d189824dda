"""Host-side lowering of the graph executor (no GPU): topological sort, dead-node
elimination, the fusion decision and zero-point folding.

Counterparts in the reference: the fusion-detection tests of
src/ir/passes/elementwise_fusion (matchers.rs:363-409 MulAdd, :483-514 DivMul; exact
two-op chains, static operands) and the lowering tests of src/ir/lowering.rs.  The
QuantizedLinear head is new here: the reference leaves MatMulInteger -> Cast -> Mul -> Add
unfused (src/cuda/inference/fusion/detection.rs:98-102).
"""
import numpy as np
import pytest

from iconnx_amd import configs, graphs
from iconnx_amd._lib import IconnxError
from iconnx_amd.executor import GpuGraphExecutor


def heads(entries):
    return [e for e in entries if e.kind == "FusedHead"]


def by_node(entries):
    return {e.node: e for e in entries}


def linear(ex, w_zp=0, chain=(), prefix="l", x="x", dql=None, w_dtype=np.int8, N=16):
    rng = np.random.default_rng(0)
    w = rng.integers(-127, 128, size=(8, N)).astype(w_dtype)
    zp = None if w_zp is None else np.asarray(w_zp, dtype=w_dtype)
    return graphs.add_quantized_linear(ex, x, w, zp, np.float32(0.02),
                                       rng.standard_normal(N).astype(np.float32), chain,
                                       prefix=prefix, dql=dql)


def test_quantized_linear_head_and_zero_point_folding():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y = linear(ex, w_zp=0)
    ex.add_output(y)
    entries, rowsums = ex.plan()
    h = heads(entries)
    assert len(h) == 1 and h[0].pattern == "QuantizedLinear"
    assert h[0].op_type == "MatMulInteger" and h[0].out == y
    assert h[0].steps == 2  # Mul(acc_f, x_scale*w_scale) and Add(bias)
    assert h[0].wzp_folded  # all-zero int8 weight zero point
    assert rowsums == []  # no weight zero point left, int8 weights: no row sums needed
    kinds = {e.node: e.kind for e in entries}
    assert kinds["l.dql"] == "Regular"
    for n in ("l.scale", "l.cast", "l.dequant", "l.bias_add"):
        assert kinds[n] == "Skip", n


def test_nonzero_weight_zero_point_requests_dql_row_sums():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y = linear(ex, w_zp=np.arange(-8, 8))
    ex.add_output(y)
    entries, rowsums = ex.plan()
    (h,) = heads(entries)
    assert not h.wzp_folded
    assert rowsums == ["l.x_q"]


def test_uint8_weights_need_row_sums_even_without_zero_point():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    rng = np.random.default_rng(1)
    y = graphs.add_quantized_linear(ex, "x", rng.integers(0, 256, (8, 16)).astype(np.uint8),
                                    None, np.float32(0.1), None, prefix="u")
    ex.add_output(y)
    entries, rowsums = ex.plan()
    (h,) = heads(entries)
    assert h.steps == 1 and rowsums == ["u.x_q"]


def test_cfg2_chain_is_absorbed_into_the_gemm_epilogue():
    ex = GpuGraphExecutor()
    y, _ = graphs.config_graph(ex, "cfg2")
    ex.add_output(y)
    entries, _ = ex.plan()
    (h,) = heads(entries)
    assert h.pattern == "QuantizedLinear" and h.steps == 6 and h.out == y
    assert sum(e.kind != "Skip" for e in entries) == 2  # DQL + fused GEMM


def test_requested_intermediate_output_stops_the_fusion():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y = linear(ex, chain=[("Mul", np.ones(16)), ("Add", np.zeros(16))])
    ex.add_output("l.linear")  # the pre-chain value must materialise
    ex.add_output(y)
    entries, _ = ex.plan()
    hs = {h.pattern: h for h in heads(entries)}
    assert hs["QuantizedLinear"].out == "l.linear" and hs["QuantizedLinear"].steps == 2
    assert hs["MulAdd"].out == y


def test_fan_out_of_the_accumulator_prevents_fusion():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y = linear(ex)
    ex.add_node("extra", "Cast", ["l.acc"], ["acc_copy"], {"to": 1})
    ex.add_output(y)
    ex.add_output("acc_copy")
    entries, _ = ex.plan()
    e = by_node(entries)
    assert e["l.mmi"].kind == "Regular"
    assert e["l.cast"].kind == "Regular"
    # the dequant Mul -> bias Add pair is still a static-operand chain? No: the dequant
    # Mul's operand is the runtime scale, so only plain ops remain.
    assert not [h for h in heads(entries) if h.pattern == "QuantizedLinear"]


@pytest.mark.parametrize("ops,pattern", [
    (("Mul", "Add"), "MulAdd"), (("Add", "Mul"), "AddMul"), (("Sub", "Mul"), "SubMul"),
    (("Div", "Mul"), "DivMul"), (("Mul", "Add", "Div"), "ElementwiseChain"),
    (("Div", "Sub"), "ElementwiseChain"),
])
def test_elementwise_chain_patterns(ops, pattern):
    ex = GpuGraphExecutor()
    ex.add_input("x", [4, 6])
    cur = "x"
    for i, op in enumerate(ops):
        ex.add_initializer("c%d" % i, np.full(6, 1.5, np.float32))
        ex.add_node("n%d" % i, op, [cur, "c%d" % i], ["t%d" % i])
        cur = "t%d" % i
    ex.add_output(cur)
    entries, _ = ex.plan()
    (h,) = heads(entries)
    assert h.pattern == pattern and h.steps == len(ops) and h.out == cur


def test_single_binary_op_and_runtime_operands_stay_regular():
    ex = GpuGraphExecutor()
    ex.add_input("x", [4, 6])
    ex.add_input("z", [4, 6])
    ex.add_initializer("c", np.ones(6, np.float32))
    ex.add_node("a", "Mul", ["x", "c"], ["t0"])
    ex.add_node("b", "Add", ["t0", "z"], ["t1"])  # runtime operand: not a static chain
    ex.add_output("t1")
    entries, _ = ex.plan()
    assert not heads(entries)
    assert [e.kind for e in entries] == ["Regular", "Regular"]


def test_chain_longer_than_eight_splits():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    chain = [("Mul", np.full(16, 1.01)), ("Add", np.full(16, 0.01))] * 5  # 10 ops
    y = linear(ex, chain=chain)
    ex.add_output(y)
    entries, _ = ex.plan()
    hs = heads(entries)
    assert [h.pattern for h in hs] == ["QuantizedLinear", "ElementwiseChain"]
    assert hs[0].steps == 8  # dequant Mul + bias Add + 6 chain ops
    assert hs[1].steps == 4 and hs[1].out == y


def test_shared_dql_for_three_projections():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    dql = graphs.add_dynamic_quantize(ex, "x", "attn")
    outs = [linear(ex, w_zp=np.arange(16) % 3, prefix=p, dql=dql) for p in ("q", "k", "v")]
    for o in outs:
        ex.add_output(o)
    entries, rowsums = ex.plan()
    assert [h.pattern for h in heads(entries)] == ["QuantizedLinear"] * 3
    assert rowsums == ["attn.x_q"]
    assert sum(e.op_type == "DynamicQuantizeLinear" and e.kind == "Regular" for e in entries) == 1


def _siblings(n, N=256, w_zps=None, chains=None, w_scales=None, dtypes=None, K=8):
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, K])
    dql = graphs.add_dynamic_quantize(ex, "x", "s")
    rng = np.random.default_rng(1)
    outs = []
    for i in range(n):
        dt = dtypes[i] if dtypes else np.int8
        w = rng.integers(0 if dt == np.uint8 else -127, 128, size=(K, N)).astype(dt)
        zp = np.asarray(w_zps[i] if w_zps else 0).astype(dt)
        sc = w_scales[i] if w_scales else np.float32(0.01 * (i + 1))
        outs.append(graphs.add_quantized_linear(ex, "x", w, zp, sc, rng.standard_normal(N).astype(np.float32),
                                                chains[i] if chains else (), prefix="h%d" % i, dql=dql))
    for o in outs:
        ex.add_output(o)
    entries, _ = ex.plan()
    return [next(e.group for e in entries if e.node == "h%d.mmi" % i) for i in range(n)]


def test_sibling_linears_group_into_one_gemm():
    assert _siblings(3) == ["h0.mmi"] * 3
    assert _siblings(2, N=512) == ["h0.mmi"] * 2
    # at most four segments per launch; the rest group among themselves
    assert _siblings(6) == ["h0.mmi"] * 4 + ["h4.mmi"] * 2
    assert _siblings(5) == ["h0.mmi"] * 4 + [None]
    # scalar and per-column scales mix (each expands to a column vector)
    assert _siblings(3, w_scales=[np.float32(0.01), np.full(256, 0.02, np.float32), np.float32(0.03)]) == \
        ["h0.mmi"] * 3
    # a lone head, widths that are not a multiple of 256, or unequal widths: no group
    assert _siblings(1) == [None]
    assert _siblings(3, N=16) == [None] * 3
    assert _siblings(3, N=384) == [None] * 3
    # a non-zero weight zero point keeps the head out; the other two still group
    assert _siblings(3, w_zps=[0, 3, 0]) == ["h0.mmi", None, "h0.mmi"]
    # a head whose chain has other steps stays single
    ch = [(), [("Mul", np.float32(2.0))], ()]
    assert _siblings(3, chains=ch) == ["h0.mmi", None, "h0.mmi"]
    # same step kinds with different constants group (constants become columns)
    ch = [[("Mul", np.float32(2.0))], [("Mul", np.float32(3.0))], [("Mul", np.arange(256, dtype=np.float32))]]
    assert _siblings(3, chains=ch) == ["h0.mmi"] * 3
    # weights of different dtypes do not share a launch
    assert _siblings(2, dtypes=[np.int8, np.uint8], w_zps=[0, 0]) == [None, None]


def test_insertion_order_does_not_matter():
    ref = GpuGraphExecutor()
    ref.add_input("x", [None, 8])
    y = linear(ref)
    ref.add_output(y)
    want, _ = ref.plan()

    # same graph, nodes added in reverse order
    class Recorder:
        def __init__(self):
            self.calls = []

        def __getattr__(self, name):
            return lambda *a, **k: self.calls.append((name, a, k))

    rec = Recorder()
    linear(rec)
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    inits = [c for c in rec.calls if c[0] == "add_initializer"]
    nodes = [c for c in rec.calls if c[0] == "add_node"]
    for name, a, k in inits + nodes[::-1]:
        getattr(ex, name)(*a, **k)
    ex.add_output(y)
    got, _ = ex.plan()
    assert [(e.op_type, e.kind, e.pattern, e.steps) for e in heads(got)] == \
        [(e.op_type, e.kind, e.pattern, e.steps) for e in heads(want)]
    order = [e.node for e in got if e.kind != "Skip"]
    assert order.index("l.dql") < order.index("l.mmi")


def test_dead_nodes_are_dropped_and_sinks_become_outputs():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y = linear(ex)
    ex.add_node("unused", "Mul", ["x", "l.bias"], ["dead"])
    ex.add_output(y)
    entries, _ = ex.plan()
    assert "unused" not in by_node(entries)
    # no requested outputs: every sink is live
    ex2 = GpuGraphExecutor()
    ex2.add_input("x", [None, 8])
    linear(ex2)
    ex2.add_initializer("k", np.ones(16, np.float32))
    ex2.add_node("side", "Mul", ["x", "k"], ["side_out"])
    entries2, _ = ex2.plan()
    assert "side" in by_node(entries2)


def test_cycle_is_an_error():
    ex = GpuGraphExecutor()
    ex.add_input("x", [2])
    ex.add_node("a", "Add", ["x", "t1"], ["t0"])
    ex.add_node("b", "Add", ["t0", "x"], ["t1"])
    ex.add_output("t1")
    with pytest.raises(IconnxError, match="cycle"):
        ex.plan()


def test_configs_plan_to_one_fused_gemm_each():
    for cfg in ("cfg1", "cfg2", "cfg4"):
        ex = GpuGraphExecutor()
        y, d = graphs.config_graph(ex, cfg)
        ex.add_output(y)
        entries, rowsums = ex.plan()
        live = [e for e in entries if e.kind != "Skip"]
        assert [e.op_type for e in live] == ["DynamicQuantizeLinear", "MatMulInteger"], cfg
        assert live[1].pattern == "QuantizedLinear"
        per_channel_zp = np.any(np.asarray(d["w_zp"]) != 0)
        assert live[1].wzp_folded == (not per_channel_zp), cfg
        assert rowsums == (["%s.x_q" % cfg] if per_channel_zp else []), cfg
        assert live[1].steps == 2 + len(d["chain"]), cfg


# ---- encoder patterns -------------------------------------------------------------------
def test_encoder_layer_plan():
    ex = GpuGraphExecutor()
    out, names, _ = graphs.encoder_graph(ex, layers=2)
    ex.add_output(out)
    entries, rowsums = ex.plan()
    live = [(e.op_type, e.pattern, e.steps) for e in entries if e.kind != "Skip"]
    layer = [("DynamicQuantizeLinear", "-", 0)] + [("MatMulInteger", "QuantizedLinear", 2)] * 3 + [
        ("Softmax", "Attention", 0), ("DynamicQuantizeLinear", "-", 0),
        ("MatMulInteger", "QuantizedLinear", 2), ("LayerNormalization", "AddLayerNorm", 0),
        ("DynamicQuantizeLinear", "-", 0), ("MatMulInteger", "QuantizedLinear", 8),
        ("DynamicQuantizeLinear", "-", 0), ("MatMulInteger", "QuantizedLinear", 2),
        ("LayerNormalization", "AddLayerNorm", 0)]
    assert live == layer * 2
    assert rowsums == []  # zero int8 weight zero points are folded
    heads = {e.node: e for e in entries if e.kind == "FusedHead"}
    assert heads["L0.ff1.mmi"].out == "L0.ff1.gelu.gelu"
    # Q / K / V run as one GEMM led by the first; O and the FFN linears stay single
    for l in (0, 1):
        for p in ("q", "k", "v"):
            assert heads["L%d.%s.mmi" % (l, p)].group == "L%d.q.mmi" % l
        for p in ("o", "ff1", "ff2"):
            assert heads["L%d.%s.mmi" % (l, p)].group is None
    assert heads["L1.attn.softmax"].out == "L1.attn.ctx"
    skipped = {e.node for e in entries if e.kind == "Skip"}
    for n in ("L0.attn.reshape_q", "L0.attn.transpose_k", "L0.attn.scale_q", "L0.attn.scores",
              "L0.attn.context", "L0.attn.transpose_c", "L0.attn.reshape_c", "L0.ln1.residual",
              "L0.ff1.gelu.erf", "L0.ff1.gelu.mulx"):
        assert n in skipped, n


def _gelu_graph(with_add):
    ex = GpuGraphExecutor()
    ex.add_input("x", [4, 16])
    src = "x"
    if with_add:
        ex.add_initializer("b", np.ones(16, np.float32))
        ex.add_node("bias", "Add", ["x", "b"], ["xb"])
        src = "xb"
    y = graphs.add_gelu(ex, src, "g")
    ex.add_output(y)
    return ex, y


@pytest.mark.parametrize("with_add,steps", [(False, 6), (True, 7)])
def test_standalone_gelu_chain(with_add, steps):
    ex, y = _gelu_graph(with_add)
    entries, _ = ex.plan()
    (h,) = heads(entries)
    assert h.pattern == "Gelu" and h.steps == steps and h.out == y
    assert sum(e.kind != "Skip" for e in entries) == 1


def test_attention_needs_its_intermediates_private():
    ex = GpuGraphExecutor()
    for n in "qkv":
        ex.add_input(n, [None, None, 128])
    ctx = graphs.add_self_attention(ex, "q", "k", "v", 2, 64, "att")
    ex.add_output(ctx)
    assert [h.pattern for h in heads(ex.plan()[0])] == ["Attention"]
    ex.add_output("att.s")  # the scores must materialise: no fusion
    entries, _ = ex.plan()
    assert not [h for h in heads(entries) if h.pattern == "Attention"]
    assert [e.op_type for e in entries if e.kind != "Skip"].count("MatMul") == 2


def test_layer_norm_without_add_is_regular_and_attrs_are_checked():
    ex = GpuGraphExecutor()
    ex.add_input("x", [2, 8])
    ex.add_initializer("g", np.ones(8, np.float32))
    ex.add_initializer("b", np.zeros(8, np.float32))
    ex.add_node("ln", "LayerNormalization", ["x", "g", "b"], ["y"], {"epsilon": 1e-6})
    ex.add_output("y")
    entries, _ = ex.plan()
    assert [(e.op_type, e.kind) for e in entries] == [("LayerNormalization", "Regular")]
    L = ex._L
    assert L.icx_graph_set_node_attr_float(ex._g, b"missing", b"epsilon", 1.0) != 0
    assert b"missing" in L.icx_last_error()


def test_encoder_dql_ranges_come_from_producers():
    """Every DynamicQuantizeLinear of the encoder except the first reads a tensor written by
    a LayerNorm, attention or quantized-linear head, which leaves its min / max for it."""
    from iconnx_amd import graphs

    ex = GpuGraphExecutor()
    out, names, _ = graphs.encoder_graph(ex, layers=2)
    got = set(ex.range_inputs())
    want = set()
    for l, t in enumerate(names):
        if l > 0:
            want.add(t["x"])   # the previous layer's LayerNorm output
        want |= {t["ctx"], t["x1"], t["h"]}
    assert got == want
    assert names[0]["x"] not in got  # the graph input has no producing kernel


def _two_linears(w2_dtype=np.int8, w2_zp=0, w1_dtype=np.int8, w1_zp=0, extra_reader=False):
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, 8])
    y1 = linear(ex, w_zp=w1_zp, prefix="l1", w_dtype=w1_dtype, N=8)
    y2 = linear(ex, w_zp=w2_zp, prefix="l2", x=y1, w_dtype=w2_dtype)
    ex.add_output(y2)
    if extra_reader:
        ex.add_initializer("one", np.ones(8, np.float32))
        ex.add_node("tap", "Mul", [y1, "one"], ["tapped"])
        ex.add_output("tapped")
    return ex, y1


def test_quantized_output_selection():
    """A quantized-linear head whose output only a DynamicQuantizeLinear reads may write that
    DQL's outputs itself: Int8 weight without zero point, no other reader, the f32 tensor not
    requested, and no GEMM reading row sums of the quantized tensor."""
    ex, y1 = _two_linears()
    assert ex.quantized_outputs() == ({y1: "l2.dql"}, 0)
    # the consumer's weight is uint8: it reads the DQL's row sums, which only the DQL writes
    assert _two_linears(w2_dtype=np.uint8)[0].quantized_outputs()[0] == {}
    assert _two_linears(w2_zp=np.arange(16) - 8)[0].quantized_outputs()[0] == {}
    # the producer's weight keeps a row term (uint8 or a nonzero zero point)
    assert _two_linears(w1_dtype=np.uint8)[0].quantized_outputs()[0] == {}
    assert _two_linears(w1_zp=np.arange(8) - 4)[0].quantized_outputs()[0] == {}
    # another reader of the f32 output (the fused head then stops before it)
    assert _two_linears(extra_reader=True)[0].quantized_outputs()[0] == {}
    # the f32 output requested
    ex, y1 = _two_linears()
    ex.add_output(y1)
    assert ex.quantized_outputs()[0] == {}


def test_quantized_input_selection():
    """A DynamicQuantizeLinear whose three outputs only one quantized-linear head reads runs
    inside that head's launch: Int8 weight without zero point, f32 output, an input no head
    leaves the range of.  Not for a weight with a row term, not when another node reads one
    of the DQL's outputs, not for a head that quantizes its own output, not for a DQL its
    producer already writes; the options turn it off."""
    def one(**kw):
        ex = GpuGraphExecutor()
        ex.add_input("x", [None, 8])
        y = linear(ex, prefix="l", **kw)
        ex.add_output(y)
        return ex, y
    ex, y = one()
    assert ex.quantized_inputs() == ({y: "l.dql"}, 0)
    entries, _ = ex.plan()
    assert by_node(entries)["l.dql"].kind == "Regular"  # the plan entry stays (it runs nothing)
    ex.set_option("quantized_inputs", False)
    assert ex.quantized_inputs()[0] == {}
    ex.set_option("quantized_inputs", True)
    ex.set_option("quantized_outputs", False)
    assert ex.quantized_inputs()[0] == {}
    with pytest.raises(IconnxError):
        ex.set_option("quantized_inputs", 3)
    assert one(w_dtype=np.uint8)[0].quantized_inputs()[0] == {}
    assert one(w_zp=np.arange(16) - 8)[0].quantized_inputs()[0] == {}
    ex, y = one()
    ex.add_initializer("one", np.ones((), np.float32))
    ex.add_node("tap", "Mul", ["l.x_scale", "one"], ["tapped"])  # another reader of the scale
    ex.add_output("tapped")
    assert ex.quantized_inputs()[0] == {}
    # two linears in a row: the first quantizes its own output (so it is no quantized-input
    # head), and the second's DQL is written by the first
    assert _two_linears()[0].quantized_inputs()[0] == {}


def test_encoder_heads_quantize_their_own_outputs():
    """The FFN-up's erf-GELU output feeds only the FFN-down's DQL and the attention context
    only the output projection's DQL: those producers quantize their own outputs; the
    LayerNorm outputs (read by a DQL and by the next residual Add) do not.  The option
    "quantized_outputs" off plans none of them."""
    ex = GpuGraphExecutor()
    out, names, _ = graphs.encoder_graph(ex, layers=2)
    ex.add_output(out)
    planned, _ = ex.quantized_outputs()
    assert set(planned) == {t[k] for k in ("h", "ctx") for t in names}
    entries, _ = ex.plan()
    dql_of = {e.node: e for e in entries if e.op_type == "DynamicQuantizeLinear"}
    assert all(d in dql_of for d in planned.values())
    ex.set_option("quantized_outputs", False)
    assert ex.quantized_outputs()[0] == {}
    ex.set_option("quantized_outputs", True)
    assert set(ex.quantized_outputs()[0]) == set(planned)
    with pytest.raises(IconnxError):
        ex.set_option("quantized_outputs", 2)
    with pytest.raises(IconnxError):
        ex.set_option("no_such_option", 1)


def _dq_graph(rank, scale_n, axis, zp):
    ex = GpuGraphExecutor()
    ex.add_input("a", [None] * (rank - 1) + [8])
    ex.add_input("a_zp", [])
    rng = np.random.default_rng(3)
    w = rng.integers(-127, 128, (8, 16)).astype(np.int8)
    scale = np.float32(0.01) if scale_n == 1 else rng.uniform(0.01, 0.02, 16).astype(np.float32)
    y = graphs.add_dequantize_linear_head(ex, "a", "a_zp", w, scale, zp, np.zeros(16, np.float32), axis=axis)
    ex.add_output(y)
    return ex, y


@pytest.mark.parametrize("rank,scale_n,axis,zp,steps", [
    (2, 1, 1, np.int32(5), 3),                  # Sub(zp), Mul(scale), Add(bias)
    (2, 16, 1, None, 2),                         # per-column scale, axis 1 = last of [M, N]
    (2, 16, 1, np.zeros(16, np.int32), 2),       # all-zero zero point: no Sub
    (3, 16, 2, np.arange(16, dtype=np.int32), 3),
    (3, 16, -1, None, 2),
    (3, 1, 1, np.int32(-2), 3),                  # per-tensor: any axis
])
def test_matmul_integer_dequantize_linear_is_one_head(rank, scale_n, axis, zp, steps):
    ex, y = _dq_graph(rank, scale_n, axis, zp)
    entries, _ = ex.plan()
    (h,) = heads(entries)
    assert h.pattern == "QuantizedLinear" and h.op_type == "MatMulInteger" and h.out == y
    assert h.steps == steps
    kinds = by_node(entries)
    assert kinds["dq.dequant"].kind == "Skip" and kinds["dq.bias_add"].kind == "Skip"


def test_dequantize_linear_along_a_non_last_axis_stays_unfused():
    """A [N] scale along axis 1 of a 3-D [B, S, N] accumulator scales rows, not columns."""
    ex, _ = _dq_graph(3, 16, 1, None)
    entries, _ = ex.plan()
    assert heads(entries) == [] or all(h.op_type != "MatMulInteger" for h in heads(entries))
    assert by_node(entries)["dq.dequant"].kind == "Regular"


# ---- the node-by-node LayerNorm (ReduceMean / Sub / Pow / Sqrt / Div ...) --------------------
LN_NODES = ("mean", "sub", "pow", "var", "add_eps", "sqrt", "div", "mul_gamma", "add_beta")


def _decomposed_ln(residual=True, affine=True, axes_attr=False, outputs=None, exponent=2.0,
                   hidden=768):
    ex = GpuGraphExecutor()
    ex.add_input("a", [None, None, hidden])
    ex.add_input("b", [None, None, hidden])
    g = np.ones(hidden, np.float32) if affine else None
    y = graphs.add_layer_norm_decomposed(ex, "a", "b" if residual else None, g, g, 1e-12, "ln",
                                         axes_attr=axes_attr)
    if exponent != 2.0:
        ex.add_initializer("ln.two", np.array(exponent, np.float32))
    for o in outputs or [y]:
        ex.add_output(o)
    return ex, y


@pytest.mark.parametrize("axes_attr", [False, True])
@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("affine", [False, True])
def test_decomposed_layer_norm_is_one_head(axes_attr, residual, affine):
    ex, y = _decomposed_ln(residual, affine, axes_attr)
    entries, _ = ex.plan()
    (h,) = heads(entries)
    assert h.pattern == "DecomposedLayerNorm" and h.op_type == "ReduceMean" and h.out == y
    kinds = by_node(entries)
    expect = [n for n in LN_NODES if affine or n not in ("mul_gamma", "add_beta")]
    for n in expect[1:] + (["residual"] if residual else []):
        assert kinds["ln." + n].kind == "Skip", n
    assert len([e for e in entries if e.kind != "Skip"]) == 1


def test_decomposed_layer_norm_stops_where_an_intermediate_is_requested():
    ex, y = _decomposed_ln(outputs=["ln.out", "ln.c"])
    entries, _ = ex.plan()
    assert not any(e.pattern == "DecomposedLayerNorm" for e in entries)
    ops = [e.op_type for e in entries if e.kind != "Skip"]
    for op in ("ReduceMean", "Pow", "Sqrt"):
        assert op in ops  # run node by node


def test_decomposed_layer_norm_needs_exponent_two():
    ex, y = _decomposed_ln(exponent=3.0)
    entries, _ = ex.plan()
    assert not any(e.pattern == "DecomposedLayerNorm" for e in entries)


def test_encoder_with_decomposed_layer_norms_plans_like_the_fused_one():
    plans = []
    for ln in ("fused", "decomposed"):
        ex = GpuGraphExecutor()
        out, _, _ = graphs.encoder_graph(ex, layers=2, layer_norm=ln)
        ex.add_output(out)
        entries, rowsums = ex.plan()
        plans.append([(e.pattern, e.steps) for e in entries if e.kind != "Skip"])
    norm = {"AddLayerNorm": "LN", "DecomposedLayerNorm": "LN"}
    a, b = ([(norm.get(p, p), s) for p, s in pl] for pl in plans)
    assert a == b
    assert sum(p == "DecomposedLayerNorm" for p, _ in plans[1]) == 4


def test_exported_encoder_plans_like_the_plain_one():
    """DistilBERT-INT8 as exported (runtime reshape targets, the padding mask as Equal /
    Reshape / Expand / Where, node-by-node LayerNorms, the UINT8 embedding Gather +
    DequantizeLinear) plans to the plain encoder's fused heads plus the embedding lookup: no
    MatMul / Softmax / Where / Expand left to run node by node, the mask's Equal(mask, 0)
    computed once for all layers, the shape arithmetic as host-side regular entries."""
    from collections import Counter
    L = 3
    ex = GpuGraphExecutor()
    out, names, params, emb = graphs.export_encoder_graph(ex, layers=L, vocab=1000)
    ex.add_output(out)
    entries, _ = ex.plan()
    live = [e for e in entries if e.kind != "Skip"]
    heads = Counter(e.pattern for e in live if e.kind == "FusedHead")
    assert heads == {"QuantizedLinear": 6 * L, "DecomposedLayerNorm": 1 + 2 * L, "Attention": L,
                     "GatherDequantize": 1}
    regular = Counter(e.op_type for e in live if e.kind == "Regular")
    assert regular["Equal"] == 1 and regular["DynamicQuantizeLinear"] == 4 * L
    for op in ("MatMul", "Softmax", "Where", "Expand", "Transpose", "Add", "Mul", "Div"):
        assert regular[op] == 0, op
    assert sorted({e.group for e in live if e.group}) == ["L%d.q.mmi" % l for l in range(L)]


def test_duplicate_nodes_merge_only_in_the_shape_and_mask_plumbing():
    """Identical Equal nodes (inputs, attributes, constant values) become one; the Q / K / V
    projections' identical x_scale * w_scale Muls stay, owned by their quantized-linear heads
    (and the three heads still run as one grouped GEMM); a duplicate whose output is requested
    stays."""
    ex = GpuGraphExecutor()
    ex.add_input("m", [None, None])
    for i in range(3):
        ex.add_initializer("z%d" % i, np.array(0, np.int64))
        ex.add_node("eq%d" % i, "Equal", ["m", "z%d" % i], ["e%d" % i])
        ex.add_node("c%d" % i, "Cast", ["e%d" % i], ["f%d" % i], {"to": 1})
    ex.add_node("sum", "Add", ["f0", "f1"], ["s01"])
    ex.add_node("sum2", "Add", ["s01", "f2"], ["s"])
    ex.add_output("s")
    ops = [e.op_type for e in ex.plan()[0] if e.kind != "Skip"]
    assert ops.count("Equal") == 1 and ops.count("Cast") == 1  # the Casts then coincide too
    ex.add_output("e2")
    ops = [e.op_type for e in ex.plan()[0] if e.kind != "Skip"]
    assert ops.count("Equal") == 2
    ex2 = GpuGraphExecutor()
    out, _, _ = graphs.encoder_graph(ex2, layers=2)
    ex2.add_output(out)
    live = [e for e in ex2.plan()[0] if e.kind != "Skip"]
    assert [e.op_type for e in live if e.kind == "Regular"] == ["DynamicQuantizeLinear"] * 8
    assert sorted({e.group for e in live if e.group}) == ["L0.q.mmi", "L1.q.mmi"]
