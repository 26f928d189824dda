"""GPU: DistilBERT-INT8 in the form an export writes it (graphs.export_encoder_graph: Hugging
Face's DistilBertModel through torch.onnx and ONNX Runtime's dynamic quantization — Int64
input_ids / attention_mask, the UINT8 word table through Gather + DequantizeLinear, position
ids sliced to the sequence length, every reshape target assembled from Shape / Gather /
Unsqueeze / Concat, the padding mask as Equal / Reshape / Expand / Where, LayerNorms node by
node), run by GpuGraphExecutor — from an .onnx file through OnnxParser / from_model, and at
the full BASELINE size (6 layers, batch 32, seq 128, vocabulary 30522) directly.

Node by node, each node group's GPU output against the oracle applied to that group's GPU
inputs: bit-exact for the embeddings (Gather, DequantizeLinear, the broadcast Add, the
LayerNorm), every DynamicQuantizeLinear (x_q, scale, zero point), every quantized linear and
every LayerNorm (the LayerNormalization arithmetic: the node-by-node form with Mul(c, c) for
Pow(c, 2), which the reference's powf matches to the last ulp or within 1e-6); within 1e-6 for
the GELU linears (device erf / exp) and 1e-5 for the masked attention (fp32 MFMA summation
order, device exp) — the tolerances of the unmasked encoder's node-by-node test.  The masked
attention runs as one fused kernel (the Where / Expand / Shape of the mask and the key's two
transposes folded into the attention head); the same graph with a sequence past the kernel's
128 runs the chunked kernel; with heads of 32 or a mask that is not per key, the nodes run one by
one; all against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import graphs
from iconnx_amd.executor import GpuGraphExecutor
from iconnx_amd.onnx import OnnxParser
from oracle import layout as L
from tests import encoder_ref as ref
from tests.golden_util import bits

pytestmark = pytest.mark.gpu
H = 12


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


def assert_bits(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = int(np.count_nonzero(bits(got) != bits(want))) if got.dtype == np.float32 else \
        int(np.count_nonzero(got != want))
    assert bad == 0, "%s: %d of %d elements differ" % (what, bad, want.size)


def wanted(names):
    want = [names["emb"], "emb.word.out", "emb.pemb", "emb.e"]
    for t in names["layers"]:
        base = t["q"].rsplit(".", 2)[0]
        for tag in ("qkv", "o", "ff1", "ff2"):
            want += ["%s.%s.x_q" % (base, tag), "%s.%s.x_scale" % (base, tag), "%s.%s.x_zp" % (base, tag)]
        want += [t[k] for k in ("q", "k", "v", "ctx", "o", "x1", "h", "f", "out")]
    return list(dict.fromkeys(want))


def check_node_by_node(got, names, params, emb, ids, mask, eps=1e-12, rows=None):
    flat = lambda a: np.asarray(a).reshape(-1, np.asarray(a).shape[-1])  # noqa: E731
    B, S = ids.shape
    # embeddings
    we = oracle.dequantize_linear(oracle.gather(emb["word"], ids), emb["scale"], emb["zp"])
    assert_bits(got["emb.word.out"], we, "word embeddings")
    pid = L.slice_(np.arange(emb["pos"].shape[0], dtype=np.int64).reshape(1, -1), [0], [S], [1])
    assert_bits(got["emb.pemb"], oracle.gather(emb["pos"], pid), "position embeddings")
    assert_bits(got["emb.e"], oracle.add(got["emb.word.out"], got["emb.pemb"]), "embedding sum")
    e_ln = oracle.layer_norm_decomposed(got["emb.e"], emb["ln"]["scale"], emb["ln"]["bias"], eps, square=True)
    assert_bits(got[names["emb"]], e_ln, "embedding LayerNorm")
    all_rows = [(0, B * S)] if rows is None else rows
    for l, t in enumerate(names["layers"]):
        base, p = "L%d" % l, params[l]

        def dql_check(src, tag):
            yq, ys, yz = oracle.dynamic_quantize_linear(got[src])
            assert_bits(got["%s.%s.x_q" % (base, tag)], yq, "%s %s x_q" % (base, tag))
            assert_bits(got["%s.%s.x_scale" % (base, tag)], np.asarray(ys, np.float32), "%s %s scale" % (base, tag))
            assert int(got["%s.%s.x_zp" % (base, tag)]) == int(yz)

        def lin_check(tag, xq_name, out_name, gelu=False):
            xq = got["%s.%s.x_q" % (base, xq_name)]
            xs = got["%s.%s.x_scale" % (base, xq_name)]
            xz = got["%s.%s.x_zp" % (base, xq_name)]
            for r0, r1 in all_rows:
                y = ref.dequant_linear(xq, xs, xz, p[tag], rows=(r0, r1), gelu=gelu)
                g = flat(got[out_name])[r0:r1]
                if gelu:
                    assert rel_err(g, y) < 1e-6, "%s %s rows %d:%d" % (base, tag, r0, r1)
                else:
                    assert_bits(g, y, "%s %s rows %d:%d" % (base, tag, r0, r1))

        def ln_check(a, b, prm, out_name):  # every row
            y = oracle.layer_norm_decomposed(flat(got[a]), prm["scale"], prm["bias"], eps, residual=flat(got[b]),
                                             square=True)
            assert_bits(flat(got[out_name]), y, "%s %s" % (base, out_name))

        dql_check(t["x"], "qkv")
        for n in ("q", "k", "v"):
            lin_check(n, "qkv", t[n])
        a = ref.attention_ref(got[t["q"]], got[t["k"]], got[t["v"]], H, 8.0, mask=mask)
        for b in range(B):
            assert rel_err(got[t["ctx"]][b], a[b]) < 1e-5, "%s masked attention batch %d" % (base, b)
        dql_check(t["ctx"], "o")
        lin_check("o", "o", t["o"])
        ln_check(t["o"], t["x"], p["ln1"], t["x1"])
        dql_check(t["x1"], "ff1")
        lin_check("ff1", "ff1", t["h"], gelu=True)
        dql_check(t["h"], "ff2")
        lin_check("ff2", "ff2", t["f"])
        ln_check(t["f"], t["x1"], p["ln2"], t["out"])


@pytest.mark.parametrize("variant", ["opset13", "per_channel", "opset17_norm"])
def test_export_model_from_file(tmp_path, variant):
    """The export at opset 13-16 (LayerNorms node by node), with ONNX Runtime's per-channel
    weight scales (zero points [N] of zeros), and at opset 17 (LayerNormalization nodes)."""
    path = str(tmp_path / "distilbert_int8_export.onnx")
    kw = {} if variant == "opset13" else {variant: True}
    out, names, params, emb = graphs.write_model(path, graphs.export_encoder_graph, layers=2, vocab=1000, **kw)
    model = OnnxParser.parse_file(path)
    ops = set(model.list_unique_operators())
    assert {"Shape", "Unsqueeze", "Concat", "Slice", "Equal", "Expand", "Where", "Pow", "ReduceMean",
            "Sqrt", "DequantizeLinear", "Gather"} <= ops
    assert ("LayerNormalization" in ops) == (variant == "opset17_norm")
    ex = GpuGraphExecutor.from_model(model)
    ids, mask = graphs.export_inputs(4, 32, 1000)
    got = ex.run({"input_ids": ids, "attention_mask": mask}, wanted(names))
    check_node_by_node(got, names, params, emb, ids, mask)
    # the padding matters: the same ids unmasked give another context
    got2 = ex.run({"input_ids": ids, "attention_mask": np.ones_like(mask)}, [names["layers"][0]["ctx"]])
    assert not np.array_equal(got2[names["layers"][0]["ctx"]], got[names["layers"][0]["ctx"]])
    # every reshape target and mask shape came from the host: no node of the shape arithmetic
    # runs as a kernel, and the quantized linears / LayerNorms still fuse
    pats = [e.pattern for e in ex.plan()[0] if e.kind == "FusedHead"]
    norms = pats.count("DecomposedLayerNorm") + pats.count("AddLayerNorm")
    assert norms == 1 + 2 * 2 and pats.count("QuantizedLinear") == 6 * 2
    assert pats.count("Attention") == 2  # the masked attention as one kernel


def test_export_model_full_size():
    cfg = graphs.ENCODER
    B, S, layers = cfg["batch"], cfg["seq"], cfg["layers"]
    ex = GpuGraphExecutor()
    out, names, params, emb = graphs.export_encoder_graph(ex, layers=layers)
    ids, mask = graphs.export_inputs(B, S)
    feeds = {"input_ids": torch.from_numpy(ids).cuda(), "attention_mask": torch.from_numpy(mask).cuda()}
    got = ex.run(feeds, wanted(names))
    rows = [(0, 8), (B * S // 2 + 3, B * S // 2 + 11), (B * S - 8, B * S)]
    check_node_by_node(got, names, params, emb, ids, mask, rows=rows)
    assert np.all(np.isfinite(got[out]))
    # captured with only the final output requested (heads then quantize their own outputs
    # for the next DQL where they can): every replay bit-identical to the eager run
    ex2 = GpuGraphExecutor()
    graphs.export_encoder_graph(ex2, layers=layers)
    ex2.capture(feeds, [out])
    for _ in range(2):
        ex2.replay()
        rep = ex2.outputs([out])[out].cpu().numpy()
        ex2.check_status()
        assert_bits(rep, got[out], "captured replay vs eager")


def attention_graph(cond=False, D=64):
    """q, k, v, x [B, S, H*D] and the Int64 mask through add_self_attention_export; with
    ``cond`` a Bool [B, 1, S, S] input is the Where's condition instead (not per key)."""
    ex = GpuGraphExecutor()
    for n in ("x", "q", "k", "v"):
        ex.add_input(n, [None, None, H * D])
    ex.add_input("mask", [None, None])
    if cond:
        ex.add_input("cond", [None, 1, None, None])
    return ex, graphs.add_self_attention_export(ex, "x", "q", "k", "v", "mask", H, D, "att",
                                                cond="cond" if cond else None)


def attention_feeds(S, B=6, seed=0, D=64):
    rng = np.random.default_rng(seed + S)
    q, k, v = (rng.standard_normal((B, S, H * D)).astype(np.float32) for _ in range(3))
    x = np.zeros((B, S, H * D), np.float32)
    lens = np.array([S, 1, S // 2, 0, S - 1, 3])[:B]
    mask = (np.arange(S)[None, :] < lens[:, None]).astype(np.int64)
    return q, k, v, x, mask


@pytest.mark.parametrize("S,D", [(128, 64), (77, 64), (130, 64), (384, 64), (512, 64), (100, 32)])
def test_masked_attention_fused_and_fallback(S, D):
    """S <= 128: the one-tile kernel with the per-key mask (a batch whose every key is padding
    included: a uniform softmax, as the node-by-node Where gives); S > 128: the chunked
    kernel with the mask; head size 32: the node-by-node fallback.  All within 1e-5 of the
    oracle."""
    q, k, v, x, mask = attention_feeds(S, D=D)
    ex, ctx = attention_graph(D=D)
    feeds = {n: torch.from_numpy(a).cuda() for n, a in (("x", x), ("q", q), ("k", k), ("v", v), ("mask", mask))}
    got = ex.run(feeds, [ctx])[ctx]
    assert [e.pattern for e in ex.plan()[0] if e.kind == "FusedHead"] == ["Attention"]
    want = ref.attention_ref(q, k, v, H, np.sqrt(D), mask=mask)
    for b in range(len(mask)):
        assert rel_err(got[b], want[b]) < 1e-5, (S, b)


def test_attention_with_a_condition_that_is_not_per_key_runs_node_by_node():
    """A causal [B, 1, S, S] condition: the head matches, the run-time check sends it node by
    node (Where broadcast over the heads, Softmax, MatMuls), against the oracle."""
    S = 96
    q, k, v, x, mask = attention_feeds(S, B=3)
    cond = np.broadcast_to(np.triu(np.ones((S, S), np.bool_), 1), (3, 1, S, S)).copy()
    ex, ctx = attention_graph(cond=True)
    feeds = {n: torch.from_numpy(a).cuda() for n, a in (("x", x), ("q", q), ("k", k), ("v", v), ("mask", mask),
                                                        ("cond", cond))}
    got = ex.run(feeds, [ctx])[ctx]
    assert [e.pattern for e in ex.plan()[0] if e.kind == "FusedHead"] == ["Attention"]
    want = ref.attention_ref(q, k, v, H, 8.0, cond=cond)
    for b in range(3):
        assert rel_err(got[b], want[b]) < 1e-5, b
