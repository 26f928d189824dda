"""GPU parity of the DistilBERT-shaped encoder run through GpuGraphExecutor.

Two kinds of evidence:
  * end to end on a small encoder (2 layers, batch 2, seq 16, three seeds) against the oracle
    composition of the same graph: the fp32 attention and exp differ from the reference's
    summation order by f32 rounding.  When that moves the extreme element of a tensor a
    DynamicQuantizeLinear reads, the scale changes and every element of that tensor is
    requantized, so the final output is compared within 2e-2 of its magnitude (a few
    quantization steps); when no range endpoint moves the outputs agree to ~1e-7;
  * node by node at the full BASELINE size (6 layers, batch 32, seq 128): each node's GPU
    output is checked against the oracle applied to that node's GPU inputs — bit-exact for
    every DynamicQuantizeLinear (x_q, scale, zero point), every quantized linear (integer
    accumulation + dequant + bias), every residual LayerNorm; within 1e-6 for the GELU
    linears (device exp) and 1e-5 for the attention (fp32 MFMA summation order).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import graphs
from iconnx_amd.executor import GpuGraphExecutor
from tests import encoder_ref as ref
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


def assert_bits(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype == np.float32:
        bad = int(np.count_nonzero(bits(got) != bits(want)))
    else:
        bad = int(np.count_nonzero(got != want))
    assert bad == 0, "%s: %d of %d elements differ (rel err %.3g)" % (
        what, bad, want.size, rel_err(got, want) if got.dtype == np.float32 else -1)


@pytest.mark.parametrize("seed", [4000, 4100, 4200])
def test_small_encoder_end_to_end(seed):
    ex = GpuGraphExecutor()
    out, names, params = graphs.encoder_graph(ex, layers=2, seed=seed)
    x = graphs.encoder_input(2, 16, seed=seed + 999)
    got = ex.run({"x": x}, [out])[out]
    entries, _ = ex.plan()
    pats = [e.pattern for e in entries if e.kind == "FusedHead"]
    assert pats.count("Attention") == 2 and pats.count("AddLayerNorm") == 4
    want = x
    for l in range(2):
        want = ref.layer_ref(want, params[l], 12, 1e-12)["out"]
    assert rel_err(got, want) < 2e-2


def test_attention_outside_the_fused_kernel_runs_node_by_node():
    """Head size 32 (the kernels take 64): the Attention head falls back to its Reshape /
    Transpose / MatMul / Softmax nodes (generic kernels), against the oracle composition; the
    same graph shape with heads of 64 runs the one-tile kernel at S = 128 and the chunked one
    at S = 130."""
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((2, 130, 4 * 32)).astype(np.float32) for _ in range(3))
    ex = GpuGraphExecutor()
    for n in "qkv":
        ex.add_input(n, [None, None, 128])
    ctx = graphs.add_self_attention(ex, "q", "k", "v", 4, 32, "att")
    got = ex.run({"q": q, "k": k, "v": v}, [ctx])[ctx]
    assert [e.pattern for e in ex.plan()[0] if e.kind == "FusedHead"] == ["Attention"]
    assert rel_err(got, ref.attention_ref(q, k, v, 4, np.sqrt(32))) < 1e-5
    q, k, v = (rng.standard_normal((2, 130, 4 * 64)).astype(np.float32) for _ in range(3))
    ex = GpuGraphExecutor()
    for n in "qkv":
        ex.add_input(n, [None, None, 256])
    ctx = graphs.add_self_attention(ex, "q", "k", "v", 4, 64, "att")
    for S in (130, 128):
        q2, k2, v2 = (t[:, :S].copy() for t in (q, k, v))
        got2 = ex.run({"q": q2, "k": k2, "v": v2}, [ctx])[ctx]
        assert rel_err(got2, ref.attention_ref(q2, k2, v2, 4)) < 1e-5, S


def test_full_size_encoder_node_by_node():
    cfg = graphs.ENCODER
    B, S, H, L = cfg["batch"], cfg["seq"], cfg["heads"], cfg["layers"]
    ex = GpuGraphExecutor()
    out, names, params = graphs.encoder_graph(ex, layers=L, heads=H)
    x = graphs.encoder_input(B, S)
    want = []
    for t in names:
        base = t["q"].rsplit(".", 2)[0]  # "L<l>"
        want += [t["x"], t["xq"], t["q"], t["k"], t["v"], t["ctx"], base + ".o.x_q",
                 base + ".o.x_scale", base + ".o.x_zp", t["o"], t["x1"], base + ".ff1.x_q",
                 base + ".ff1.x_scale", base + ".ff1.x_zp", t["h"], base + ".ff2.x_q",
                 base + ".ff2.x_scale", base + ".ff2.x_zp", t["f"], t["out"],
                 base + ".qkv.x_scale", base + ".qkv.x_zp"]
    want = [w for w in dict.fromkeys(want) if w != "x"]
    got = ex.run({"x": torch.from_numpy(x).cuda()}, want)
    got["x"] = x
    live = [e for e in ex.plan()[0] if e.kind != "Skip"]
    assert len(live) == 13 * L  # 4 DQL, 6 fused linears, attention, 2 residual norms per layer
    rows = [(0, 8), (B * S // 2 + 3, B * S // 2 + 11), (B * S - 8, B * S)]
    eps = cfg["eps"]
    for l, t in enumerate(names):
        base, p = "L%d" % l, params[l]
        flat = lambda a: np.asarray(a).reshape(-1, np.asarray(a).shape[-1])

        def dql_check(src, tag):
            yq, ys, yz = oracle.dynamic_quantize_linear(got[src])
            assert_bits(got["%s.%s.x_q" % (base, tag)], yq, "%s %s x_q" % (base, tag))
            assert_bits(got["%s.%s.x_scale" % (base, tag)], np.asarray(ys, np.float32), "%s %s scale" % (base, tag))
            assert int(got["%s.%s.x_zp" % (base, tag)]) == int(yz)

        def lin_check(tag, xq_name, out_name, gelu=False):
            xq = got["%s.%s.x_q" % (base, xq_name)]
            xs = got["%s.%s.x_scale" % (base, xq_name)]
            xz = got["%s.%s.x_zp" % (base, xq_name)]
            for r0, r1 in rows:
                y = ref.dequant_linear(xq, xs, xz, p[tag], rows=(r0, r1), gelu=gelu)
                g = flat(got[out_name])[r0:r1]
                if gelu:
                    assert rel_err(g, y) < 1e-6, "%s %s rows %d:%d" % (base, tag, r0, r1)
                else:
                    assert_bits(g, y, "%s %s rows %d:%d" % (base, tag, r0, r1))

        def ln_check(a, b, prm, out_name):  # every row
            y = ref.add_layer_norm_ref(flat(got[a]), flat(got[b]), prm, eps)
            assert_bits(flat(got[out_name]), y, "%s %s" % (base, out_name))

        dql_check(t["x"], "qkv")
        for n in ("q", "k", "v"):
            lin_check(n, "qkv", t[n])
        # attention on every sequence of the batch
        a = ref.attention_ref(got[t["q"]], got[t["k"]], got[t["v"]], H, 8.0)
        for b in range(B):
            assert rel_err(got[t["ctx"]][b], a[b]) < 1e-5, "%s attention batch %d" % (base, b)
        dql_check(t["ctx"], "o")
        lin_check("o", "o", t["o"])
        ln_check(t["o"], t["x"], p["ln1"], t["x1"])
        dql_check(t["x1"], "ff1")
        lin_check("ff1", "ff1", t["h"], gelu=True)
        dql_check(t["h"], "ff2")
        lin_check("ff2", "ff2", t["f"])
        ln_check(t["f"], t["x1"], p["ln2"], t["out"])
    assert np.all(np.isfinite(got[out]))


def ff2_names(names, tag="ff2"):
    out = []
    for t in names:
        base = t["q"].rsplit(".", 2)[0]
        out += [base + ".%s.x_q" % tag, base + ".%s.x_scale" % tag, base + ".%s.x_zp" % tag]
    return out


def test_full_size_encoder_as_benched():
    """The 6-layer b32 s128 encoder exactly as bench.py runs it: captured with only the final
    output requested, so every FFN-up GEMM quantizes its own output for the FFN-down's DQL and
    every attention its context for the output projection's DQL (2L fused launches), and
    every other DQL takes its range from its producer; replayed twice.  The reference run is
    the same graph run eagerly with those fusions turned off (the planner option
    "quantized_outputs": every DQL a launch of its own on the f32 tensor, which the
    node-by-node test pins to the oracle; those DQLs are checked against the oracle here
    too).  The bar is bit equality of every layer's quantized GEMM inputs (x_q, scale, zero
    point) and of the final output."""
    cfg = graphs.ENCODER
    B, S, H, L = cfg["batch"], cfg["seq"], cfg["heads"], cfg["layers"]
    x = torch.from_numpy(graphs.encoder_input(B, S)).cuda()

    ref_ex = GpuGraphExecutor()
    out, names, _ = graphs.encoder_graph(ref_ex, layers=L, heads=H)
    ref_ex.set_option("quantized_outputs", False)
    qnames = ff2_names(names) + ff2_names(names, "o") + ff2_names(names, "ff1") + ff2_names(names, "qkv")
    srcs = [t[k] for k in ("h", "ctx", "x1", "out") for t in names]
    want = ref_ex.run({"x": x}, list(dict.fromkeys([out] + srcs + qnames)))
    assert ref_ex.quantized_outputs() == ({}, 0)
    for j, (src, base) in enumerate((("h", 0), ("ctx", 3 * L), ("x1", 6 * L), ("out", 9 * L))):
        for l, t in enumerate(names):
            if src == "out":  # the Q/K/V DQL of layer l + 1 reads layer l's output
                if l == L - 1:
                    continue
                i = base + 3 * (l + 1)
            else:
                i = base + 3 * l
            yq, ys, yz = oracle.dynamic_quantize_linear(want[t[src]])
            assert_bits(want[qnames[i]], yq, "L%d DQL of %s x_q (unfused) vs oracle" % (l, src))
            assert_bits(want[qnames[i + 1]], np.asarray(ys, np.float32), "L%d DQL of %s scale vs oracle" % (l, src))
            assert int(want[qnames[i + 2]]) == int(yz)
    fused = sorted([t[k] for k in ("h", "ctx") for t in names])
    n_fused = 2 * L

    # as benched: only the final output
    ex = GpuGraphExecutor()
    graphs.encoder_graph(ex, layers=L, heads=H)
    xin = x.clone()
    ex.capture({"x": xin}, [out])
    planned, launches = ex.quantized_outputs()
    assert sorted(planned) == fused
    # capture runs the plan twice on the host (the warm-up run, then the recorded one): every
    # planned head launch took the fused form both times
    assert launches == 2 * n_fused, "%d fused launches for %d layers" % (launches, L)
    for rep in range(2):
        ex.replay()
        got = ex.outputs([out])[out].cpu().numpy()
        ex.check_status()
        assert_bits(got, want[out], "final output, replay %d" % rep)

    # the same capture with the FFN-down inputs also requested: the same plan (requesting a
    # DQL's outputs does not touch the fusion), so its quantized tensors are the benched ones
    ex2 = GpuGraphExecutor()
    graphs.encoder_graph(ex2, layers=L, heads=H)
    ex2.capture({"x": xin}, [out] + qnames)
    assert ex2.plan()[0] == ex.plan()[0]
    assert ex2.quantized_outputs() == (planned, 2 * n_fused)
    for rep in range(2):
        ex2.replay()
        got = {k: v.cpu().numpy() for k, v in ex2.outputs([out] + qnames).items()}
        ex2.check_status()
        for n in qnames:
            assert_bits(got[n], want[n], "%s, replay %d" % (n, rep))
        assert_bits(got[out], want[out], "final output (second capture), replay %d" % rep)
