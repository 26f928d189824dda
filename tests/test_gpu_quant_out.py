"""GPU parity of the quantized linear that quantizes its own output.

When a QuantizedLinear head's f32 output is read only by a DynamicQuantizeLinear, the
executor runs one GEMM launch that writes the DQL's outputs (y u8, scale, zero point) and
never forms the f32 tensor.  The bar is bit-exact: the same graph with the f32 tensor also
requested as an output (so that it must be formed, and the DQL runs as its own launch) gives
the reference's results — its f32 output against the oracle's DQL of it, bit for bit — and
the fused run must give exactly the same u8 values, scale and zero point.

Reference behaviour mirrored: DynamicQuantizeLinear (src/operators/dynamic_quantize_linear.rs:32-112)
applied to the output of MatMulInteger -> Cast -> Mul -> Add [-> erf-GELU] as the reference's
separate nodes compute it (src/cuda/inference/mod.rs:428 dispatches them one by one).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd.executor import GpuGraphExecutor
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def build(ex, K, N, gelu, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    inits = {
        "w": w,
        "w_scale": np.array(0.004 + 0.001 * (seed % 3), np.float32),
        "bias": (0.05 * rng.standard_normal(N)).astype(np.float32),
        "c_sqrt2": np.array(1.4142135, np.float32),
        "c_one": np.array(1.0, np.float32),
        "c_half": np.array(0.5, np.float32),
    }
    ex.add_input("x", [None, K])
    for name, arr in inits.items():
        ex.add_initializer(name, arr)
    ex.add_node("dql_x", "DynamicQuantizeLinear", ["x"], ["xq", "xs", "xzp"])
    ex.add_node("mm", "MatMulInteger", ["xq", "w", "xzp"], ["acc"])
    ex.add_node("cast", "Cast", ["acc"], ["accf"], {"to": 1})
    ex.add_node("scale", "Mul", ["xs", "w_scale"], ["s"])
    ex.add_node("deq", "Mul", ["accf", "s"], ["lin0"])
    ex.add_node("bias_add", "Add", ["lin0", "bias"], ["lin"])
    h = "lin"
    if gelu:
        ex.add_node("g_div", "Div", ["lin", "c_sqrt2"], ["g0"])
        ex.add_node("g_erf", "Erf", ["g0"], ["g1"])
        ex.add_node("g_add", "Add", ["g1", "c_one"], ["g2"])
        ex.add_node("g_mul", "Mul", ["lin", "g2"], ["g3"])
        ex.add_node("g_half", "Mul", ["g3", "c_half"], ["h"])
        h = "h"
    ex.add_node("dql_h", "DynamicQuantizeLinear", [h], ["hq", "hs", "hzp"])
    return h


def check_same(fused, ref, what):
    for name in ("hq", "hs", "hzp"):
        a, b = fused[name], ref[name]
        assert a.shape == b.shape, (what, name)
        bad = int(np.count_nonzero(bits(a) != bits(b)))
        assert bad == 0, "%s %s: %d of %d differ" % (what, name, bad, b.size)


@pytest.mark.parametrize("M,K,N,gelu", [
    (4096, 768, 3072, True),   # the encoder's FFN-up: 256 tiles of 256x192, one per CU
    (1000, 256, 384, True),    # ragged rows: the last tile row is partly outside M
    (300, 512, 960, False),    # Mul / Add only (the plain column chain)
    (33, 128, 192, True),      # one tile
])
def test_quantized_output_matches_separate_dql(M, K, N, gelu):
    x = np.random.default_rng(M + N).standard_normal((M, K)).astype(np.float32)
    ref_ex, fused_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build(ref_ex, K, N, gelu, seed=K)
    build(fused_ex, K, N, gelu, seed=K)
    ref = ref_ex.run({"x": x}, [h, "hq", "hs", "hzp"])
    assert ref_ex.quantized_outputs()[0] == {}  # the f32 output is requested: not fused
    # the separate DQL is the reference's, bit for bit, on the f32 output
    yq, ys, yzp = oracle.dynamic_quantize_linear(ref[h])
    check_same(ref, {"hq": yq, "hs": ys, "hzp": yzp}, "separate DQL vs oracle")
    fused = fused_ex.run({"x": x}, ["hq", "hs", "hzp"])
    planned, launches = fused_ex.quantized_outputs()
    assert planned == {h: "dql_h"}
    assert launches == 1, "the fused GEMM did not run"
    check_same(fused, ref, "fused vs separate")
    assert np.isfinite(fused["hs"]).all()


def test_quantized_output_repeated_runs_and_smaller_input():
    """Two calls in a row, the second with fewer rows (fewer blocks meet at the grid
    barrier), then the first size again: the barrier counters are back at rest after each."""
    K, N = 768, 3072
    fused_ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build(fused_ex, K, N, True, seed=7)
    build(ref_ex, K, N, True, seed=7)
    rng = np.random.default_rng(11)
    for i, M in enumerate((2048, 700, 2048)):
        x = rng.standard_normal((M, K)).astype(np.float32) * (1.0 + i)
        fused = fused_ex.run({"x": x}, ["hq", "hs", "hzp"])
        ref = ref_ex.run({"x": x}, [h, "hq", "hs", "hzp"])
        check_same(fused, ref, "run %d (M=%d)" % (i, M))
    assert fused_ex.quantized_outputs()[1] == 3


@pytest.mark.parametrize("M,K,N", [
    (64, 256, 200),     # N not a multiple of 192
    (8192, 768, 3072),  # 512 tiles of 256x192: more than can be resident at once
])
def test_quantized_output_falls_back_outside_the_kernel(M, K, N):
    """Outside the fused kernel (shape, or a grid that would not be resident at once) the GEMM
    writes f32 and the DQL runs as its own launch; the results are the same."""
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    fused_ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build(fused_ex, K, N, True, seed=5)
    build(ref_ex, K, N, True, seed=5)
    fused = fused_ex.run({"x": x}, ["hq", "hs", "hzp"])
    ref = ref_ex.run({"x": x}, [h, "hq", "hs", "hzp"])
    planned, launches = fused_ex.quantized_outputs()
    assert planned == {h: "dql_h"} and launches == 0
    check_same(fused, ref, "fallback")


def test_quantized_output_capture_and_replay():
    """The fused launch recorded into a HIP graph and replayed several times, with eager work
    between the replays, matches eager runs bit for bit."""
    K, N, M = 768, 3072, 1024
    ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build(ex, K, N, True, seed=9)
    build(ref_ex, K, N, True, seed=9)
    xs = [torch.from_numpy(np.random.default_rng(s).standard_normal((M, K)).astype(np.float32)).cuda()
          for s in (1, 2, 3)]
    want = [ref_ex.run({"x": x}, [h, "hq", "hs", "hzp"]) for x in xs]
    xin = xs[0].clone()
    ex.capture({"x": xin}, ["hq", "hs", "hzp"])
    for rep in range(6):
        i = rep % 3
        xin.copy_(xs[i])
        ex.replay()
        got = {k: v.cpu().numpy() for k, v in ex.outputs(["hq", "hs", "hzp"]).items()}
        check_same(got, want[i], "replay %d" % rep)
        _ = (xs[i] * 2.0).sum().item()
        torch.cuda.synchronize()


def build_int8_act(ex, K, N, seed):
    """MatMulInteger over an Int8 graph input with an Int8 zero point, then the dequant, a
    bias and a column-vector Div / Mul chain, then a DQL."""
    rng = np.random.default_rng(seed)
    inits = {
        "w": rng.integers(-127, 128, (K, N)).astype(np.int8),
        "a_zp": np.array(-3, np.int8),
        "s": np.array(0.0037, np.float32),
        "bias": (0.05 * rng.standard_normal(N)).astype(np.float32),
        "d": rng.uniform(0.5, 2.5, N).astype(np.float32),
        "m": rng.uniform(0.5, 1.5, N).astype(np.float32),
    }
    ex.add_input("a", [None, K])
    for name, arr in inits.items():
        ex.add_initializer(name, arr)
    ex.add_node("mm", "MatMulInteger", ["a", "w", "a_zp"], ["acc"])
    ex.add_node("cast", "Cast", ["acc"], ["accf"], {"to": 1})
    ex.add_node("deq", "Mul", ["accf", "s"], ["l0"])
    ex.add_node("bias_add", "Add", ["l0", "bias"], ["l1"])
    ex.add_node("div", "Div", ["l1", "d"], ["l2"])
    ex.add_node("mul", "Mul", ["l2", "m"], ["h"])
    ex.add_node("dql_h", "DynamicQuantizeLinear", ["h"], ["hq", "hs", "hzp"])
    return "h"


@pytest.mark.parametrize("M,K,N", [(2048, 768, 3072), (257, 384, 576)])
def test_quantized_output_int8_activations_and_column_division(M, K, N):
    a = np.random.default_rng(M).integers(-128, 128, (M, K)).astype(np.int8)
    ref_ex, fused_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build_int8_act(ref_ex, K, N, seed=N)
    build_int8_act(fused_ex, K, N, seed=N)
    ref = ref_ex.run({"a": a}, [h, "hq", "hs", "hzp"])
    yq, ys, yzp = oracle.dynamic_quantize_linear(ref[h])
    check_same(ref, {"hq": yq, "hs": ys, "hzp": yzp}, "separate DQL vs oracle")
    fused = fused_ex.run({"a": a}, ["hq", "hs", "hzp"])
    planned, launches = fused_ex.quantized_outputs()
    assert planned == {h: "dql_h"} and launches == 1
    check_same(fused, ref, "fused vs separate (int8 activations)")


def test_exchange_that_gives_up_is_an_error_status():
    """A launch in which a block's bounded wait for the others' ranges runs out is reported
    as ICX_ERR_KERNEL by the status check (the reference's CudaError::Kernel,
    src/cuda/executor/mod.rs:169-186), not only as a NaN scale.  The host-side test hook makes
    every wait expect a tag no block publishes, with a short bound, so every block takes the
    failure path and exits normally.  The record is cleared by the check: a normal run after
    it is correct and reports no error."""
    from iconnx_amd._lib import IconnxError, lib

    K, N, M = 768, 3072, 1024
    x = np.random.default_rng(21).standard_normal((M, K)).astype(np.float32)
    ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = build(ex, K, N, True, seed=13)
    build(ref_ex, K, N, True, seed=13)
    want = ref_ex.run({"x": x}, [h, "hq", "hs", "hzp"])
    L = lib()
    L.icx_debug_qout_fault(64)
    try:
        got = ex.run_device({"x": x}, ["hq", "hs", "hzp"])
        with pytest.raises(IconnxError) as e:
            ex.check_status()
    finally:
        L.icx_debug_qout_fault(0)
    assert e.value.status == 7 and "range exchange" in str(e.value)
    assert ex.quantized_outputs()[1] == 1
    assert np.isnan(got["hs"].cpu().numpy()) and not got["hq"].cpu().numpy().any()
    ex.check_status()  # cleared
    check_same(ex.run({"x": x}, ["hq", "hs", "hzp"]), want, "normal run after the failure")
    # run() itself raises when the failure happens in it
    L.icx_debug_qout_fault(64)
    try:
        with pytest.raises(IconnxError) as e:
            ex.run({"x": x}, ["hq", "hs", "hzp"])
    finally:
        L.icx_debug_qout_fault(0)
    assert e.value.status == 7
    check_same(ex.run({"x": x}, ["hq", "hs", "hzp"]), want, "normal run after the second failure")


# ---- the attention that quantizes its own context ---------------------------------------------
def build_attention(ex, H):
    """q, k, v [B, S, H*64] -> the exported self-attention -> DynamicQuantizeLinear(ctx)."""
    from iconnx_amd import graphs

    for n in "qkv":
        ex.add_input(n, [None, None, H * 64])
    ctx = graphs.add_self_attention(ex, "q", "k", "v", H, 64, "att")
    ex.add_node("dql_ctx", "DynamicQuantizeLinear", [ctx], ["cq", "cs", "czp"])
    return ctx


def qkv(B, S, H, seed):
    rng = np.random.default_rng(seed)
    return {n: (rng.standard_normal((B, S, H * 64)) * (1.0 + i)).astype(np.float32) for i, n in enumerate("qkv")}


def check_attention_same(fused, ref, what):
    check_same({"hq": fused["cq"], "hs": fused["cs"], "hzp": fused["czp"]},
               {"hq": ref["cq"], "hs": ref["cs"], "hzp": ref["czp"]}, what)


@pytest.mark.parametrize("B,S,H,fused_launch", [
    (32, 128, 12, True),   # the encoder's attention: 768 blocks of 64 queries
    (4, 100, 12, True),    # partial last block of queries
    (3, 64, 4, True),      # one block per (batch, head)
    (64, 128, 12, False),  # 1536 blocks: more than the exchange holds -> f32 context + DQL launch
])
def test_attention_quantized_output_matches_separate_dql(B, S, H, fused_launch):
    """The attention whose context only a DynamicQuantizeLinear reads writes that DQL's u8
    output, scale and zero point itself (the context is never formed); the same graph with the
    context requested runs the attention and then the DQL, whose result is the oracle's DQL of
    that context bit for bit.  The fused and the separate results are bit-identical."""
    feeds = qkv(B, S, H, seed=B * S + H)
    ref_ex, fused_ex = GpuGraphExecutor(), GpuGraphExecutor()
    ctx = build_attention(ref_ex, H)
    build_attention(fused_ex, H)
    ref = ref_ex.run(feeds, [ctx, "cq", "cs", "czp"])
    assert ref_ex.quantized_outputs()[0] == {}
    yq, ys, yz = oracle.dynamic_quantize_linear(ref[ctx])
    check_attention_same(ref, {"cq": yq, "cs": ys, "czp": yz}, "separate DQL vs oracle")
    fused = fused_ex.run(feeds, ["cq", "cs", "czp"])
    planned, launches = fused_ex.quantized_outputs()
    assert planned == {ctx: "dql_ctx"}
    assert launches == (1 if fused_launch else 0)
    check_attention_same(fused, ref, "fused vs separate (B=%d S=%d H=%d)" % (B, S, H))


def test_attention_quantized_output_capture_replay_and_failure():
    """Recorded and replayed with eager work between the replays (bit-identical to eager
    runs), then the exchange's failure path: with the test hook every wait gives up, the
    status check reports ICX_ERR_KERNEL, and a normal run afterwards is correct."""
    from iconnx_amd._lib import IconnxError, lib

    B, S, H = 32, 128, 12
    ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    ctx = build_attention(ex, H)
    build_attention(ref_ex, H)
    inputs = [{n: torch.from_numpy(a).cuda() for n, a in qkv(B, S, H, seed=s).items()} for s in (1, 2)]
    bound = {n: t.clone() for n, t in inputs[0].items()}
    ex.capture(bound, ["cq", "cs", "czp"])
    for rep in range(3):
        src = inputs[rep % 2]
        for n in bound:
            bound[n].copy_(src[n])
        ex.replay()
        got = {k: v.cpu().numpy() for k, v in ex.outputs(["cq", "cs", "czp"]).items()}
        ex.check_status()
        want = ref_ex.run({n: t.cpu().numpy() for n, t in src.items()}, [ctx, "cq", "cs", "czp"])
        check_attention_same(got, want, "replay %d" % rep)
        _ = (src["q"] * 2.0).sum().item()  # eager work between the replays
    run_ex = GpuGraphExecutor()
    build_attention(run_ex, H)
    L = lib()
    L.icx_debug_qout_fault(64)
    try:
        bad = run_ex.run_device(inputs[0], ["cq", "cs", "czp"])
        with pytest.raises(IconnxError) as e:
            run_ex.check_status()
    finally:
        L.icx_debug_qout_fault(0)
    assert e.value.status == 7
    assert np.isnan(bad["cs"].cpu().numpy()) and not bad["cq"].cpu().numpy().any()
    want = ref_ex.run({n: t.cpu().numpy() for n, t in inputs[0].items()}, [ctx, "cq", "cs", "czp"])
    check_attention_same(run_ex.run(inputs[0], ["cq", "cs", "czp"]), want, "normal run after the failure")


def test_attention_quantized_outputs_interleaved_with_gemm_exchanges():
    """Two attentions that quantize their contexts, with a quantized-output GEMM (the other
    kind of range exchange, which keeps its own launch numbers in the same buffer) between
    them, in one graph run three times: every quantized tensor equals the separate DQL's."""
    from iconnx_amd import graphs

    H, K = 12, 768
    def make(ex):
        for n in "qkv":
            ex.add_input(n, [None, None, H * 64])
        c1 = graphs.add_self_attention(ex, "q", "k", "v", H, 64, "a1")
        ex.add_node("dql1", "DynamicQuantizeLinear", [c1], ["c1q", "c1s", "c1z"])
        rng = np.random.default_rng(4)
        ex.add_initializer("w", rng.integers(-127, 128, (K, 3072)).astype(np.int8))
        ex.add_initializer("ws", np.array(0.003, np.float32))
        ex.add_initializer("b", (0.05 * rng.standard_normal(3072)).astype(np.float32))
        ex.add_node("mm", "MatMulInteger", ["c1q", "w", "c1z"], ["acc"])
        ex.add_node("cast", "Cast", ["acc"], ["accf"], {"to": 1})
        ex.add_node("sc", "Mul", ["c1s", "ws"], ["s"])
        ex.add_node("deq", "Mul", ["accf", "s"], ["l0"])
        ex.add_node("bias", "Add", ["l0", "b"], ["lin"])
        ex.add_node("dqlh", "DynamicQuantizeLinear", ["lin"], ["hq", "hs", "hz"])
        c2 = graphs.add_self_attention(ex, "k", "v", "q", H, 64, "a2")
        ex.add_node("dql2", "DynamicQuantizeLinear", [c2], ["c2q", "c2s", "c2z"])
        return c1, c2
    ref_ex, ex = GpuGraphExecutor(), GpuGraphExecutor()
    c1, c2 = make(ref_ex)
    make(ex)
    names = ["c1q", "c1s", "c1z", "hq", "hs", "hz", "c2q", "c2s", "c2z"]
    for s in range(3):
        feeds = qkv(32, 128, H, seed=40 + s)
        want = ref_ex.run(feeds, [c1, c2, "lin"] + names)
        got = ex.run(feeds, names)
        for n in names:
            assert got[n].shape == want[n].shape, (s, n)
            bad = int(np.count_nonzero(bits(got[n]) != bits(want[n])))
            assert bad == 0, "run %d: %s: %d of %d differ" % (s, n, bad, want[n].size)
    planned, launches = ex.quantized_outputs()
    assert sorted(planned) == sorted([c1, c2, "lin"]) and launches == 9
