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
    assert e.value.status == 7 and "1 launch" in str(e.value)
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
