"""GPU parity of the graph executor: ORT-style quantized-linear graphs built node by node
and run through GpuGraphExecutor (lowering, fusion, packing, pool, dispatch all native),
against the oracle run op by op in graph order.

Reference behaviour mirrored: GpuGraphExecutor::run (src/cuda/inference/mod.rs:428) with
its input-shape guard (:441-460) and the unsupported-op error of dispatch
(src/cuda/executor/mod.rs:169-178).  The bar is bit-exact (every fp32 op rounds once, as
the reference's separate nodes do).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import configs, graphs
from iconnx_amd._lib import IconnxError
from iconnx_amd.executor import GpuGraphExecutor
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def assert_bits_equal(got, want, what):
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = int(np.count_nonzero(bits(got) != bits(want)))
    assert bad == 0, "%s: %d of %d elements differ" % (what, bad, want.size)


def run_config(cfg, sample, x_shape=None):
    ex = GpuGraphExecutor()
    y, d = graphs.config_graph(ex, cfg, x_shape=x_shape)
    x = d["x"]
    got = ex.run({"x": torch.from_numpy(x).cuda()}, [y])[y]
    assert got.shape == x.shape[:-1] + (d["w"].shape[1],)
    got2 = got.reshape(-1, got.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    for r0, r1 in sample(M):
        ref = oracle.qlinear_graph(x2, d["w"], d["w_zp"], d["w_scale"], d["bias"],
                                   [(op, c, False) for op, c in d["chain"]], rows=(r0, r1))
        assert_bits_equal(got2[r0:r1], ref["y"][r0:r1], "%s rows %d:%d" % (cfg, r0, r1))
    return ex


def test_cfg1_graph_all_rows():
    run_config("cfg1", lambda M: [(0, M)], x_shape=[1, 128, 768])


def test_cfg2_graph_ffn_up_with_chain():
    run_config("cfg2", lambda M: [(0, 24), (M // 2, M // 2 + 8), (M - 16, M)])


def test_cfg4_graph_per_channel_zero_points_use_dql_row_sums():
    ex = run_config("cfg4", lambda M: [(0, 8), (M - 8, M)])
    _, rowsums = ex.plan()
    assert rowsums == ["cfg4.x_q"]


def test_unfused_path_matches_fused():
    """Requesting the intermediates forces MatMulInteger, Cast, Mul and Add to run as
    separate ops; every intermediate and the output match the oracle bit for bit."""
    d = configs.make("cfg1")
    ex = GpuGraphExecutor()
    ex.add_input("x", [1, 128, 768])
    y = graphs.add_quantized_linear(ex, "x", d["w"], d["w_zp"], d["w_scale"], d["bias"],
                                    prefix="u")
    names = ["u.x_q", "u.x_scale", "u.x_zp", "u.acc", "u.acc_f", "u.scale", "u.linear0", y]
    out = ex.run({"x": d["x"]}, names)
    entries, _ = ex.plan()
    assert not [e for e in entries if e.kind == "FusedHead"]
    ref = oracle.qlinear_graph(d["x"], d["w"], d["w_zp"], d["w_scale"], d["bias"])
    np.testing.assert_array_equal(out["u.x_q"].reshape(-1, 768), ref["xq"])
    assert_bits_equal(out["u.x_scale"], np.asarray(ref["x_scale"]), "x_scale")
    np.testing.assert_array_equal(out["u.x_zp"], ref["x_zp"])
    np.testing.assert_array_equal(out["u.acc"].reshape(-1, 768), ref["acc"])
    assert_bits_equal(out["u.acc_f"].reshape(-1, 768), ref["cast"], "cast")
    assert_bits_equal(out["u.scale"], np.asarray(ref["scale"]), "scale")
    assert_bits_equal(out[y].reshape(-1, 768), ref["y"], "y")


def test_dequantize_linear_epilogue_and_standalone_chain():
    """MatMulInteger -> DequantizeLinear(acc, scale) -> Mul -> Add: one QuantizedLinear head
    (Mul(scale), Mul(m), Add(b) in the GEMM store); with the accumulator requested, the
    DequantizeLinear runs on its own and the Mul / Add become a MulAdd head."""
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, (96, 64)).astype(np.uint8)
    w = rng.integers(-127, 128, (64, 80)).astype(np.int8)
    m = rng.standard_normal(80).astype(np.float32)
    b = rng.standard_normal(80).astype(np.float32)
    a_zp, s = np.array(131, np.uint8), np.array(0.003, np.float32)
    ex = GpuGraphExecutor()
    ex.add_input("a", [None, 64])
    for name, arr in (("w", w), ("a_zp", a_zp), ("s", s), ("m", m), ("b", b)):
        ex.add_initializer(name, arr)
    ex.add_node("mm", "MatMulInteger", ["a", "w", "a_zp"], ["acc"])
    ex.add_node("dq", "DequantizeLinear", ["acc", "s"], ["y0"])
    ex.add_node("mul", "Mul", ["y0", "m"], ["y1"])
    ex.add_node("add", "Add", ["y1", "b"], ["y2"])
    out = ex.run({"a": a}, ["y2"])["y2"]
    entries, _ = ex.plan()
    assert [(e.pattern, e.steps) for e in entries if e.kind == "FusedHead"] == [("QuantizedLinear", 3)]
    acc = oracle.matmul_integer(a, w, a_zp, None)
    want = oracle.add(oracle.mul(oracle.dequantize_linear(acc, s, None), m), b)
    assert_bits_equal(out, want, "MatMulInteger + DequantizeLinear + Mul + Add in one head")
    got = ex.run({"a": a}, ["y2", "acc"])
    assert [e.pattern for e in ex.plan()[0] if e.kind == "FusedHead"] == ["MulAdd"]
    assert np.array_equal(got["acc"], acc)
    assert_bits_equal(got["y2"], want, "dequantize + MulAdd")


def test_shape_guard_and_dynamic_dims():
    d = configs.make("cfg1")
    ex = GpuGraphExecutor()
    y, _ = graphs.config_graph(ex, "cfg1", x_shape=[1, 128, 768])
    with pytest.raises(IconnxError, match="does not match the compiled plan"):
        ex.run({"x": d["x"][:, :64]}, [y])
    # dynamic batch / sequence: any [B, S, 768]
    ex2 = GpuGraphExecutor()
    y2, _ = graphs.config_graph(ex2, "cfg1")
    part = np.ascontiguousarray(d["x"][:, :40])
    got = ex2.run({"x": part}, [y2])[y2]
    ref = oracle.qlinear_graph(part, d["w"], d["w_zp"], d["w_scale"], d["bias"])
    assert_bits_equal(got.reshape(-1, 768), ref["y"], "dynamic dims")


def test_unsupported_op_names_the_node():
    ex = GpuGraphExecutor()
    ex.add_input("x", [4])
    ex.add_node("my_conv", "Conv", ["x"], ["y"])
    with pytest.raises(IconnxError, match="my_conv.*Conv.*not on the quantized-linear path"):
        ex.run({"x": np.ones(4, np.float32)}, ["y"])


def test_pool_reuse_across_runs_and_device_inputs():
    d = configs.make("cfg2")
    ex = GpuGraphExecutor()
    y, _ = graphs.config_graph(ex, "cfg2")
    x = torch.from_numpy(d["x"]).cuda()
    first = ex.run_device({"x": x}, [y])[y]
    m1, h1, held1 = ex.pool_stats()
    second = ex.run_device({"x": x}, [y])[y]
    m2, h2, held2 = ex.pool_stats()
    torch.cuda.synchronize()
    assert m2 == m1 and held2 == held1, "second run reached hipMalloc"
    assert h2 > h1
    assert torch.equal(first, second)


def test_shared_dql_three_projections_per_channel():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 48, 64)).astype(np.float32)
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, None, 64])
    dql = graphs.add_dynamic_quantize(ex, "x", "attn")
    params, outs = {}, []
    for p in ("q", "k", "v"):
        w = rng.integers(-127, 128, (64, 96)).astype(np.int8)
        zp = rng.integers(-8, 9, 96).astype(np.int8)
        sc = rng.uniform(0.005, 0.03, 96).astype(np.float32)
        b = rng.standard_normal(96).astype(np.float32)
        params[p] = (w, zp, sc, b)
        outs.append(graphs.add_quantized_linear(ex, "x", w, zp, sc, b, prefix=p, dql=dql))
    got = ex.run({"x": x}, outs)
    entries, rowsums = ex.plan()
    assert rowsums == ["attn.x_q"]
    assert sum(e.op_type == "DynamicQuantizeLinear" for e in entries) == 1
    for p, o in zip("qkv", outs):
        w, zp, sc, b = params[p]
        ref = oracle.qlinear_graph(x, w, zp, sc, b)
        assert_bits_equal(got[o].reshape(-1, 96), ref["y"], p)


def test_capture_and_replay_match_eager_runs():
    """A recorded run replayed several times, with eager work and synchronisations between
    the replays and new data written into the bound input in between, matches eager runs
    bit for bit; a host-bound input is refused."""
    from iconnx_amd import graphs

    ex = GpuGraphExecutor()
    out, _, _ = graphs.encoder_graph(ex, layers=2, seed=4100)
    xs = [torch.from_numpy(graphs.encoder_input(2, 16, seed=s)).cuda() for s in (1, 2, 3)]
    want = [ex.run({"x": x}, [out])[out] for x in xs]
    xin = xs[0].clone()
    ex.capture({"x": xin}, [out])
    for rep in range(6):
        i = rep % 3
        xin.copy_(xs[i])
        ex.replay()
        got = ex.outputs([out])[out].cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), "replay %d" % rep
        # eager work on the same stream between replays
        _ = (xs[i] * 2.0).sum().item()
        torch.cuda.synchronize()
    # an eager run after the capture (same bound tensor), then replays again
    assert np.array_equal(ex.run({"x": xin}, [out])[out].view(np.uint32), want[2].view(np.uint32))
    xin.copy_(xs[1])
    ex.replay()
    assert np.array_equal(ex.outputs([out])[out].cpu().numpy().view(np.uint32), want[1].view(np.uint32))
    # rebinding another tensor drops the recording; a new capture reads the new tensor
    other = xs[0].clone()
    ex.capture({"x": other}, [out])
    ex.replay()
    assert np.array_equal(ex.outputs([out])[out].cpu().numpy().view(np.uint32), want[0].view(np.uint32))
    ex2 = GpuGraphExecutor()
    out2, _, _ = graphs.encoder_graph(ex2, layers=1, seed=4100)
    with pytest.raises(IconnxError):
        ex2.capture({"x": graphs.encoder_input(2, 16, seed=1)}, [out2])


def test_run_with_profiling_covers_every_planned_op():
    """GpuGraphExecutor.run_with_profiling (the reference's run_with_profiling,
    src/cuda/inference/mod.rs:649-658): on the full cfg3 encoder every executed op of the
    plan has a record, labelled as the reference labels them (op type, or Fused_<pattern>),
    the outputs equal a plain run's, and the per-op GPU times add up to the forward's own
    event time (a plain eager run bracketed by two events) within 20 %: each event between
    two ops costs 1.3-1.8 us on the GPU (its timestamp packet waits for the previous kernel
    to drain before the next dispatch starts; the events already skip the system-scope
    fence), 78 ops here, measured 3-15 % over MI355X boxes."""
    from iconnx_amd import graphs

    cfg = graphs.ENCODER
    ex = GpuGraphExecutor()
    out, _, _ = graphs.encoder_graph(ex, layers=cfg["layers"], heads=cfg["heads"])
    x = torch.from_numpy(graphs.encoder_input(cfg["batch"], cfg["seq"])).cuda()
    want = ex.run({"x": x}, [out])[out]
    got, prof = ex.run_with_profiling({"x": x}, [out])
    assert np.array_equal(got[out].view(np.uint32), want.view(np.uint32))
    live = [e for e in ex.plan()[0] if e.kind != "Skip"]
    assert [o[0] for o in prof.ops] == [e.node for e in live]
    labels = {("Fused_" + e.pattern) if e.kind == "FusedHead" else e.op_type for e in live}
    assert set(prof.gpu_op_times) == labels == set(prof.op_times)
    assert sum(c for _, c in prof.gpu_op_times.values()) == len(live)
    assert prof.gpu_op_times["Fused_QuantizedLinear"][1] == 6 * cfg["layers"]
    assert all(o[2] > 0 for o in prof.ops)
    # the per-op times against the forward timed as a whole (warm, same stream; medians of 5)
    ex.run_device({"x": x}, [out])
    torch.cuda.synchronize()
    whole, summed = [], []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ex.run_device({"x": x}, [out])
        e1.record()
        torch.cuda.synchronize()
        whole.append(1000.0 * e0.elapsed_time(e1))
        _, prof = ex.run_with_profiling({"x": x}, [out])
        summed.append(sum(us for us, _ in prof.gpu_op_times.values()))
    whole_us, total = float(np.median(whole)), float(np.median(summed))
    assert abs(total - whole_us) <= 0.20 * whole_us, (total, whole_us)
    assert "Fused_Attention" in prof.summary()
