"""GPU parity of DynamicQuantizeLinear and the quantized linear that reads it run as ONE
launch (icx_dql_qlinear_f32).

The fused launch must give the DQL's outputs (y u8, scale, zero point) and the linear's f32
output Y bit for bit as the two separate entry points do (icx_dynamic_quantize_linear, then
icx_qlinear_f32 over its y): those are pinned to the oracle by tests/test_gpu_dql.py and
tests/test_gpu_epilogue.py, and here the DQL outputs are also compared with the oracle
directly and Y with the oracle's graph on sampled rows.

Reference behaviour mirrored: DynamicQuantizeLinear (src/operators/dynamic_quantize_linear.rs:
32-112) followed by MatMulInteger -> Cast -> Mul(x_scale * w_scale) -> Add(bias) [-> chain]
(src/operators/matmul_integer.rs:239-267 and the elementwise nodes the reference dispatches
one by one, src/cuda/inference/mod.rs:428).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import configs, ops
from iconnx_amd._lib import IconnxError, lib
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def epilogue_of(w_scale, bias, chain, gelu=False):
    consts = {}
    if gelu:
        consts = {n: dev(np.array(v, np.float32)) for n, v in
                  (("sqrt2", 1.4142135), ("one", 1.0), ("half", 0.5))}

    def epi(ys):
        e = [("Mul", (ys, w_scale), False), ("Add", bias, False)]
        e += [(op, c, False) for op, c in chain]
        if gelu:  # erf-GELU: x * (erf(x / sqrt2) + 1) * 0.5
            e += [("Save", None, False), ("Div", consts["sqrt2"], False), ("Erf", None, False),
                  ("Add", consts["one"], False), ("MulSaved", None, False), ("Mul", consts["half"], False)]
        return e
    return epi


def separate(x, w, epi):
    xq, xs, xzp = ops.gpu_dynamic_quantize_linear(x)[:3]
    y = ops.gpu_qlinear(xq, w, xzp, None, epilogue=epi(xs))
    return xq, xs, xzp, y


def assert_same(fused, ref, what):
    for name, a, b in zip(("y", "scale", "zp", "Y"), fused, ref):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert a.shape == b.shape, (what, name)
        bad = int(np.count_nonzero(bits(a) != bits(b)))
        assert bad == 0, "%s %s: %d of %d differ" % (what, name, bad, b.size)


def make_case(M, K, N, seed, chain=True):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * (1.0 + seed % 3)).astype(np.float32)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    bias = (0.02 * rng.standard_normal(N)).astype(np.float32)
    ch = configs.chain_constants(N, seed) if chain else []
    return x, w, np.array(0.004 + 0.001 * (seed % 4), np.float32), bias, ch


def test_cfg2_one_launch_equals_the_two_and_the_oracle():
    """cfg2 (the metric's FFN-up shape with its Mul/Add/Div/Mul chain): 256 blocks of
    256x192, each quantizing 16 rows of its panel."""
    d = configs.make("cfg2")
    x = d["x"].reshape(-1, 768)
    xd, w = dev(x), ops.PackedWeight(dev(d["w"]))
    epi = epilogue_of(dev(d["w_scale"]), dev(d["bias"]), [(op, dev(c)) for op, c in d["chain"]])
    sync = ops.exchange_buffer()
    fused = ops.gpu_dql_qlinear(xd, w, epi, sync)
    ref = separate(xd, w, epi)
    torch.cuda.synchronize()
    assert_same(fused, ref, "cfg2")
    assert lib().icx_exchange_status(ops._stream(), ops._p(sync)) == 0
    yq, ys, yz = oracle.dynamic_quantize_linear(x)
    assert np.array_equal(fused[0].cpu().numpy(), yq)
    assert bits(fused[1].cpu().numpy()) == bits(np.float32(ys)) and int(fused[2].cpu().numpy()) == int(yz)
    Y = fused[3].cpu().numpy()
    chain = [(op, c, False) for op, c in d["chain"]]
    for r0, r1 in ((0, 24), (2040, 2056), (4072, 4096)):
        want = oracle.qlinear_graph(x, d["w"], d["w_zp"], d["w_scale"], d["bias"], chain, rows=(r0, r1))["y"]
        assert np.array_equal(bits(Y[r0:r1]), bits(want[r0:r1])), "rows %d:%d vs oracle" % (r0, r1)


@pytest.mark.parametrize("M,K,N,gelu", [
    (1000, 768, 3072, False),  # ragged last panel (232 rows)
    (33, 768, 3072, True),     # one panel of 33 rows: blocks 3.. have empty slices
    (2048, 1024, 4608, True),  # 24 tiles per panel, 11 rows of 1024 each
    (512, 384, 1536, False),   # 8 tiles per panel, 32 rows of 384
])
def test_shapes_equal_the_two_launches(M, K, N, gelu):
    x, w8, ws, bias, ch = make_case(M, K, N, seed=M + N, chain=not gelu)
    xd, w = dev(x), ops.PackedWeight(dev(w8))
    epi = epilogue_of(dev(ws), dev(bias), [(op, dev(c)) for op, c in ch], gelu=gelu)
    sync = ops.exchange_buffer()
    fused = ops.gpu_dql_qlinear(xd, w, epi, sync)
    ref = separate(xd, w, epi)
    torch.cuda.synchronize()
    assert_same(fused, ref, "M=%d K=%d N=%d" % (M, K, N))


@pytest.mark.parametrize("M,K,N,supported", [
    (4096, 768, 768, True),     # 64x96 tiles (256x192 ones would give a block 64 rows of 768)
    (128, 768, 768, True),      # cfg1's batch-1 activation: 16 tiles of 64x96
    (4096, 768, 1000, False),   # N not a multiple of 96
    (4096, 700, 3072, False),   # K not a multiple of 128
    (8192, 768, 3072, False),   # 512 tiles of 256x192 (more than one per CU), 4096 of 64x96
])
def test_outside_the_kernel_is_unsupported_or_exact(M, K, N, supported):
    x, w8, ws, bias, _ = make_case(M, K, N, seed=7, chain=False)
    xd = dev(x)
    w = ops.PackedWeight(dev(w8))
    epi = epilogue_of(dev(ws), dev(bias), [])
    sync = ops.exchange_buffer()
    try:
        fused = ops.gpu_dql_qlinear(xd, w, epi, sync)
    except IconnxError as e:
        assert e.status == 6 and not supported, str(e)  # ICX_ERR_UNSUPPORTED, nothing launched
        return
    assert supported
    assert_same(fused, separate(xd, w, epi), "M=%d K=%d N=%d" % (M, K, N))


def test_repeated_calls_smaller_input_capture_and_failure():
    """Calls in a row share the exchange buffer (the launch number advances), the second
    with fewer rows; a recorded graph of the call replays bit-identically with eager work
    between the replays; then the failure path: with the test hook every wait gives up,
    icx_exchange_status reports ICX_ERR_KERNEL and the scale is NaN, and a normal call
    afterwards is exact again."""
    M, K, N = 4096, 768, 3072
    x, w8, ws, bias, ch = make_case(M, K, N, seed=5)
    w = ops.PackedWeight(dev(w8))
    epi = epilogue_of(dev(ws), dev(bias), [(op, dev(c)) for op, c in ch])
    sync = ops.exchange_buffer()
    L = lib()
    for rows in (M, 1500, M):
        xd = dev(x[:rows] * (1.0 + rows / 1000.0))
        assert_same(ops.gpu_dql_qlinear(xd, w, epi, sync), separate(xd, w, epi), "rows %d" % rows)
    assert L.icx_exchange_status(ops._stream(), ops._p(sync)) == 0
    # capture: fixed buffers, one call recorded
    xin = dev(x)
    y = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    ys = torch.empty((), dtype=torch.float32, device="cuda")
    yz = torch.empty((), dtype=torch.uint8, device="cuda")
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    chn, keep = ops.build_chain(epi(ys), M, N)
    s = torch.cuda.Stream()
    import ctypes
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        rc = L.icx_dql_qlinear_f32(ctypes.c_void_p(s.cuda_stream), ops._p(xin), M, K, ops._p(y), ops._p(ys),
                                   ops._p(yz), ops._p(w.packed), ops._DT[w.dtype], ops._p(w.colsum), N, ctypes.byref(chn),
                                   ops._p(Y), ops._p(sync))
    assert rc == 0
    for rep in range(3):
        src = dev(x * (1.0 + rep))
        xin.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        assert_same((y, ys, yz, Y), separate(src, w, epi), "replay %d" % rep)
        _ = (src * 2.0).sum().item()  # eager work between the replays
    assert L.icx_exchange_status(ops._stream(), ops._p(sync)) == 0
    del keep
    # failure path
    L.icx_debug_qout_fault(64)
    try:
        bad = ops.gpu_dql_qlinear(dev(x), w, epi, sync)
        rc = L.icx_exchange_status(ops._stream(), ops._p(sync))
    finally:
        L.icx_debug_qout_fault(0)
    assert rc == 7
    assert np.isnan(bad[1].cpu().numpy())
    assert L.icx_exchange_status(ops._stream(), ops._p(sync)) == 0  # cleared
    xd = dev(x)
    assert_same(ops.gpu_dql_qlinear(xd, w, epi, sync), separate(xd, w, epi), "after the failure")


# ---- through the graph executor -----------------------------------------------------------
def qlinear_graph(ex, K, N, gelu, seed):
    from tests.test_gpu_quant_out import build
    h = build(ex, K, N, gelu, seed)
    ex.add_node("after", "Add", [h, h], ["out"])  # a reader other than a DQL: h is formed
    return h


@pytest.mark.parametrize("M,K,N,gelu,fused", [
    (4096, 768, 3072, False, True),   # cfg2's shape
    (1000, 768, 3072, True, True),    # erf-GELU chain, ragged last panel
    (4096, 768, 768, False, True),    # 64x96 tiles
    (128, 768, 768, True, False),     # the erf-GELU chain on 64x96 tiles: the DQL on its own first
])
def test_executor_runs_the_input_dql_in_the_gemm_launch(M, K, N, gelu, fused):
    """GpuGraphExecutor plans the DQL whose outputs only one quantized-linear head reads into
    that head's launch; the results equal the same graph with the fusions off (every DQL its
    own launch), including the DQL's outputs requested as graph outputs."""
    from iconnx_amd.executor import GpuGraphExecutor

    x = (np.random.default_rng(M + N).standard_normal((M, K)) * 2.0).astype(np.float32)
    ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    h = qlinear_graph(ex, K, N, gelu, seed=3)
    qlinear_graph(ref_ex, K, N, gelu, seed=3)
    ref_ex.set_option("quantized_outputs", False)
    names = ["out", h, "xq", "xs", "xzp"]
    want = ref_ex.run({"x": x}, names)
    assert ref_ex.quantized_inputs() == ({}, 0)
    for rep in range(2):
        got = ex.run({"x": x * (1.0 + rep)}, names)
        want = ref_ex.run({"x": x * (1.0 + rep)}, names)
        for n in names:
            bad = int(np.count_nonzero(bits(got[n]) != bits(want[n])))
            assert bad == 0, "run %d %s: %d of %d differ" % (rep, n, bad, want[n].size)
    planned, launches = ex.quantized_inputs()
    assert planned == {h: "dql_x"}
    assert launches == (2 if fused else 0)
    ex.check_status()


@pytest.mark.parametrize("case", ["nan_zero_subnormal", "all_zero", "huge", "one_sided"])
def test_special_values_equal_the_two_launches(case):
    """The DQL's edge cases inside the fused launch: NaN skipped by the range and quantized to
    0 (the reference's saturating cast of NaN), -0.0 and
    subnormals, an all-zero input (empty range: scale 0, zero point 0, y all 0), magnitudes
    near the f32 limit, and an input that is all positive (range [0, max]).  Bit-identical to
    the DQL launch followed by the GEMM; the DQL outputs also equal the oracle's."""
    M, K, N = 1024, 768, 3072
    rng = np.random.default_rng(17)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if case == "nan_zero_subnormal":
        x[::7, ::5] = np.nan
        x[1::9, ::3] = -0.0
        x[2::11, 1::4] = np.float32(1e-41)
    elif case == "all_zero":
        x[:] = 0.0
    elif case == "huge":
        x *= np.float32(1e37)
    else:
        x = np.abs(x) + np.float32(0.25)
    w8 = rng.integers(-127, 128, (K, N)).astype(np.int8)
    xd, w = dev(x), ops.PackedWeight(dev(w8))
    epi = epilogue_of(dev(np.array(0.003, np.float32)), dev((0.02 * rng.standard_normal(N)).astype(np.float32)), [])
    sync = ops.exchange_buffer()
    fused = ops.gpu_dql_qlinear(xd, w, epi, sync)
    ref = separate(xd, w, epi)
    torch.cuda.synchronize()
    assert lib().icx_exchange_status(ops._stream(), ops._p(sync)) == 0
    assert_same(fused, ref, case)
    yq, ys, yz = oracle.dynamic_quantize_linear(x)
    assert np.array_equal(fused[0].cpu().numpy(), yq)
    assert bits(fused[1].cpu().numpy()) == bits(np.float32(ys)) and int(fused[2].cpu().numpy()) == int(yz)


def test_cfg2_graph_with_a_3d_activation_runs_as_one_launch():
    """cfg2 as its graph (x [32, 128, 768] with dynamic batch and sequence dims, the chain of
    the config) through GpuGraphExecutor: the DQL runs inside the GEMM's launch, the output
    keeps x's leading dims, and every output equals the graph with the fusions off — also
    captured and replayed, and again with a smaller batch."""
    from iconnx_amd import graphs
    from iconnx_amd.executor import GpuGraphExecutor

    ex, ref_ex = GpuGraphExecutor(), GpuGraphExecutor()
    y, d = graphs.config_graph(ex, "cfg2")
    graphs.config_graph(ref_ex, "cfg2")
    ref_ex.set_option("quantized_outputs", False)
    names = [y, "cfg2.x_q", "cfg2.x_scale", "cfg2.x_zp"]
    for batch in (32, 5):
        x = d["x"][:batch]
        got, want = ex.run({"x": x}, names), ref_ex.run({"x": x}, names)
        assert got[y].shape == (batch, 128, 3072)
        for n in names:
            bad = int(np.count_nonzero(bits(got[n]) != bits(want[n])))
            assert bad == 0, "batch %d %s: %d of %d differ" % (batch, n, bad, want[n].size)
    planned, launches = ex.quantized_inputs()
    assert planned == {y: "cfg2.dql"} and launches == 2
    xin = torch.from_numpy(np.ascontiguousarray(d["x"])).cuda()
    ex.capture({"x": xin}, [y])
    want = ref_ex.run({"x": d["x"]}, [y])[y]
    for rep in range(2):
        ex.replay()
        got = ex.outputs([y])[y].cpu().numpy()
        ex.check_status()
        assert np.array_equal(bits(got), bits(want)), "replay %d" % rep
