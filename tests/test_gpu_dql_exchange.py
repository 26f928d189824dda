"""GPU parity of the single-launch DynamicQuantizeLinear the graph executor runs for an input
of up to 1024 resident blocks of 256 lanes holding 1, 2 or 4 float4 each (4 Mi elements,
e.g. the encoder's [32, 128, 768] activation) when no producer left the input's range and
no GEMM reads row sums of its output: the blocks keep x in registers and trade their
(min, max) through the graph's exchange buffer.

The bar is the two-launch path's: y, scale and zero point bit-exact against the oracle
(DynamicQuantizeLinear::forward, src/operators/dynamic_quantize_linear.rs:32-112; the
reference's own test is tests/dynamic_quantize_linear_test.rs:28-136), over sizes that
take one to 1024 blocks at each of the three widths, the scalar tail, the edge values the
two-launch tests cover, inputs past the limit (two-launch fallback), captured replays, and
the failure path of the exchange.
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd._lib import IconnxError, lib
from iconnx_amd.executor import GpuGraphExecutor
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def dql_graph():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None])
    ex.add_node("dql", "DynamicQuantizeLinear", ["x"], ["y", "s", "zp"])
    return ex


def check_oracle(got, x, what):
    ey, es, ezp = oracle.dynamic_quantize_linear(x)
    bad = int(np.count_nonzero(got["y"] != ey))
    assert bad == 0, "%s: %d of %d y elements differ" % (what, bad, ey.size)
    assert bits(got["s"]) == bits(es), (what, float(got["s"]), float(es))
    assert int(got["zp"]) == int(ezp), what


# 256 lanes per block holding 1 float4 each up to 1024 blocks (1 Mi elements), then 2, then 4
# (4 Mi elements); with and without a scalar tail, and each width's first and last grid
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 1024, 1025, 65536 + 7, 128 * 768, 128 * 1024,
                               128 * 1024 + 3, 128 * 1024 + 4, (1 << 20) + 3, (1 << 20) + 4,
                               (2 << 20) + 3, (2 << 20) + 5, 4096 * 768, (4 << 20) + 3])
def test_single_launch_matches_oracle(n):
    x = (np.random.default_rng(n).standard_normal(n) * 3.0).astype(np.float32)
    ex = dql_graph()
    got = ex.run({"x": x}, ["y", "s", "zp"])
    assert ex.single_launch_dqls() == 1, "the single-launch DQL did not run"
    check_oracle(got, x, "n=%d" % n)


def test_edge_values():
    """Dense exact ties, NaN, signed zero, constant inputs, subnormals, extreme scales and
    near-tie quotients (the cases of the two-launch tests), each as a single launch."""
    rng = np.random.default_rng(0)
    cases = []
    x = (rng.integers(-64, 64, 100003) / 4.0).astype(np.float32)
    cases.append(x.copy())
    x[::97] = np.nan
    x[5] = -0.0
    cases.append(x)
    cases += [np.full(4097, np.nan, np.float32), np.full(1000, 3.5, np.float32),
              np.full(1000, -3.5, np.float32), np.zeros(77, np.float32),
              np.array([1e-40, -3e-39, 2e-45, 0.5, -0.25] * 50, np.float32),
              (rng.standard_normal(5000) * 1e-33).astype(np.float32),
              (rng.standard_normal(5000) * 1e33).astype(np.float32),
              np.array([0.0, 2.0, 4.0], np.float32), np.array([-1.0, 0.0, 1.0], np.float32)]
    lo, hi = np.float32(-1.7), np.float32(2.9)
    s = (np.float64(hi) - np.float64(lo)) / 255.0
    vals = [lo, hi, np.float32(0.0)]
    for k in range(-100, 150, 7):
        for d in (0.0, 1e-7, 1e-6, 1e-5, 3e-5, 9e-5, 1e-4, 1.2e-4, 5e-4, 1e-2):
            for sign in (1.0, -1.0):
                vals.append(np.float32((k + 0.5 + sign * d) * s))
    cases.append(np.array(vals, np.float32))
    ex = dql_graph()
    for i, x in enumerate(cases):
        check_oracle(ex.run({"x": x}, ["y", "s", "zp"]), x, "case %d" % i)
    assert ex.single_launch_dqls() == len(cases)


def test_reference_literals():
    """The reference test's literal expectations (dynamic_quantize_linear_test.rs:28-136)."""
    ex = dql_graph()
    got = ex.run({"x": np.array([0.0, 2.0, 4.0], np.float32)}, ["y", "s", "zp"])
    assert got["y"].tolist() == [0, 128, 255] and int(got["zp"]) == 0
    got = ex.run({"x": np.array([-1.0, 0.0, 1.0], np.float32)}, ["y", "s", "zp"])
    assert int(got["zp"]) == 128
    got = ex.run({"x": np.zeros(5, np.float32)}, ["y", "s", "zp"])
    assert got["y"].tolist() == [0] * 5 and float(got["s"]) == 0.0 and int(got["zp"]) == 0


def test_consecutive_runs_of_different_sizes():
    """Launches of different grids in a row share the exchange buffer: each leaves it at
    rest for the next (the launch number advances, the counter is back at 0)."""
    ex = dql_graph()
    rng = np.random.default_rng(5)
    for i, n in enumerate((128 * 768, 1000, 4096 * 768, 128 * 1024 + 3, 3, (2 << 20) + 5, 128 * 768)):
        x = (rng.standard_normal(n) * (1.0 + i)).astype(np.float32)
        check_oracle(ex.run({"x": x}, ["y", "s", "zp"]), x, "run %d (n=%d)" % (i, n))
    assert ex.single_launch_dqls() == 7


@pytest.mark.parametrize("n", [(4 << 20) + 4, 24576 * 1024])
def test_larger_inputs_take_two_launches(n):
    """Past 1024 blocks of 4 float4 per lane (one float4 more than the limit; cfg4's
    activation) the DQL runs as two launches; the results are the same."""
    x = (np.random.default_rng(n).standard_normal(n) * 3.0).astype(np.float32)
    ex = dql_graph()
    got = ex.run({"x": x}, ["y", "s", "zp"])
    assert ex.single_launch_dqls() == 0
    check_oracle(got, x, "n=%d (two launches)" % n)


def test_capture_and_replay():
    """Recorded into a HIP graph and replayed with new data in the bound input, eager work
    and synchronisations between replays: every replay matches the oracle."""
    n = 128 * 768
    xs = [(np.random.default_rng(s).standard_normal(n) * (s + 1)).astype(np.float32) for s in range(3)]
    xs[2][123] = np.nan
    ex = dql_graph()
    xin = torch.from_numpy(xs[0]).cuda()
    ex.capture({"x": xin}, ["y", "s", "zp"])
    for rep in range(6):
        i = rep % 3
        xin.copy_(torch.from_numpy(xs[i]))
        ex.replay()
        got = {k: v.cpu().numpy() for k, v in ex.outputs(["y", "s", "zp"]).items()}
        ex.check_status()
        check_oracle(got, xs[i], "replay %d" % rep)
        _ = (xin * 2.0).sum().item()
        torch.cuda.synchronize()


def test_exchange_that_gives_up_is_an_error_status():
    """The host-side test hook makes every wait expect a tag no block publishes, with a short
    bound: every block exits through the failure path (y = 0), the scale is NaN, and the
    status check reports ICX_ERR_KERNEL once; a normal run afterwards is correct."""
    n = 128 * 768
    x = np.random.default_rng(8).standard_normal(n).astype(np.float32)
    ex = dql_graph()
    L = lib()
    L.icx_debug_qout_fault(64)
    try:
        got = ex.run_device({"x": x}, ["y", "s", "zp"])
        with pytest.raises(IconnxError) as e:
            ex.check_status()
    finally:
        L.icx_debug_qout_fault(0)
    assert e.value.status == 7 and "range exchange" in str(e.value)
    assert np.isnan(got["s"].cpu().numpy()) and not got["y"].cpu().numpy().any()
    ex.check_status()  # cleared
    check_oracle(ex.run({"x": x}, ["y", "s", "zp"]), x, "normal run after the failure")
    assert ex.single_launch_dqls() == 2


def test_c_abi_single_launch_op():
    """icx_dynamic_quantize_linear_exchange on one zeroed buffer kept across calls (what a
    per-op caller does): calls of six sizes in a row, each bit-exact against the oracle and
    checked clean by icx_exchange_status; an input past the limit is ICX_ERR_UNSUPPORTED
    with nothing launched; with the test hook every block's wait gives up, the status check
    reports ICX_ERR_KERNEL once (y = 0, scale NaN), and the next call is correct again."""
    import ctypes

    from iconnx_amd._lib import ICX_ERR_KERNEL, ICX_ERR_UNSUPPORTED

    L = lib()
    P = ctypes.c_void_p
    sync = torch.zeros(L.icx_exchange_buffer_size(), dtype=torch.uint8, device="cuda")
    stream = P(torch.cuda.current_stream().cuda_stream)

    def call(x):
        xd = torch.from_numpy(x).cuda()
        y = torch.empty(x.size, dtype=torch.uint8, device="cuda")
        s = torch.empty((), dtype=torch.float32, device="cuda")
        zp = torch.empty((), dtype=torch.uint8, device="cuda")
        rc = L.icx_dynamic_quantize_linear_exchange(stream, P(xd.data_ptr()), x.size, P(y.data_ptr()),
                                                    P(s.data_ptr()), P(zp.data_ptr()), P(sync.data_ptr()))
        return rc, {"y": y, "s": s, "zp": zp}

    rng = np.random.default_rng(21)
    for n in (3, 1000, 128 * 1024 + 3, (1 << 20) + 4, 4096 * 768, 4 << 20):
        x = (rng.standard_normal(n) * 2.5).astype(np.float32)
        rc, out = call(x)
        assert rc == 0, L.icx_last_error()
        assert L.icx_exchange_status(stream, P(sync.data_ptr())) == 0
        check_oracle({k: v.cpu().numpy() for k, v in out.items()}, x, "C ABI n=%d" % n)
    rc, _ = call(np.ones((4 << 20) + 4, np.float32))
    assert rc == ICX_ERR_UNSUPPORTED
    x = (rng.standard_normal(4096 * 768)).astype(np.float32)
    L.icx_debug_qout_fault(64)
    try:
        rc, bad = call(x)
        assert rc == 0
        assert L.icx_exchange_status(stream, P(sync.data_ptr())) == ICX_ERR_KERNEL
    finally:
        L.icx_debug_qout_fault(0)
    assert np.isnan(bad["s"].cpu().numpy()) and not bad["y"].cpu().numpy().any()
    assert L.icx_exchange_status(stream, P(sync.data_ptr())) == 0  # cleared by the check
    rc, out = call(x)
    assert rc == 0 and L.icx_exchange_status(stream, P(sync.data_ptr())) == 0
    check_oracle({k: v.cpu().numpy() for k, v in out.items()}, x, "C ABI after the give-up")
