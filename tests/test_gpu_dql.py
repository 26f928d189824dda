"""GPU parity: DynamicQuantizeLinear (HIP) vs the oracle — bit-exact y, scale, zero point.

Mirrors tests/dynamic_quantize_linear_test.rs:28-136 of the reference (exact equality with
the CPU forward) and extends it to the BASELINE sizes, tie cases, NaN and the row sums.
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import configs, ops
from iconnx_amd._lib import IconnxError
from tests.golden_util import bits, tensor

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run(x_np, row_len=None):
    outs = ops.gpu_dynamic_quantize_linear(dev(x_np), rowsum_row_len=row_len)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def assert_dql_equal(x_np, row_len=None):
    ey, es, ezp = oracle.dynamic_quantize_linear(x_np)
    got = run(x_np, row_len)
    y, s, zp = got[:3]
    assert y.shape == ey.shape and s.shape == () and zp.shape == ()
    mism = np.count_nonzero(y != ey)
    assert mism == 0, "%d of %d y elements differ" % (mism, y.size)
    assert bits(s) == bits(es), (float(s), float(es))
    assert int(zp) == int(ezp)
    if row_len:
        ers = ey.reshape(-1, row_len).astype(np.int64).sum(1)
        np.testing.assert_array_equal(got[3], ers)


@pytest.mark.parametrize("case", ["test_dynamicquantizelinear",
                                  "test_dynamicquantizelinear_max_adjusted",
                                  "test_dynamicquantizelinear_min_adjusted"])
def test_onnx_goldens(goldens, case):
    g = goldens[case]
    assert_dql_equal(tensor(g["inputs"][0]))


def test_reference_contract_literals(literals):
    y, s, zp = run(np.array([0.0, 2.0, 4.0], np.float32))
    assert y.tolist() == [0, 128, 255] and int(zp) == 0
    _, _, zp = run(np.array([-1.0, 0.0, 1.0], np.float32))
    assert int(zp) == 128
    y, s, zp = run(np.zeros(5, np.float32))
    assert y.tolist() == [0] * 5 and float(s) == 0.0 and int(zp) == 0
    x = (np.arange(24, dtype=np.float32) * np.float32(0.1)).reshape(2, 3, 4)
    assert_dql_equal(x)


def test_rejects_non_float_input():
    with pytest.raises(IconnxError):
        ops.gpu_dynamic_quantize_linear(torch.tensor([1, 2, 3], dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("n", [1, 3, 15, 16, 17, 63, 1000, 4099, 65536 + 7, 1 << 20])
def test_sizes_and_tails(n):
    rng = np.random.default_rng(n)
    assert_dql_equal((rng.standard_normal(n) * 2).astype(np.float32))


def test_ties_nan_signed_zero_and_constant():
    rng = np.random.default_rng(0)
    x = (rng.integers(-64, 64, 100003) / 4.0).astype(np.float32)  # dense exact ties
    assert_dql_equal(x)
    x[::97] = np.nan
    x[5] = -0.0
    assert_dql_equal(x)
    assert_dql_equal(np.full(4097, np.nan, np.float32))
    assert_dql_equal(np.full(1000, 3.5, np.float32))  # all positive: min is 0
    assert_dql_equal(np.full(1000, -3.5, np.float32))


def test_unaligned_input():
    rng = np.random.default_rng(9)
    base = torch.from_numpy(rng.standard_normal(4097).astype(np.float32)).cuda()
    x = base[1:]  # 4-byte aligned only: exercises the scalar path
    outs = ops.gpu_dynamic_quantize_linear(x)
    ey, es, ezp = oracle.dynamic_quantize_linear(x.cpu().numpy())
    assert np.array_equal(outs[0].cpu().numpy(), ey)
    assert bits(outs[1].cpu().numpy()) == bits(es) and int(outs[2].cpu()) == int(ezp)


@pytest.mark.parametrize("row_len", [768, 1024, 3072, 7])
def test_rowsums(row_len):
    rng = np.random.default_rng(row_len)
    x = rng.standard_normal((97, row_len)).astype(np.float32)
    assert_dql_equal(x, row_len=row_len)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg4"])
def test_baseline_activations_full_size(cfg):
    """Bit-exact at the configs' full activation sizes (the C oracle runs them in <1 s)."""
    x = configs.make(cfg)["x"]
    assert_dql_equal(x, row_len=x.shape[-1])


def test_size_independent_invariants_full_cfg4():
    x = configs.make("cfg4")["x"]
    y, s, zp = run(x)
    # zero maps to zp; y is monotone in x; the extremes hit 0 and 255
    order = np.argsort(x.reshape(-1), kind="stable")
    ys = y.reshape(-1)[order].astype(np.int64)
    assert np.all(np.diff(ys) >= 0)
    assert ys[0] == 0 and ys[-1] == 255
    z = run(np.concatenate([x.reshape(-1), np.zeros(1, np.float32)]))
    assert int(z[0][-1]) == int(z[2])


def test_near_tie_quotients_and_extreme_scales():
    """Quotients x/scale placed at controlled distances from half-integers (inside and
    outside the f32 fast path's 1e-4 guard band), subnormal inputs, and scales outside
    [1e-30, 1e30] where only the f64 path is used."""
    lo, hi = np.float32(-1.7), np.float32(2.9)
    s = (np.float64(hi) - np.float64(lo)) / 255.0
    vals = [lo, hi, np.float32(0.0)]
    for k in range(-100, 150, 7):
        for d in (0.0, 1e-7, 1e-6, 1e-5, 3e-5, 9e-5, 1e-4, 1.2e-4, 5e-4, 1e-2):
            for sign in (1.0, -1.0):
                vals.append(np.float32((k + 0.5 + sign * d) * s))
    x = np.array(vals, np.float32)
    assert_dql_equal(x)
    assert_dql_equal(np.ascontiguousarray(np.tile(x, 37)[: 37 * len(x) - 3]))
    # subnormal elements next to normal ones
    sub = np.array([1e-40, -3e-39, 2e-45, 0.5, -0.25] * 50, np.float32)
    assert_dql_equal(sub)
    # tiny and huge scales (outside the fast path's range)
    rng = np.random.default_rng(3)
    assert_dql_equal((rng.standard_normal(5000) * 1e-33).astype(np.float32))
    assert_dql_equal((rng.standard_normal(5000) * 1e33).astype(np.float32))
