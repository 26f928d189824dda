"""GPU parity: MatMulInteger on int8 MFMA vs the oracle — bit-exact int32.

Mirrors tests/matmul_integer_test.rs:34-171 of the reference (exact equality with the CPU
forward), then covers every sign combination, zero points, ragged shapes (K not a multiple
of 16, M/N not multiples of the 128 tile), packed and unpacked weights, the per-column
b_zero_point extension and the BASELINE GEMM shapes (row samples against the oracle plus
full-size checks by exact float64 products and column checksums).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import configs, ops
from iconnx_amd._lib import IconnxError
from tests.golden_util import tensor

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_mmi(a, b, azp=None, bzp=None, packed=False, rowsum=None):
    bb = ops.PackedWeight(dev(b)) if packed else dev(b)
    out = ops.gpu_matmul_integer(dev(a), bb, None if azp is None else dev(azp),
                                 None if bzp is None else dev(bzp),
                                 a_rowsum=None if rowsum is None else dev(rowsum))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_onnx_golden(goldens):
    g = goldens["test_matmulinteger"]
    a, b, azp, bzp = (tensor(t) for t in g["inputs"])
    for packed in (False, True):
        np.testing.assert_array_equal(gpu_mmi(a, b, azp, bzp, packed), tensor(g["outputs"][0]))


def test_reference_contract_literals():
    a = np.array([1, 2, 3, 4, 5, 6], np.uint8).reshape(2, 3)
    b = np.array([1, 2, 3, 4, 5, 6], np.int8).reshape(3, 2)
    assert gpu_mmi(a, b).reshape(-1).tolist() == [22, 28, 49, 64]
    out = gpu_mmi(np.ones((4, 768), np.uint8), np.ones((768, 4), np.int8))
    assert out.shape == (4, 4) and np.all(out == 768)
    out = gpu_mmi(np.full((1, 3072), 100, np.uint8), np.full((3072, 1), 100, np.int8))
    assert out.shape == (1, 1) and int(out[0, 0]) == 30_720_000
    out = gpu_mmi(np.array([10, 20, 30, 40], np.int8).reshape(2, 2),
                  np.array([1, 2, 3, 4], np.int8).reshape(2, 2),
                  np.array(5, np.int8), np.array(1, np.int8))
    assert out.reshape(-1).tolist() == [30, 50, 70, 130]


def test_rejects_like_reference():
    f = torch.ones((2, 2), dtype=torch.float32, device="cuda")
    i8 = torch.ones((2, 2), dtype=torch.int8, device="cuda")
    with pytest.raises(IconnxError):
        ops.gpu_matmul_integer(f, i8)  # non-int8 a
    with pytest.raises(IconnxError):
        ops.gpu_matmul_integer(torch.ones(3, dtype=torch.int8, device="cuda"), i8)  # rank 1
    with pytest.raises(IconnxError):
        ops.gpu_matmul_integer(torch.ones((2, 3), dtype=torch.int8, device="cuda"),
                               torch.ones((4, 2), dtype=torch.int8, device="cuda"))  # K
    with pytest.raises(IconnxError):  # per-axis a zero point
        ops.gpu_matmul_integer(i8, i8, torch.zeros(2, dtype=torch.int8, device="cuda"))
    with pytest.raises(IconnxError):  # zp dtype mismatch
        ops.gpu_matmul_integer(i8, i8, torch.zeros((), dtype=torch.uint8, device="cuda"))


@pytest.mark.parametrize("adt,bdt", [(np.uint8, np.int8), (np.int8, np.int8),
                                     (np.int8, np.uint8), (np.uint8, np.uint8)])
@pytest.mark.parametrize("packed", [False, True])
def test_sign_combinations_zero_points_ragged(adt, bdt, packed):
    rng = np.random.default_rng(17)
    shapes = [(1, 1, 1), (2, 3, 2), (5, 16, 7), (33, 64, 65), (130, 100, 129),
              (128, 768, 128), (257, 48, 255), (64, 3072, 96)]
    for M, K, N in shapes:
        a = rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1, (M, K)).astype(adt)
        b = rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1, (K, N)).astype(bdt)
        azp = np.array(rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1), adt)
        bzp = np.array(rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1), bdt)
        for zps in ((None, None), (azp, None), (None, bzp), (azp, bzp)):
            want = oracle.matmul_integer(a, b, *zps)
            got = gpu_mmi(a, b, *zps, packed=packed)
            assert np.array_equal(got, want), (M, K, N, zps)


def test_per_column_b_zero_point():
    rng = np.random.default_rng(4)
    M, K, N = 300, 1024, 520
    a = rng.integers(0, 256, (M, K)).astype(np.uint8)
    b = rng.integers(-127, 128, (K, N)).astype(np.int8)
    azp = np.array(141, np.uint8)
    bzp = rng.integers(-8, 9, N).astype(np.int8)
    want = oracle.matmul_integer(a, b, azp, bzp, per_column_b_zp=True)
    for packed in (False, True):
        np.testing.assert_array_equal(gpu_mmi(a, b, azp, bzp, packed), want)
    # with the DQL-style raw row sums supplied instead of computed
    rs = a.astype(np.int64).sum(1).astype(np.int32)
    np.testing.assert_array_equal(gpu_mmi(a, b, azp, bzp, True, rowsum=rs), want)


def test_wraparound_matches_int32_modular_arithmetic():
    """Past INT32 the reference CPU op panics and its GPU kernel wraps; the MFMA path wraps
    identically (the zero-point expansion is exact modulo 2^32)."""
    K = 40000
    a = np.full((2, K), 255, np.uint8)
    b = np.full((K, 3), -128, np.int8)
    bzp = np.array(127, np.int8)
    got = gpu_mmi(a, b, None, bzp)
    want = np.int64(255) * np.int64(-255) * K
    wrapped = ((want + 2**31) % 2**32) - 2**31
    assert np.all(got == wrapped)
    with pytest.raises(oracle.OracleError):
        oracle.matmul_integer(a, b, None, bzp)


def _exact_f64(a, b, azp, bzp):
    """Full-size exact reference on the GPU: integer operands as float64 (every product and
    partial sum is an integer below 2^53, so float64 GEMM is exact)."""
    A = dev(a).to(torch.float64) - float(azp)
    B = dev(b).to(torch.float64) - torch.from_numpy(np.asarray(bzp, np.float64)).cuda()
    return (A @ B).round().to(torch.int64).cpu().numpy()


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg4", "cfg5a"])
def test_baseline_gemm_shapes(cfg):
    d = configs.make(cfg)
    if cfg == "cfg5a":
        a, b, azp, bzp = d["a"], d["b"], d["a_zp"], d["b_zp"]
    else:
        x = d["x"].reshape(-1, d["x"].shape[-1])
        a, _, azp = oracle.dynamic_quantize_linear(x)
        b, bzp = d["w"], d["w_zp"]
    per_col = np.asarray(bzp).ndim == 1
    M = a.shape[0]
    got = gpu_mmi(a, b, azp, bzp, packed=True)
    # rows sampled across the whole M range against the oracle (bit-exact)
    rows = sorted(set([0, 1, M // 2, M - 1] + list(range(100, min(M, 132)))))
    for r in rows:
        want = oracle.matmul_integer(a[r:r + 1], b, azp, bzp, per_column_b_zp=per_col)
        assert np.array_equal(got[r:r + 1], want), (cfg, r)
    # every element against the exact float64 product
    np.testing.assert_array_equal(got.astype(np.int64), _exact_f64(a, b, azp, bzp))
    # column checksum: sum_m C[m,n] == (sum_m (a - azp)) . (b - bzp)
    lhs = got.astype(np.int64).sum(0)
    ra = (a.astype(np.int64) - int(azp)).sum(0)
    rhs = ra @ (b.astype(np.int64) - np.asarray(bzp, np.int64))
    np.testing.assert_array_equal(lhs, rhs)


# Shapes with K >= 2048 and fewer 64x64 tiles than CUs take the persistent producer /
# consumer kernel; the rest of this file covers the multi-block kernels.
@pytest.mark.parametrize("adt,bdt", [(np.uint8, np.int8), (np.int8, np.uint8)])
def test_persistent_kernel_shapes(adt, bdt):
    rng = np.random.default_rng(23)
    for M, K, N in [(512, 2048, 384), (300, 3072, 520), (64, 4096, 64), (129, 2112, 257)]:
        a = rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1, (M, K)).astype(adt)
        b = rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1, (K, N)).astype(bdt)
        azp = np.array(rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1), adt)
        bzp = np.array(rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1), bdt)
        bzp_col = rng.integers(-8, 9, N).astype(bdt)
        for zps in ((None, None), (azp, bzp), (azp, bzp_col)):
            per_col = zps[1] is not None and np.asarray(zps[1]).ndim == 1
            want = oracle.matmul_integer(a, b, *zps, per_column_b_zp=per_col)
            assert np.array_equal(gpu_mmi(a, b, *zps, packed=True), want), (M, K, N, per_col)
        rs = a.astype(np.int64).sum(1).astype(np.int32)
        want = oracle.matmul_integer(a, b, azp, bzp_col, per_column_b_zp=True)
        assert np.array_equal(gpu_mmi(a, b, azp, bzp_col, True, rowsum=rs), want)


def test_encoder_ffn_down_shape():
    """The DistilBERT FFN-down GEMM (4096 x 3072 x 768, 128x96 tiles) at full size: every
    element against the exact float64 product, rows against the oracle."""
    rng = np.random.default_rng(29)
    a = rng.integers(0, 256, (4096, 3072)).astype(np.uint8)
    b = rng.integers(-127, 128, (3072, 768)).astype(np.int8)
    azp, bzp = np.array(117, np.uint8), np.array(0, np.int8)
    got = gpu_mmi(a, b, azp, bzp, packed=True)
    np.testing.assert_array_equal(got.astype(np.int64), _exact_f64(a, b, azp, bzp))
    for r in (0, 2049, 4095):
        assert np.array_equal(got[r:r + 1], oracle.matmul_integer(a[r:r + 1], b, azp, bzp))


# At least 512 tiles of 256x256 take the large-tile kernels: K % 128 == 0 the 128-byte-row
# main loop, K % 128 == 64 the 64-byte-row one.  Ragged M / N exercise the clamped rows.
@pytest.mark.parametrize("K", [256, 320])
@pytest.mark.parametrize("adt,bdt", [(np.uint8, np.int8), (np.int8, np.uint8)])
def test_large_tile_kernels_ragged(K, adt, bdt):
    rng = np.random.default_rng(31 + K)
    M, N = 8000, 4100
    a = rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1, (M, K)).astype(adt)
    b = rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1, (K, N)).astype(bdt)
    azp = np.array(rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1), adt)
    bzp = np.array(rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1), bdt)
    got = gpu_mmi(a, b, azp, bzp, packed=True)
    np.testing.assert_array_equal(got.astype(np.int64), _exact_f64(a, b, azp, bzp))
    for r in (0, 255, 256, 4001, M - 1):
        assert np.array_equal(got[r:r + 1], oracle.matmul_integer(a[r:r + 1], b, azp, bzp)), r


# 256x192 tiles (12 waves) when they give every CU at least one: N % 192 == 0, K % 128 == 0,
# cdiv(M, 256) * N / 192 >= CUs; ragged M exercises the clamped rows.
@pytest.mark.parametrize("M", [4000, 4100])
def test_mid_tile_kernel_ragged(M):
    rng = np.random.default_rng(37 + M)
    K, N = 256, 3072
    a = rng.integers(0, 256, (M, K)).astype(np.uint8)
    b = rng.integers(-128, 128, (K, N)).astype(np.int8)
    azp, bzp = np.array(131, np.uint8), np.array(-3, np.int8)
    got = gpu_mmi(a, b, azp, bzp, packed=True)
    np.testing.assert_array_equal(got.astype(np.int64), _exact_f64(a, b, azp, bzp))
    for r in (0, 255, 256, 3999, M - 1):
        assert np.array_equal(got[r:r + 1], oracle.matmul_integer(a[r:r + 1], b, azp, bzp)), r


# 128x96 tiles (12 waves of 32x32) when they give every CU at least one: N % 96 == 0,
# K % 128 == 0, cdiv(M, 128) * N / 96 >= CUs, not taken by a larger tile; ragged M exercises
# the clamped rows.
@pytest.mark.parametrize("M,K", [(4000, 256), (4100, 768)])
def test_narrow_tile_kernel_ragged(M, K):
    rng = np.random.default_rng(41 + M)
    N = 768
    a = rng.integers(0, 256, (M, K)).astype(np.uint8)
    b = rng.integers(-128, 128, (K, N)).astype(np.int8)
    azp, bzp = np.array(7, np.uint8), np.array(5, np.int8)
    got = gpu_mmi(a, b, azp, bzp, packed=True)
    np.testing.assert_array_equal(got.astype(np.int64), _exact_f64(a, b, azp, bzp))
    for r in (0, 127, 128, 3999, M - 1):
        assert np.array_equal(got[r:r + 1], oracle.matmul_integer(a[r:r + 1], b, azp, bzp)), r
