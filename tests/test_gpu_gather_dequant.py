"""GPU parity of Gather (the UINT8 embedding front end of DistilBERT-INT8) and of the
MatMulInteger -> DequantizeLinear form of the quantized linear, fused into the GEMM store.

* Gather: the ONNX goldens through the per-op wrapper (gpu_gather_from_gpu,
  src/cuda/ops/layout/mod.rs:900; gather_u8_kernel, src/cuda/ops/quantize_kernels.rs:203-224),
  then Gather(UInt8 table [vocab, 768], Int64 ids) -> DequantizeLinear through
  GpuGraphExecutor, bit-exact against the oracle (gather then DequantizeLinear, the CPU
  forward's (x as f32 - zp as f32) * scale, src/operators/dequantize_linear.rs:158-174).
* MatMulInteger -> DequantizeLinear -> Add: the plan holds one QuantizedLinear head (the
  DequantizeLinear becomes Sub(zp as f32), Mul(scale) after the GEMM's Cast), and its output
  is bit-exact against the oracle's op-by-op MatMulInteger, DequantizeLinear, Add — per-tensor
  and per-column scales and zero points, 2-D and 3-D activations — and equal to the same graph
  run unfused (the accumulator requested as an output).
"""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import graphs, ops
from iconnx_amd.executor import GpuGraphExecutor
from tests.golden_util import bits, tensor

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("case", ["test_gather_0", "test_gather_1", "test_gather_2d_indices",
                                  "test_gather_negative_indices"])
def test_gather_onnx_goldens(goldens, case):
    g = goldens[case]
    data, idx = (tensor(t) for t in g["inputs"])
    axis = (g["attributes"] or {}).get("axis", 0)
    got = ops.gpu_gather_from_gpu(dev(data), dev(idx), axis=axis).cpu().numpy()
    want = tensor(g["outputs"][0])
    assert got.shape == want.shape
    assert np.array_equal(bits(got), bits(want))
    # Int32 indices give the same result
    got32 = ops.gpu_gather_from_gpu(dev(data), dev(idx.astype(np.int32)), axis=axis).cpu().numpy()
    assert np.array_equal(bits(got32), bits(want))


@pytest.mark.parametrize("dtype,shape,axis", [(np.uint8, (50, 33), 0), (np.int8, (7, 9, 5), 1),
                                              (np.int32, (4, 6, 3), 2), (np.int64, (9, 2), 0),
                                              (np.uint8, (100, 3), 0)])
def test_gather_dtypes_axes_and_clamped_indices(dtype, shape, axis):
    rng = np.random.default_rng(len(shape) + axis)
    info = np.iinfo(dtype)
    data = rng.integers(max(info.min, -1000), min(info.max, 1000) + 1, shape).astype(dtype)
    n = shape[axis]
    idx = rng.integers(-n - 3, n + 3, (3, 4)).astype(np.int64)  # some out of range: clamped
    got = ops.gpu_gather_from_gpu(dev(data), dev(idx), axis=axis).cpu().numpy()
    want = oracle.gather(data, idx, axis=axis)
    assert got.dtype == want.dtype and np.array_equal(got, want)


def test_uint8_embedding_gather_then_dequantize():
    """DistilBERT-INT8's front end at its real size: word_embeddings.weight_quantized is a
    UInt8 [30522, 768] table; input_ids Int64 [32, 128]."""
    rng = np.random.default_rng(30522)
    table = rng.integers(0, 256, (30522, 768)).astype(np.uint8)
    scale, zp = np.float32(0.0123), np.uint8(131)
    ids = rng.integers(0, 30522, (32, 128)).astype(np.int64)
    ids[0, :4] = [-1, -30522, 0, 30521]
    ex = GpuGraphExecutor()
    ex.add_input("ids", [None, None])
    out = graphs.add_quantized_embedding(ex, "ids", table, scale, zp)
    got = ex.run({"ids": dev(ids)}, [out, "emb.q"])
    gathered = oracle.gather(table, ids, axis=0)
    assert np.array_equal(got["emb.q"], gathered)
    want = oracle.dequantize_linear(gathered, np.asarray(scale), np.asarray(zp))
    assert got[out].shape == (32, 128, 768)
    assert np.array_equal(bits(got[out]), bits(want))


@pytest.mark.parametrize("dtype,idx_dt,zp", [(np.uint8, np.int64, 131), (np.int8, np.int32, -7),
                                           (np.uint8, np.int64, None)])
def test_embedding_gather_dequantize_fused(dtype, idx_dt, zp):
    """Only the dequantized embeddings requested: Gather + DequantizeLinear plan as one
    GatherDequantize head, one launch; bit-exact against the oracle's two ops (negative and
    out-of-range indices under the Gather's rules)."""
    rng = np.random.default_rng(768)
    lo, hi = (0, 256) if dtype == np.uint8 else (-128, 128)
    table = rng.integers(lo, hi, (30522, 768)).astype(dtype)
    ids = rng.integers(0, 30522, (32, 128)).astype(idx_dt)
    ids[0, :5] = [-1, -30522, 0, 30521, 30521]
    scale = np.float32(0.0173)
    ex = GpuGraphExecutor()
    ex.add_input("ids", [None, None])
    ex.add_initializer("table", table)
    ex.add_initializer("scale", scale)
    ins = ["q", "scale"]
    if zp is not None:
        ex.add_initializer("zp", np.array(zp, dtype))
        ins.append("zp")
    ex.add_node("g", "Gather", ["table", "ids"], ["q"], {"axis": 0})
    ex.add_node("d", "DequantizeLinear", ins, ["y"])
    got = ex.run({"ids": dev(ids)}, ["y"])["y"]
    live = [e for e in ex.plan()[0] if e.kind != "Skip"]
    assert [e.pattern for e in live] == ["GatherDequantize"]
    want = oracle.dequantize_linear(oracle.gather(table, ids, axis=0), np.asarray(scale),
                                    None if zp is None else np.asarray(zp, dtype))
    assert got.shape == (32, 128, 768) and np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("shape,per_col,zp_kind,axis", [
    ((512, 768), True, "col", 1),
    ((512, 768), False, "scalar", 1),
    ((4, 100, 256), True, "col", 2),
    ((4, 100, 256), False, None, 1),
    ((333, 384), True, "zero", -1),
])
def test_matmul_integer_dequantize_linear_head(shape, per_col, zp_kind, axis):
    K = shape[-1]
    N = 576
    rng = np.random.default_rng(K + N + len(shape))
    a = rng.integers(0, 256, shape).astype(np.uint8)
    a_zp = np.uint8(121)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    scale = rng.uniform(1e-4, 3e-4, N).astype(np.float32) if per_col else np.float32(2.1e-4)
    zp = {"col": rng.integers(-50000, 50000, N).astype(np.int32), "scalar": np.int32(-777),
          "zero": np.zeros(N, np.int32), None: None}[zp_kind]
    if zp is not None and not per_col:
        zp = np.int32(zp)
    bias = (0.05 * rng.standard_normal(N)).astype(np.float32)

    def build(ex):
        ex.add_input("a", [None] * (len(shape) - 1) + [K])
        ex.add_initializer("a_zp", np.asarray(a_zp))
        return graphs.add_dequantize_linear_head(ex, "a", "a_zp", w, scale, zp, bias, axis=axis)

    fused_ex, plain_ex = GpuGraphExecutor(), GpuGraphExecutor()
    y = build(fused_ex)
    build(plain_ex)
    got = fused_ex.run({"a": dev(a)}, [y])[y]
    heads = [e for e in fused_ex.plan()[0] if e.kind == "FusedHead"]
    assert len(heads) == 1 and heads[0].pattern == "QuantizedLinear" and heads[0].out == y
    plain = plain_ex.run({"a": dev(a)}, [y, "dq.acc"])  # accumulator requested: not fused
    assert all(e.kind != "FusedHead" or e.op_type != "MatMulInteger" for e in plain_ex.plan()[0])

    a2 = a.reshape(-1, K)
    acc = oracle.matmul_integer(a2, w, np.asarray(a_zp))
    assert np.array_equal(plain["dq.acc"].reshape(-1, N), acc)
    deq = oracle.dequantize_linear(acc, np.asarray(scale), None if zp is None else np.asarray(zp), axis=1)
    want = oracle.add(deq, bias).reshape(shape[:-1] + (N,))
    assert np.array_equal(bits(got), bits(want)), int(np.count_nonzero(bits(got) != bits(want)))
    assert np.array_equal(bits(plain[y]), bits(want))
