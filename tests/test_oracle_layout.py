"""CPU: the oracle of the shape / mask plumbing (oracle/layout.py) pinned before it checks the
GPU path:

* against every ONNX 1.18 node golden the reference vendors for Shape, Unsqueeze, Squeeze,
  Concat, Slice, Expand, Equal and Where (tests/golden/onnx_node/, copied by
  tests/golden/copy_onnx_models.py from tests/conformance_data/onnx-1.18/node/): exact,
  dtype included;
* against numpy's own slicing, broadcasting and comparison on random cases — an independent
  implementation of the same definitions (Python's slice semantics equal the reference's GPU
  normalisation whenever the clamped end is not -1, which is where a Python slice needs None);
* Cast at the edges of Rust's ``as`` rules (NaN, saturation, truncation toward zero, wrap).
"""
import glob
import os

import numpy as np
import pytest

from iconnx_amd.onnx import OnnxParser, decode_tensor
from oracle import OracleError
from oracle import layout as L

HERE = os.path.dirname(os.path.abspath(__file__))
OPS = ("Shape", "Unsqueeze", "Squeeze", "Concat", "Slice", "Expand", "Equal", "Where")


def cases():
    out = []
    for d in sorted(glob.glob(os.path.join(HERE, "golden", "onnx_node", "*"))):
        m = OnnxParser.parse_file(os.path.join(d, "model.onnx"))
        if m.computation_graph().nodes()[0].op_type in OPS:
            out.append(d)
    return out


def load(d):
    m = OnnxParser.parse_file(os.path.join(d, "model.onnx"))
    node = m.computation_graph().nodes()[0]
    ins = []
    for i, _ in enumerate(m.inputs()):
        with open(os.path.join(d, "test_data_set_0", "input_%d.pb" % i), "rb") as f:
            ins.append(decode_tensor(f.read())[1])
    with open(os.path.join(d, "test_data_set_0", "output_0.pb"), "rb") as f:
        want = decode_tensor(f.read())[1]
    return node, ins, want


def oracle_of(node, ins):
    """The oracle for one node of these ops on its inputs (also used by the GPU tests)."""
    op, a = node.op_type, node.attributes
    if op == "Shape":
        return L.shape(ins[0].shape, a.get("start", 0), a.get("end"))
    if op == "Unsqueeze":
        return L.unsqueeze(ins[0], list(ins[1]) if len(ins) > 1 else a["axes"])
    if op == "Squeeze":
        axes = list(ins[1]) if len(ins) > 1 else a.get("axes")
        return L.squeeze(ins[0], axes)
    if op == "Concat":
        return L.concat(ins, a.get("axis", 0))
    if op == "Slice":
        return L.slice_(ins[0], ins[1], ins[2], ins[3] if len(ins) > 3 else None, ins[4] if len(ins) > 4 else None)
    if op == "Expand":
        return L.expand(ins[0], ins[1])
    if op == "Equal":
        return L.equal(ins[0], ins[1])
    if op == "Where":
        return L.where(*ins)
    raise KeyError(op)


CASES = cases()


def test_every_layout_golden_is_here():
    names = {os.path.basename(d) for d in CASES}
    assert len(names) == 45, sorted(names)


@pytest.mark.parametrize("d", CASES, ids=[os.path.basename(d) for d in CASES])
def test_oracle_matches_onnx_golden(d):
    node, ins, want = load(d)
    got = oracle_of(node, ins)
    assert got.dtype == want.dtype and got.shape == want.shape, (got.dtype, got.shape, want.dtype, want.shape)
    assert np.array_equal(got, want)


def test_slice_against_python_slicing():
    rng = np.random.default_rng(3)
    for _ in range(400):
        shape = tuple(int(v) for v in rng.integers(1, 7, rng.integers(1, 4)))
        x = rng.standard_normal(shape).astype(np.float32)
        nd = len(shape)
        axes = [int(a) for a in rng.permutation(nd)[: rng.integers(1, nd + 1)]]
        starts = [int(v) for v in rng.integers(-9, 9, len(axes))]
        ends = [int(v) for v in rng.integers(-9, 9, len(axes))]
        steps = [int(v) for v in rng.choice([-3, -2, -1, 1, 2, 3], len(axes))]
        neg_axes = [a - nd if rng.random() < 0.5 else a for a in axes]
        first, step, length = L.slice_params(shape, starts, ends, neg_axes, steps)
        sl = [slice(None)] * nd
        for a, s, e, st in zip(axes, starts, ends, steps):
            sl[a] = slice(s, e, st)
        # Python clamps the same way except that a negative step's end of -1 after clamping
        # means "past index 0" there, which Python writes as None
        clamped_end_minus1 = any(
            st < 0 and (e < 0 and shape[a] + e <= -1 or False) for a, e, st in zip(axes, ends, steps))
        got = L.slice_(x, starts, ends, neg_axes, steps)
        if not clamped_end_minus1:
            want = x[tuple(sl)]
            assert got.shape == want.shape and np.array_equal(got, want), (shape, axes, starts, ends, steps)
        assert list(got.shape) == length


def test_slice_reference_normalisation_edge():
    """The reference's GPU Slice turns a negative end below -dim into 0 before a negative
    step clamps it to -1, so index 0 is left out (an ONNX reading would keep it): the oracle
    follows the reference."""
    x = np.arange(5, dtype=np.float32)
    assert L.slice_(x, [4], [-100], [0], [-1]).tolist() == [4.0, 3.0, 2.0, 1.0]
    assert L.slice_(x, [4], [-6], [0], [-1]).tolist() == [4.0, 3.0, 2.0, 1.0]
    assert L.slice_(x, [10], [0], [0], [-2]).tolist() == [4.0, 2.0]
    with pytest.raises(OracleError):
        L.slice_(x, [0], [3], [0], [0])


def test_broadcasting_ops_against_numpy():
    rng = np.random.default_rng(4)
    for _ in range(200):
        out = tuple(int(v) for v in rng.integers(1, 5, rng.integers(1, 5)))
        def sub():
            r = int(rng.integers(0, len(out) + 1))
            s = list(out[len(out) - r:])
            return tuple(1 if rng.random() < 0.4 else v for v in s)
        a = rng.integers(-2, 3, sub()).astype(np.int64)
        b = rng.integers(-2, 3, sub()).astype(np.int64)
        c = rng.integers(0, 2, sub()).astype(np.bool_)
        assert np.array_equal(L.equal(a, b), np.equal(a, b))
        x = rng.standard_normal(sub()).astype(np.float32)
        y = rng.standard_normal(sub()).astype(np.float32)
        assert np.array_equal(L.where(c, x, y), np.where(c, x, y))
        e = L.expand(a, out)
        assert np.array_equal(e, np.broadcast_to(a, np.broadcast_shapes(a.shape, out)))


def test_concat_unsqueeze_squeeze_shape_against_numpy():
    rng = np.random.default_rng(5)
    for _ in range(100):
        shape = tuple(int(v) for v in rng.integers(1, 4, rng.integers(1, 4)))
        ax = int(rng.integers(-len(shape), len(shape)))
        parts = []
        for _ in range(int(rng.integers(1, 4))):
            s = list(shape)
            s[ax] = int(rng.integers(0, 3))
            parts.append(rng.integers(0, 9, s).astype(np.int32))
        assert np.array_equal(L.concat(parts, ax), np.concatenate(parts, ax))
        x = parts[0]
        u = L.unsqueeze(x, [0, -1])
        assert u.shape == np.expand_dims(x, (0, -1)).shape
        assert L.squeeze(u).shape == np.squeeze(u).shape
        assert L.squeeze(u, [0]).shape == np.squeeze(u, 0).shape
        assert L.shape(x.shape).tolist() == list(x.shape)
        assert L.shape(x.shape, -1).tolist() == list(x.shape)[-1:]


def test_cast_follows_rust_as():
    f = np.array([np.nan, 1e30, -1e30, 2.9, -2.9, 2147483520.0, 3e9, -0.0], np.float32)
    assert L.cast(f, 7).tolist() == [0, 2**63 - 1, -2**63, 2, -2, 2147483520, 3000000000, 0]
    assert L.cast(f, 6).tolist() == [0, 2**31 - 1, -2**31, 2, -2, 2147483520, 2**31 - 1, 0]
    assert L.cast(f, 9).tolist() == [True, True, True, True, True, True, True, False]
    i = np.array([2**40 + 7, -1, 2**31, 16777217, 16777219], np.int64)
    assert L.cast(i, 6).tolist() == [7, -1, -2**31, 16777217, 16777219]
    # to Float32: nearest, ties to even (2^24 + 1 -> 2^24, 2^24 + 3 -> 2^24 + 4)
    assert L.cast(i, 1).tolist() == [float(2**40), -1.0, 2147483648.0, 16777216.0, 16777220.0]
    assert L.cast(np.array([True, False]), 1).tolist() == [1.0, 0.0]
