"""ONNX file I/O (iconnx_amd.onnx): the reference's vendored ONNX 1.18 node-test models are
parsed, their input / output tensors decoded and cross-checked against the JSON goldens
that tests/golden/make_golden.py decoded independently; synthetic graphs round-trip through
ModelWriter -> bytes -> OnnxParser; the wire rules of the reference's tensor decoder
(src/onnx_parser.rs:470-700: int32_data for INT8 / UINT8 / INT32, float_data, int64_data,
raw_data, element-count check) are exercised one by one."""
import glob
import os
import struct

import numpy as np
import pytest

from iconnx_amd import graphs
from iconnx_amd.onnx import (ModelWriter, OnnxParser, ParseError, _int_field, _len_field,
                             _str_field, decode_tensor, encode_tensor)
from tests.golden_util import tensor

HERE = os.path.dirname(os.path.abspath(__file__))
MODELS = sorted(glob.glob(os.path.join(HERE, "golden", "onnx_node", "*")))


def load_pb(path):
    with open(path, "rb") as f:
        return decode_tensor(f.read())[1]


def test_vendored_models_parse():
    assert len(MODELS) >= 20
    for d in MODELS:
        m = OnnxParser.parse_file(os.path.join(d, "model.onnx"))
        g = m.computation_graph()
        assert g.node_count() == 1, d
        assert m.opset_imports() and m.opset_imports()[0][0] in ("", "ai.onnx")
        ins = sorted(glob.glob(os.path.join(d, "test_data_set_0", "input_*.pb")))
        assert len(ins) == len(m.inputs()), d
        assert m.list_unique_operators() == [g.nodes()[0].op_type]


def test_vendored_tensors_match_independent_decoder(goldens):
    checked = 0
    for d in MODELS:
        name = os.path.basename(d)
        if name not in goldens:
            continue
        g = goldens[name]
        m = OnnxParser.parse_file(os.path.join(d, "model.onnx"))
        node = m.computation_graph().nodes()[0]
        assert node.op_type == g["op_type"]
        for i, want in enumerate(g["inputs"]):
            got = load_pb(os.path.join(d, "test_data_set_0", "input_%d.pb" % i))
            w = tensor(want)
            assert got.dtype == w.dtype and np.array_equal(got.reshape(-1).view(np.uint8),
                                                           w.reshape(-1).view(np.uint8)), (name, i)
        for i, want in enumerate(g["outputs"]):
            got = load_pb(os.path.join(d, "test_data_set_0", "output_%d.pb" % i))
            w = tensor(want)
            assert np.array_equal(got.reshape(-1).view(np.uint8), w.reshape(-1).view(np.uint8)), (name, i)
        checked += 1
    assert checked >= 18


def test_attributes_decode():
    by = {os.path.basename(d): OnnxParser.parse_file(os.path.join(d, "model.onnx")) for d in MODELS}
    ln = by["test_layer_normalization_3d_axis_negative_1_epsilon"].computation_graph().nodes()[0]
    assert ln.attributes["axis"] == -1
    assert np.float32(ln.attributes["epsilon"]) == np.float32(0.1)
    sm = by["test_softmax_axis_2"].computation_graph().nodes()[0]
    assert sm.attributes == {"axis": 2}
    tp = by["test_transpose_all_permutations_0"].computation_graph().nodes()[0]
    assert tp.attributes["perm"] == [0, 1, 2]
    assert by["test_dequantizelinear_axis"].input_shapes() == [("x", [1, 3, 3, 2]), ("x_scale", [3]),
                                                               ("x_zero_point", [3])]


def _graph_signature(model):
    nodes = [(n.op_type, n.inputs, n.outputs,
              {k: (np.asarray(v).tolist() if not isinstance(v, float) else np.float32(v))
               for k, v in n.attributes.items()}) for n in model.computation_graph()]
    return nodes, model.input_shapes()


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg4"])
def test_config_graphs_round_trip(cfg, tmp_path):
    path = str(tmp_path / ("%s.onnx" % cfg))
    out, d = graphs.write_model(path, graphs.config_graph, cfg)
    m = OnnxParser.parse_file(path)
    assert m.outputs() == [out]
    assert m.input_shapes() == [("x", [None, None, d["x"].shape[-1]])]
    w = m.extract_weights()
    assert np.array_equal(w["%s.W" % cfg], d["w"]) and w["%s.W" % cfg].dtype == d["w"].dtype
    assert np.array_equal(w["%s.bias" % cfg].view(np.uint32), np.asarray(d["bias"]).view(np.uint32))
    # the same graph recorded directly has the same nodes
    rec = ModelWriter()
    graphs.config_graph(rec, cfg)
    direct = OnnxParser.parse_bytes(rec.to_bytes())
    assert _graph_signature(m) == _graph_signature(direct)
    ops = [n.op_type for n in m.computation_graph()]
    assert ops[:4] == ["DynamicQuantizeLinear", "Mul", "MatMulInteger", "Cast"]


def test_encoder_graph_round_trip(tmp_path):
    path = str(tmp_path / "encoder.onnx")
    out, names, params = graphs.write_model(path, graphs.encoder_graph, layers=1)
    m = OnnxParser.parse_file(path)
    ops = m.list_unique_operators()
    for op in ("DynamicQuantizeLinear", "MatMulInteger", "LayerNormalization", "Softmax", "Erf",
               "Transpose", "Reshape", "MatMul"):
        assert op in ops
    w = m.extract_weights()
    assert np.array_equal(w["L0.ff1.W"], params[0]["ff1"]["w"])
    assert w["L0.attn.split"].dtype == np.int64 and w["L0.attn.split"].tolist() == [0, 0, 12, 64]
    perms = [n.attributes["perm"] for n in m.computation_graph() if n.op_type == "Transpose"]
    assert [0, 2, 3, 1] in perms


def _tensor_msg(dims, dtype, name="t", **payload):
    out = b"".join(_int_field(1, d) for d in dims) + _int_field(2, dtype) + _str_field(8, name)
    for field, blob in payload.items():
        num = {"float_data": 4, "int32_data": 5, "int64_data": 7, "raw_data": 9}[field]
        out += _len_field(num, blob)
    return out


def _packed_varints(vals):
    from iconnx_amd.onnx import _enc_varint

    return b"".join(_enc_varint(v) for v in vals)


def test_tensor_payload_rules():
    # INT8 in int32_data: low 8 bits, sign-extended (negative values are 10-byte varints)
    buf = _tensor_msg([4], 3, int32_data=_packed_varints([-128, -1, 0, 127]))
    assert decode_tensor(buf)[1].tolist() == [-128, -1, 0, 127]
    # UINT8 in int32_data: low 8 bits, zero-extended
    buf = _tensor_msg([3], 2, int32_data=_packed_varints([0, 200, 255]))
    assert decode_tensor(buf)[1].dtype == np.uint8 and decode_tensor(buf)[1].tolist() == [0, 200, 255]
    # INT32 in int32_data
    buf = _tensor_msg([2], 6, int32_data=_packed_varints([-2 ** 31, 2 ** 31 - 1]))
    assert decode_tensor(buf)[1].tolist() == [-2 ** 31, 2 ** 31 - 1]
    # FLOAT in float_data (packed fixed32)
    buf = _tensor_msg([2], 1, float_data=struct.pack("<2f", 1.5, -0.0))
    got = decode_tensor(buf)[1]
    assert got.tolist() == [1.5, -0.0] and np.signbit(got[1])
    # INT64 in int64_data
    buf = _tensor_msg([2], 7, int64_data=_packed_varints([-5, 2 ** 40]))
    assert decode_tensor(buf)[1].tolist() == [-5, 2 ** 40]
    # raw_data, every dtype, through the encoder
    for arr in (np.arange(-3, 3, dtype=np.int8), np.arange(6, dtype=np.uint8).reshape(2, 3),
                np.float32([[1e-38, np.inf, -2.5]]), np.int64([7, -9]), np.int32([[-1]]),
                np.array(3.25, np.float32)):
        name, got = decode_tensor(encode_tensor("x", arr))
        assert name == "x" and got.dtype == arr.dtype and got.shape == arr.shape
        assert np.array_equal(got.reshape(-1).view(np.uint8), arr.reshape(-1).view(np.uint8))
    # element count must match dims (src/onnx_parser.rs:773-796)
    with pytest.raises(ParseError):
        decode_tensor(_tensor_msg([3], 3, raw_data=b"\x01\x02"))
    with pytest.raises(ParseError):
        decode_tensor(_tensor_msg([1], 1, raw_data=b"\x01\x02\x03"))  # not a multiple of 4
    with pytest.raises(ParseError):
        decode_tensor(_tensor_msg([1], 8))  # STRING is not an initializer dtype here
    # zero-element tensors are empty, not an error
    assert decode_tensor(_tensor_msg([0, 4], 1))[1].shape == (0, 4)


def test_malformed_buffers_raise():
    good = encode_tensor("w", np.arange(10, dtype=np.int8))
    for cut in (1, 3, len(good) - 2):
        with pytest.raises(ParseError):
            decode_tensor(good[:cut])
    with pytest.raises(ParseError):
        OnnxParser.parse_bytes(_int_field(1, 10))  # a model without a graph
