"""ONNX model files for the quantized-linear path.

``OnnxParser.parse_file(path)`` returns an ``OnnxModel`` with the reference's accessors
(src/onnx_parser.rs:133-167 for the parser, :174-316 and :358-560 for the model: inputs,
input_shapes, outputs, list_weight_names, opset_imports, extract_weights,
computation_graph, list_unique_operators), so ``GpuGraphExecutor.from_model`` reads a file
exactly as the reference's does (src/cuda/inference/mod.rs:250-271).  ``ModelWriter``
records the same add_input / add_initializer / add_node / add_output calls the executor
takes and serialises them, which is how the synthetic configs become .onnx files.

The protobuf wire format is decoded and encoded here directly (varints, fixed32/64 and
length-delimited fields) for the subset of onnx.proto the path uses: ModelProto
(ir_version 1, opset_import 8, graph 7), OperatorSetIdProto (domain 1, version 2),
GraphProto (node 1, name 2, initializer 5, input 11, output 12, value_info 13), NodeProto
(input 1, output 2, name 3, op_type 4, attribute 5, domain 7), AttributeProto (name 1, f 2,
i 3, s 4, t 5, floats 7, ints 8, type 20), TensorProto (dims 1, data_type 2, float_data 4,
int32_data 5, int64_data 7, name 8, raw_data 9, double_data 10), ValueInfoProto (name 1,
type 2), TypeProto (tensor_type 1), TypeProto.Tensor (elem_type 1, shape 2),
TensorShapeProto (dim 1), Dimension (dim_value 1, dim_param 2).  Unknown fields are
skipped, as protobuf decoders do.
"""
import struct

import numpy as np

# TensorProto.DataType -> numpy dtype (the initializer dtypes the reference decodes,
# src/onnx_parser.rs:395-470)
_DTYPE = {1: np.float32, 2: np.uint8, 3: np.int8, 6: np.int32, 7: np.int64, 9: np.bool_,
          10: np.float16, 11: np.float64}
_CODE = {np.dtype(v): k for k, v in _DTYPE.items()}


class ParseError(ValueError):
    """A malformed or unsupported model (the reference's ParseError)."""


# ---- wire format ----------------------------------------------------------------------
def _varint(buf, i):
    shift = result = 0
    while True:
        if i >= len(buf):
            raise ParseError("truncated varint")
        b = buf[i]
        i += 1
        result |= (b & 0x7F) << shift
        if b < 0x80:
            return result, i
        shift += 7
        if shift > 70:
            raise ParseError("varint too long")


def _fields(buf):
    """(field number, wire type, value) of one message: ints for varint / fixed32 /
    fixed64 (raw bits), bytes for length-delimited fields."""
    i, n = 0, len(buf)
    while i < n:
        key, i = _varint(buf, i)
        field, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            if i + 8 > n:
                raise ParseError("truncated fixed64")
            v = struct.unpack_from("<Q", buf, i)[0]
            i += 8
        elif wt == 2:
            ln, i = _varint(buf, i)
            if i + ln > n:
                raise ParseError("truncated length-delimited field %d" % field)
            v = bytes(buf[i:i + ln])
            i += ln
        elif wt == 5:
            if i + 4 > n:
                raise ParseError("truncated fixed32")
            v = struct.unpack_from("<I", buf, i)[0]
            i += 4
        else:
            raise ParseError("unsupported wire type %d (field %d)" % (wt, field))
        yield field, wt, v


def _int64(v):
    return v - (1 << 64) if v >= 1 << 63 else v


def _varints(wt, v):
    """A repeated integer field: packed (length-delimited) or one value."""
    if wt != 2:
        return [_int64(v)]
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(_int64(x))
    return out


def _floats(wt, v):
    if wt == 2:
        return list(struct.unpack("<%df" % (len(v) // 4), v))
    return [struct.unpack("<f", struct.pack("<I", v))[0]]


def _doubles(wt, v):
    if wt == 2:
        return list(struct.unpack("<%dd" % (len(v) // 8), v))
    return [struct.unpack("<d", struct.pack("<Q", v))[0]]


def _enc_varint(v):
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field, wt):
    return _enc_varint((field << 3) | wt)


def _len_field(field, payload):
    return _key(field, 2) + _enc_varint(len(payload)) + payload


def _int_field(field, v):
    return _key(field, 0) + _enc_varint(v)


def _str_field(field, s):
    return _len_field(field, s.encode())


# ---- tensors --------------------------------------------------------------------------
def decode_tensor(buf):
    """TensorProto -> (name, numpy array), with the reference's payload rules
    (src/onnx_parser.rs:470-700): FLOAT from float_data else little-endian raw_data; INT64
    from int64_data else raw_data; INT32 / INT8 / UINT8 from int32_data (the low bits) else
    raw_data; DOUBLE from double_data else raw_data; the element count must match dims."""
    dims, dtype, name = [], 1, ""
    f32, i32, i64, f64, raw = [], [], [], [], None
    for field, wt, v in _fields(buf):
        if field == 1:
            dims += _varints(wt, v)
        elif field == 2:
            dtype = v
        elif field == 4:
            f32 += _floats(wt, v)
        elif field == 5:
            i32 += _varints(wt, v)
        elif field == 7:
            i64 += _varints(wt, v)
        elif field == 8:
            name = v.decode()
        elif field == 9:
            raw = v
        elif field == 10:
            f64 += _doubles(wt, v)
    if dtype not in _DTYPE:
        raise ParseError("initializer '%s': unsupported data type %d" % (name, dtype))
    np_dt = np.dtype(_DTYPE[dtype])
    count = int(np.prod(dims)) if dims else 1
    if count == 0:
        return name, np.zeros(dims, np_dt)
    if dtype == 1 and f32:
        data = np.array(f32, np.float32)
    elif dtype == 7 and i64:
        data = np.array(i64, np.int64)
    elif dtype in (2, 3, 6, 9) and i32:
        data = np.array(i32, np.int64).astype(np.uint32)  # two's complement, low 32 bits
        data = {2: data.astype(np.uint8), 3: data.astype(np.uint8).view(np.int8),
                6: data.view(np.int32), 9: data.astype(bool)}[dtype]
    elif dtype == 10 and i32:
        data = np.array(i32, np.int64).astype(np.uint16).view(np.float16)
    elif dtype == 11 and f64:
        data = np.array(f64, np.float64)
    elif raw:
        if len(raw) % np_dt.itemsize:
            raise ParseError("initializer '%s': raw_data length %d is not a multiple of %d"
                             % (name, len(raw), np_dt.itemsize))
        data = np.frombuffer(raw, np_dt.newbyteorder("<")).astype(np_dt)
    else:
        raise ParseError("initializer '%s': no data" % name)
    if data.size != count:
        raise ParseError("initializer '%s': %d elements, dims %s say %d"
                         % (name, data.size, dims, count))
    return name, data.reshape(dims)


def encode_tensor(name, arr):
    """numpy array -> TensorProto bytes (raw_data, little-endian)."""
    arr = np.asarray(arr)
    code = _CODE.get(arr.dtype)
    if code is None:
        raise ParseError("tensor '%s': dtype %s has no ONNX encoding here" % (name, arr.dtype))
    out = bytearray()
    for d in arr.shape:
        out += _int_field(1, d)
    out += _int_field(2, code)
    out += _str_field(8, name)
    out += _len_field(9, np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes())
    return bytes(out)


def _decode_attribute(buf):
    name, value, kind = "", None, None
    ints, floats = [], []
    for field, wt, v in _fields(buf):
        if field == 1:
            name = v.decode()
        elif field == 2:
            value = _floats(wt, v)[0]
        elif field == 3:
            value = _int64(v)
        elif field == 4:
            value = v.decode(errors="replace")
        elif field == 5:
            value = decode_tensor(v)[1]
        elif field == 7:
            floats += _floats(wt, v)
        elif field == 8:
            ints += _varints(wt, v)
        elif field == 20:
            kind = v
    if ints:
        value = ints
    elif floats:
        value = floats
    elif value is None and kind in (7, 6):  # an empty list
        value = []
    return name, value


def _encode_attribute(name, value):
    out = bytearray(_str_field(1, name))
    if isinstance(value, (bool, int, np.integer)):
        out += _int_field(3, int(value)) + _int_field(20, 2)
    elif isinstance(value, (float, np.floating)):
        out += _key(2, 5) + struct.pack("<f", float(value)) + _int_field(20, 1)
    elif isinstance(value, str):
        out += _len_field(4, value.encode()) + _int_field(20, 3)
    elif isinstance(value, np.ndarray):
        out += _len_field(5, encode_tensor("", value)) + _int_field(20, 4)
    elif all(isinstance(x, (int, np.integer)) for x in value):
        out += _len_field(8, b"".join(_enc_varint(int(x)) for x in value)) + _int_field(20, 7)
    else:
        out += _len_field(7, struct.pack("<%df" % len(value), *value)) + _int_field(20, 6)
    return bytes(out)


def _decode_value_info(buf):
    name, elem, shape = "", None, None
    for field, _, v in _fields(buf):
        if field == 1:
            name = v.decode()
        elif field == 2:
            for tf, _, tv in _fields(v):
                if tf != 1:  # tensor_type
                    continue
                for sf, _, sv in _fields(tv):
                    if sf == 1:
                        elem = sv
                    elif sf == 2:
                        shape = []
                        for df, _, dv in _fields(sv):
                            if df != 1:
                                continue
                            dim = None
                            for ddf, _, ddv in _fields(dv):
                                if ddf == 1 and _int64(ddv) >= 0:
                                    dim = _int64(ddv)
                            shape.append(dim)
    return name, elem, shape


def _encode_value_info(name, elem, shape):
    dims = b""
    for d in shape or []:
        dims += _len_field(1, _int_field(1, d) if d is not None else _str_field(2, "dyn"))
    tensor = _int_field(1, elem) + (_len_field(2, dims) if shape is not None else b"")
    return _str_field(1, name) + _len_field(2, _len_field(1, tensor))


# ---- the model ------------------------------------------------------------------------
class GraphNode:
    """One node of the computation graph (src/onnx_parser.rs:1304)."""

    def __init__(self, op_type, inputs, outputs, attributes, name="", domain=""):
        self.op_type, self.inputs, self.outputs = op_type, list(inputs), list(outputs)
        self.attributes, self.name, self.domain = dict(attributes), name, domain

    def __repr__(self):
        return "GraphNode(%s, %s -> %s)" % (self.op_type, self.inputs, self.outputs)


class ComputationGraph:
    def __init__(self, nodes):
        self._nodes = list(nodes)

    def nodes(self):
        return list(self._nodes)

    def node_count(self):
        return len(self._nodes)

    def __iter__(self):
        return iter(self._nodes)


class OnnxModel:
    """A decoded ModelProto with the reference OnnxModel's accessors."""

    def __init__(self, buf):
        self.ir_version, self._opsets, graph = 0, [], None
        for field, _, v in _fields(buf):
            if field == 1:
                self.ir_version = v
            elif field == 7:
                graph = v
            elif field == 8:
                dom, ver = "", 0
                for of, _, ov in _fields(v):
                    if of == 1:
                        dom = ov.decode()
                    elif of == 2:
                        ver = _int64(ov)
                self._opsets.append((dom, ver))
        if graph is None:
            raise ParseError("ONNX model has no graph")
        self.graph_name = ""
        self._nodes, self._inits, self._inputs, self._outputs = [], [], [], []
        for field, _, v in _fields(graph):
            if field == 1:
                self._nodes.append(v)
            elif field == 2:
                self.graph_name = v.decode()
            elif field == 5:
                self._inits.append(v)
            elif field == 11:
                self._inputs.append(_decode_value_info(v))
            elif field == 12:
                self._outputs.append(_decode_value_info(v))

    def inputs(self):
        return [n for n, _, _ in self._inputs]

    def input_shapes(self):
        """[(name, [dim or None])]: a dim_param or an unset / negative dim_value is dynamic;
        an input without a shape gives [] (src/onnx_parser.rs:213-249)."""
        return [(n, list(s) if s is not None else []) for n, _, s in self._inputs]

    def input_dtypes(self):
        return [e for _, e, _ in self._inputs]

    def outputs(self):
        return [n for n, _, _ in self._outputs]

    def output_dtypes(self):
        return [e for _, e, _ in self._outputs]

    def list_weight_names(self):
        return [decode_tensor_name(t) for t in self._inits]

    def opset_imports(self):
        return list(self._opsets)

    def extract_weights(self):
        """{name: numpy array} of every initializer (src/onnx_parser.rs:358-470)."""
        return dict(decode_tensor(t) for t in self._inits)

    def computation_graph(self):
        nodes = []
        for buf in self._nodes:
            op, ins, outs, attrs, name, dom = "", [], [], {}, "", ""
            for field, _, v in _fields(buf):
                if field == 1:
                    ins.append(v.decode())
                elif field == 2:
                    outs.append(v.decode())
                elif field == 3:
                    name = v.decode()
                elif field == 4:
                    op = v.decode()
                elif field == 5:
                    k, val = _decode_attribute(v)
                    attrs[k] = val
                elif field == 7:
                    dom = v.decode()
            nodes.append(GraphNode(op, ins, outs, attrs, name, dom))
        return ComputationGraph(nodes)

    def list_unique_operators(self):
        return sorted({n.op_type for n in self.computation_graph()})


def decode_tensor_name(buf):
    for field, _, v in _fields(buf):
        if field == 8:
            return v.decode()
    return ""


class OnnxParser:
    """src/onnx_parser.rs:133-167."""

    @staticmethod
    def parse_file(path):
        with open(path, "rb") as f:
            return OnnxModel(f.read())

    @staticmethod
    def parse_bytes(buf):
        return OnnxModel(buf)


# ---- writing --------------------------------------------------------------------------
class ModelWriter:
    """Records the executor's construction calls (add_input, add_initializer, add_node,
    add_output) and serialises them as a ModelProto (opset 21, IR version 10)."""

    def __init__(self, name="iconnx_amd", opset=21):
        self.name, self.opset = name, opset
        self.inputs, self.inits, self.nodes, self.outputs = [], [], [], []
        self._elem = {}

    def add_input(self, name, shape, elem_type=1):
        self.inputs.append((name, elem_type, [None if d is None or d < 0 else int(d) for d in shape]))

    def add_initializer(self, name, tensor):
        arr = np.asarray(tensor)
        self.inits.append((name, arr))
        self._elem[name] = _CODE.get(arr.dtype, 1)

    def add_node(self, name, op_type, inputs, outputs, attributes=None):
        self.nodes.append((name, op_type, list(inputs), list(outputs), dict(attributes or {})))

    def add_output(self, name, elem_type=1):
        if name not in [o[0] for o in self.outputs]:
            self.outputs.append((name, elem_type, None))

    def to_bytes(self):
        g = bytearray()
        for name, op, ins, outs, attrs in self.nodes:
            nb = bytearray()
            for x in ins:
                nb += _str_field(1, x)
            for x in outs:
                nb += _str_field(2, x)
            nb += _str_field(3, name) + _str_field(4, op)
            for k, v in attrs.items():
                nb += _len_field(5, _encode_attribute(k, v))
            g += _len_field(1, bytes(nb))
        g += _str_field(2, self.name)
        for name, arr in self.inits:
            g += _len_field(5, encode_tensor(name, arr))
        for name, elem, shape in self.inputs:
            g += _len_field(11, _encode_value_info(name, elem, shape))
        for name, elem, shape in self.outputs:
            g += _len_field(12, _encode_value_info(name, elem, shape))
        opset = _str_field(1, "") + _int_field(2, self.opset)
        return _int_field(1, 10) + _str_field(2, "iconnx_amd") + _len_field(7, bytes(g)) + _len_field(8, opset)

    def save(self, path):
        with open(path, "wb") as f:
            f.write(self.to_bytes())
