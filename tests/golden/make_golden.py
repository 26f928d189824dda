"""Write the ONNX node-test golden vectors the reference vendors as small JSON fixtures.

Run in the build container only (it reads the reference checkout, which does not exist on
the GPU box); its output ``onnx_node_goldens.json`` is committed and is what the tests read.

Source data: ``tests/conformance_data/onnx-1.18/node/<test>/{model.onnx,test_data_set_0/*.pb}``
in the reference. The reference's own conformance harness only parses these
(``tests/onnx_conformance.rs:199-228`` returns ``ParserOnlyOk``), so the expected outputs
were never compared there; here they pin the CPU oracle.

Only data is read: each ``.pb`` is an ONNX ``TensorProto`` and ``model.onnx`` a
``ModelProto``; both are decoded with the minimal protobuf wire reader below (field numbers
from the public ``onnx.proto``), nothing is executed.
"""
import json
import os
import struct
import sys

REF = os.environ.get("ICONNX_REFERENCE", "/root/reference")
NODE_DIR = os.path.join(REF, "tests/conformance_data/onnx-1.18/node")
TESTS = [
    "test_dynamicquantizelinear",
    "test_dynamicquantizelinear_max_adjusted",
    "test_dynamicquantizelinear_min_adjusted",
    "test_matmulinteger",
    "test_dequantizelinear",
    "test_dequantizelinear_axis",
    "test_mul",
    "test_mul_bcast",
    "test_add",
    "test_add_bcast",
    "test_div",
    "test_div_bcast",
    # encoder ops (fp32): LayerNormalization over the last axis, Softmax, Erf, MatMul,
    # Transpose
    "test_layer_normalization_2d_axis1",
    "test_layer_normalization_2d_axis_negative_1",
    "test_layer_normalization_3d_axis2_epsilon",
    "test_layer_normalization_3d_axis_negative_1_epsilon",
    "test_layer_normalization_4d_axis3",
    "test_layer_normalization_4d_axis_negative_1",
    "test_softmax_example",
    "test_softmax_axis_2",
    "test_softmax_default_axis",
    "test_softmax_negative_axis",
    "test_softmax_large_number",
    "test_erf",
    "test_matmul_2d",
    "test_matmul_3d",
    "test_matmul_4d",
    "test_transpose_default",
    "test_transpose_all_permutations_0",
    "test_transpose_all_permutations_1",
    "test_transpose_all_permutations_2",
    "test_transpose_all_permutations_3",
    "test_transpose_all_permutations_4",
    "test_transpose_all_permutations_5",
    # Gather (the UINT8 embedding table of DistilBERT-INT8 goes through it)
    "test_gather_0", "test_gather_1", "test_gather_2d_indices", "test_gather_negative_indices",
    # the LayerNorm of an export below opset 17, node by node: ReduceMean, Pow, Sqrt
    "test_reduce_mean_default_axes_keepdims_example", "test_reduce_mean_default_axes_keepdims_random",
    "test_reduce_mean_do_not_keepdims_example", "test_reduce_mean_do_not_keepdims_random",
    "test_reduce_mean_keepdims_example", "test_reduce_mean_keepdims_random",
    "test_reduce_mean_negative_axes_keepdims_example", "test_reduce_mean_negative_axes_keepdims_random",
    "test_pow", "test_pow_bcast_array", "test_pow_bcast_scalar", "test_pow_example",
    "test_sqrt", "test_sqrt_example",
]

# TensorProto.DataType values used by these tests.
DT = {1: "f32", 2: "u8", 3: "i8", 6: "i32", 7: "i64"}


def _varint(buf, i):
    shift = 0
    val = 0
    while True:
        b = buf[i]
        i += 1
        val |= (b & 0x7F) << shift
        if not b & 0x80:
            return val, i
        shift += 7


def fields(buf):
    """Yield (field_number, wire_type, value) for one protobuf message."""
    i = 0
    while i < len(buf):
        key, i = _varint(buf, i)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            v = buf[i:i + 8]
            i += 8
        elif wt == 2:
            ln, i = _varint(buf, i)
            v = buf[i:i + ln]
            i += ln
        elif wt == 5:
            v = buf[i:i + 4]
            i += 4
        else:
            raise ValueError("unsupported wire type %d" % wt)
        yield fno, wt, v


def _packed_varints(v):
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(x)
    return out


def _signed(x, bits):
    return x - (1 << bits) if x >= (1 << (bits - 1)) else x


def decode_tensor(buf):
    dims, dtype, raw, f32, i32, i64, name = [], None, None, [], [], [], ""
    for fno, wt, v in fields(buf):
        if fno == 1:
            dims += _packed_varints(v) if wt == 2 else [v]
        elif fno == 2:
            dtype = v
        elif fno == 4:
            f32 += list(struct.unpack("<%df" % (len(v) // 4), v)) if wt == 2 else [struct.unpack("<f", v)[0]]
        elif fno == 5:
            i32 += _packed_varints(v) if wt == 2 else [v]
        elif fno == 7:
            i64 += _packed_varints(v) if wt == 2 else [v]
        elif fno == 8:
            name = v.decode()
        elif fno == 9:
            raw = bytes(v)
    n = 1
    for d in dims:
        n *= d
    kind = DT[dtype]
    if raw is not None:
        fmt = {"f32": "f", "u8": "B", "i8": "b", "i32": "i", "i64": "q"}[kind]
        vals = list(struct.unpack("<%d%s" % (n, fmt), raw))
    elif kind == "f32":
        vals = f32
    elif kind in ("u8", "i8", "i32"):
        # int32_data carries u8/i8/i32 as (sign-extended) varints
        vals = [_signed(x & 0xFFFFFFFFFFFFFFFF, 64) for x in i32]
        if kind == "u8":
            vals = [x & 0xFF for x in vals]
    else:
        vals = [_signed(x, 64) for x in i64]
    t = {"name": name, "dtype": kind, "dims": dims}
    if kind == "f32":
        t["bits"] = [struct.unpack("<I", struct.pack("<f", x))[0] for x in vals]
        t["values"] = [float(x) for x in vals]
    else:
        t["values"] = [int(x) for x in vals]
    return t


def decode_node(model_buf):
    """Return (op_type, inputs, outputs, attrs) of the single node in a node-test model."""
    for fno, _, v in fields(model_buf):
        if fno != 7:  # ModelProto.graph
            continue
        for gf, _, gv in fields(v):
            if gf != 1:  # GraphProto.node
                continue
            ins, outs, op, attrs = [], [], "", {}
            for nf, _, nv in fields(gv):
                if nf == 1:
                    ins.append(nv.decode())
                elif nf == 2:
                    outs.append(nv.decode())
                elif nf == 4:
                    op = nv.decode()
                elif nf == 5:
                    aname, aval, ints = "", None, []
                    for af, awt, av in fields(nv):
                        if af == 1:
                            aname = av.decode()
                        elif af == 2:  # AttributeProto.f
                            aval = struct.unpack("<f", av)[0]
                        elif af == 3:  # AttributeProto.i
                            aval = _signed(av, 64)
                        elif af == 8:  # AttributeProto.ints
                            ints += [_signed(x, 64) for x in (_packed_varints(av) if awt == 2 else [av])]
                    attrs[aname] = ints if ints else aval
            return op, ins, outs, attrs
    raise ValueError("no node")


def main(out_path):
    cases = {}
    for t in TESTS:
        d = os.path.join(NODE_DIR, t)
        with open(os.path.join(d, "model.onnx"), "rb") as f:
            op, ins, outs, attrs = decode_node(f.read())
        ds = os.path.join(d, "test_data_set_0")
        inputs = []
        for i in range(len(ins)):
            with open(os.path.join(ds, "input_%d.pb" % i), "rb") as f:
                inputs.append(decode_tensor(f.read()))
        outputs = []
        for i in range(len(outs)):
            with open(os.path.join(ds, "output_%d.pb" % i), "rb") as f:
                outputs.append(decode_tensor(f.read()))
        cases[t] = {
            "source": "tests/conformance_data/onnx-1.18/node/%s" % t,
            "op_type": op,
            "attributes": attrs,
            "inputs": inputs,
            "outputs": outputs,
        }
    with open(out_path, "w") as f:
        json.dump(cases, f, indent=1, sort_keys=True)
    print("wrote %d cases to %s" % (len(cases), out_path))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(__file__), "onnx_node_goldens.json"))
