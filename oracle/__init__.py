"""CPU oracle for the int8 dynamic-quantized linear path — TEST INFRASTRUCTURE ONLY.

numpy-facing wrappers over ``liboracle.so`` (``oracle.c``), a single-threaded C
restatement of the reference's CPU operators.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker; the product (``iconnx_amd``) never calls it.

Each wrapper mirrors the reference operator's ``forward`` (argument meaning and the
conditions under which it panics — raised here as :class:`OracleError`):

* :func:`dynamic_quantize_linear` — ``src/operators/dynamic_quantize_linear.rs:32-112``
* :func:`matmul_integer` — ``src/operators/matmul_integer.rs:52-267``
* :func:`cast_i32_f32` — ``src/operators/cast.rs:46-49``
* :func:`add`/:func:`sub`/:func:`mul`/:func:`div` — ``src/operators/{add,mul,div}.rs``
* :func:`dequantize_linear` — ``src/operators/dequantize_linear.rs:32-214``
* :func:`layer_norm` — ``src/operators/layer_normalization.rs:25-80`` (last axis)
* :func:`reduce_mean` — ``src/operators/reduce_mean.rs:19-105``
* :func:`pow` — ``src/operators/pow.rs:18-45`` (the C library's powf, as Rust's f32::powf)
* :func:`sqrt` — ``src/operators/sqrt.rs:18-30``
* :func:`layer_norm_decomposed` — the node-by-node LayerNorm of an export below opset 17
  (ReduceMean, Sub, Pow, ReduceMean, Add, Sqrt, Div, Mul, Add), composed from the above
* :func:`softmax` — ``src/operators/softmax.rs:25-40`` (last axis)
* :func:`erf` — ``src/operators/erf.rs:21-31``
* :func:`matmul_f32` — ``src/operators/matmul.rs:20-150`` (f64-accumulated; tolerance)
* :func:`transpose` — ``src/operators/transpose.rs:10-40``
* :func:`gather` — ``src/operators/gather.rs:21-205`` (numpy index arithmetic; the index clamp
  of the GPU kernels, ``src/cuda/ops/quantize_kernels.rs:203-224``)

Parity pins (tests/test_oracle.py): the ONNX 1.18 node goldens the reference vendors
(tests/golden/onnx_node_goldens.json), the reference's unit-test literals, brute-force
int64/float64 checks and closed forms (Gather: the four ONNX ``test_gather_*`` goldens plus a
brute-force loop with negative and out-of-range indices).  The per-column ``b_zero_point`` form of
:func:`matmul_integer` is an extension the reference rejects; it is pinned only by the
ONNX definition (closed form + brute force) — reference parity unpinned for it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

DT_I8, DT_U8, DT_I32 = 0, 1, 2
ADD, SUB, MUL, DIV = 0, 1, 2, 3


class OracleError(RuntimeError):
    """Raised where the reference CPU operator panics."""


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.check_call(["make", "-s", "-C", _HERE, "-B", "liboracle.so"])


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    S = ctypes.c_size_t
    lib.orc_dql_u8.argtypes = [P, S, P, P, P, P]
    lib.orc_dql_u8.restype = None
    lib.orc_matmul_integer_rows.argtypes = [P, ctypes.c_int, P, ctypes.c_int, S, S, S,
                                            ctypes.c_int32, P, S, S, S, P]
    lib.orc_matmul_integer_rows.restype = ctypes.c_int
    lib.orc_cast_i32_f32.argtypes = [P, S, P]
    lib.orc_cast_i32_f32.restype = None
    lib.orc_binary_f32.argtypes = [ctypes.c_int, P, P, ctypes.c_int, P, P, ctypes.c_int,
                                   P, P, P]
    lib.orc_binary_f32.restype = ctypes.c_int
    lib.orc_dequantize_linear.argtypes = [P, ctypes.c_int, P, P, S, S, S, P]
    lib.orc_dequantize_linear.restype = None
    lib.orc_sum_unrolled8.argtypes = [P, S]
    lib.orc_sum_unrolled8.restype = ctypes.c_float
    lib.orc_layer_norm.argtypes = [P, S, S, P, P, ctypes.c_float, P]
    lib.orc_layer_norm.restype = None
    lib.orc_softmax_last.argtypes = [P, S, S, P]
    lib.orc_softmax_last.restype = None
    lib.orc_erf.argtypes = [P, S, P]
    lib.orc_erf.restype = None
    lib.orc_matmul_f32.argtypes = [P, P, S, ctypes.c_int, S, S, S, P]
    lib.orc_matmul_f32.restype = None
    lib.orc_transpose.argtypes = [P, S, ctypes.c_int, P, P, P]
    lib.orc_transpose.restype = None
    lib.orc_reduce_mean.argtypes = [P, S, S, S, ctypes.c_int, P]
    lib.orc_reduce_mean.restype = None
    lib.orc_pow_f32.argtypes = [P, P, S, P]
    lib.orc_pow_f32.restype = None
    lib.orc_sqrt_f32.argtypes = [P, S, P]
    lib.orc_sqrt_f32.restype = None
    _lib = lib
    return lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _dt(a):
    if a.dtype == np.int8:
        return DT_I8
    if a.dtype == np.uint8:
        return DT_U8
    if a.dtype == np.int32:
        return DT_I32
    raise OracleError("unsupported dtype %s" % a.dtype)


def dynamic_quantize_linear(x, return_scale64=False):
    """(y u8 same shape, y_scale f32 scalar, y_zero_point u8 scalar)."""
    x = np.asarray(x)
    if x.dtype != np.float32:
        raise OracleError("DynamicQuantizeLinear: input must be Float32, got %s" % x.dtype)
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape, np.uint8)
    s = np.zeros((), np.float32)
    zp = np.zeros((), np.uint8)
    s64 = np.zeros((), np.float64)
    _load().orc_dql_u8(_ptr(x), x.size, _ptr(y), _ptr(s), _ptr(zp), _ptr(s64))
    if return_scale64:
        return y, s, zp, float(s64)
    return y, s, zp


def _extract_zp(zp, operand_dtype, label, n_cols=None):
    """extract_scalar_zp (matmul_integer.rs:189-223); n_cols enables the per-column form."""
    if zp is None:
        return np.zeros(1, np.int32)
    zp = np.asarray(zp)
    if zp.dtype != operand_dtype:
        raise OracleError("MatMulInteger: %s_zero_point dtype %s must match operand dtype %s"
                          % (label, zp.dtype, operand_dtype))
    if zp.ndim == 0 or (zp.ndim == 1 and zp.shape[0] == 1):
        return zp.reshape(1).astype(np.int32)
    if n_cols is not None and zp.ndim == 1 and zp.shape[0] == n_cols:
        return zp.astype(np.int32)
    raise OracleError("MatMulInteger: %s_zero_point must be scalar (got shape %s); "
                      "per-axis zp is not supported" % (label, list(zp.shape)))


def matmul_integer(a, b, a_zp=None, b_zp=None, per_column_b_zp=False, rows=None):
    """int32 [M,N].  ``per_column_b_zp`` admits a [N] b_zero_point (ONNX form; not in the
    reference).  ``rows=(r0, r1)`` computes only those output rows (others left 0)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    for t, lab in ((a, "a"), (b, "b")):
        if t.dtype not in (np.int8, np.uint8):
            raise OracleError("MatMulInteger: input %s must be Int8 or UInt8, got %s"
                              % (lab, t.dtype))
    if a.ndim != 2 or b.ndim != 2:
        raise OracleError("MatMulInteger: a and b must be 2-D (got ranks %d, %d)"
                          % (a.ndim, b.ndim))
    M, K = a.shape
    if b.shape[0] != K:
        raise OracleError("MatMulInteger: K mismatch — a is %s, b is %s"
                          % (list(a.shape), list(b.shape)))
    N = b.shape[1]
    azp = _extract_zp(a_zp, a.dtype, "a")
    bzp = _extract_zp(b_zp, b.dtype, "b", N if per_column_b_zp else None)
    out = np.zeros((M, N), np.int32)
    r0, r1 = (0, M) if rows is None else rows
    rc = _load().orc_matmul_integer_rows(_ptr(a), _dt(a), _ptr(b), _dt(b), M, K, N,
                                         int(azp[0]), _ptr(bzp), bzp.size, r0, r1, _ptr(out))
    if rc == 1:
        raise OracleError("MatMulInteger: i32 overflow")
    if rc != 0:
        raise OracleError("MatMulInteger: invalid arguments")
    return out


def cast_i32_f32(x):
    x = np.asarray(x)
    if x.dtype != np.int32:
        raise OracleError("Cast: only Int32 -> Float32 is on this path")
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape, np.float32)
    _load().orc_cast_i32_f32(_ptr(x), x.size, _ptr(y))
    return y


def _contig(x, dtype):
    """C-contiguous array of ``dtype`` keeping a 0-d input 0-d (np.ascontiguousarray would
    make it 1-d; the reference's scalar tensors stay rank 0 through Mul / Add / Div)."""
    x = np.asarray(x, dtype=dtype)
    return x if x.flags.c_contiguous else x.copy(order="C")


def _binary(op, a, b):
    a = _contig(a, np.float32)
    b = _contig(b, np.float32)
    r = max(a.ndim, b.ndim)
    out_shape = np.zeros(8, np.uintp)
    out_rank = ctypes.c_int(0)
    shp = np.broadcast_shapes(a.shape, b.shape) if _broadcastable(a.shape, b.shape) else None
    if shp is None:
        raise OracleError("Failed to broadcast %s with %s" % (list(a.shape), list(b.shape)))
    out = np.empty(shp, np.float32)
    ash = np.array(a.shape or [1], np.uintp)
    bsh = np.array(b.shape or [1], np.uintp)
    rc = _load().orc_binary_f32(op, _ptr(a), _ptr(ash), a.ndim, _ptr(b), _ptr(bsh), b.ndim,
                                _ptr(out), _ptr(out_shape), ctypes.byref(out_rank))
    if rc != 0 or out_rank.value != r:
        raise OracleError("broadcast failed")
    return out


def _broadcastable(s1, s2):
    for x, y in zip(reversed(s1), reversed(s2)):
        if x != y and x != 1 and y != 1:
            return False
    return True


def add(a, b):
    return _binary(ADD, a, b)


def sub(a, b):
    return _binary(SUB, a, b)


def mul(a, b):
    return _binary(MUL, a, b)


def div(a, b):
    return _binary(DIV, a, b)


def dequantize_linear(x, scale, zp=None, axis=1):
    """DequantizeLinear::forward; ``axis`` only consulted for a per-axis (1-D) scale."""
    x = np.ascontiguousarray(x)
    if x.dtype not in (np.int8, np.uint8, np.int32):
        raise OracleError("DequantizeLinear: input dtype %s unsupported" % x.dtype)
    scale = np.asarray(scale)
    if scale.dtype != np.float32:
        raise OracleError("DequantizeLinear: scale must be Float32, got %s" % scale.dtype)
    per_tensor = scale.ndim == 0 or (scale.ndim == 1 and scale.size == 1)
    if per_tensor:
        axis_size, inner = 1, max(x.size, 1)
    else:
        ax = axis + x.ndim if axis < 0 else axis
        if not 0 <= ax < x.ndim:
            raise OracleError("DequantizeLinear: axis %d out of range for ndim %d"
                              % (axis, x.ndim))
        if scale.size != x.shape[ax]:
            raise OracleError("DequantizeLinear: per-axis scale length %d doesn't match "
                              "input shape[%d] = %d" % (scale.size, ax, x.shape[ax]))
        axis_size = x.shape[ax]
        inner = int(np.prod(x.shape[ax + 1:])) if ax + 1 < x.ndim else 1
    zpp = None
    if zp is not None:
        zp = np.asarray(zp)
        if zp.dtype != x.dtype:
            raise OracleError("DequantizeLinear: zero_point dtype %s must match input dtype %s"
                              % (zp.dtype, x.dtype))
        if zp.shape != scale.shape:
            raise OracleError("DequantizeLinear: zero_point shape %s must match scale shape %s"
                              % (list(zp.shape), list(scale.shape)))
        zpp = np.ascontiguousarray(zp.reshape(-1))
    sc = np.ascontiguousarray(scale.reshape(-1), dtype=np.float32)
    y = np.empty(x.shape, np.float32)
    _load().orc_dequantize_linear(_ptr(x), _dt(x), _ptr(sc),
                                  _ptr(zpp) if zpp is not None else None,
                                  x.size, axis_size, inner, _ptr(y))
    return y


def qlinear_graph(x, w, w_zp, x_scale_times_w_scale_inputs, bias, chain=(), rows=None):
    """Run the quantized-linear subgraph op by op in graph order, as the reference
    GraphExecutor does (src/graph_executor.rs:205-216 for DQL's three outputs, :356-432):

        DynamicQuantizeLinear(x) -> (xq, xs, xzp)
        MatMulInteger(xq, w, xzp, w_zp) -> acc i32
        Cast(acc) -> f32;  Mul(xs, w_scale) -> s;  Mul(cast, s);  Add(., bias)
        then each (op, operand, operand_is_lhs) of ``chain`` in order.

    ``x`` is [..., K] (flattened to 2-D like the GPU executor's 3-D x 2-D arm,
    src/cuda/executor/layout.rs:1058-1090).  ``x_scale_times_w_scale_inputs`` is the
    w_scale tensor (scalar or [N]).  Returns a dict of every intermediate.
    """
    x2 = np.ascontiguousarray(x).reshape(-1, x.shape[-1])
    xq, xs, xzp = dynamic_quantize_linear(x2)
    per_col = np.asarray(w_zp).ndim == 1 and np.asarray(w_zp).size > 1
    acc = matmul_integer(xq, w, xzp, w_zp, per_column_b_zp=per_col, rows=rows)
    cast = cast_i32_f32(acc)
    s = mul(xs, x_scale_times_w_scale_inputs)
    y = mul(cast, s)
    y = add(y, bias)
    out = {"xq": xq, "x_scale": xs, "x_zp": xzp, "acc": acc, "cast": cast, "scale": s,
           "linear": y}
    for op, operand, operand_is_lhs in chain:
        fn = {"Mul": mul, "Add": add, "Div": div, "Sub": sub}[op]
        y = fn(operand, y) if operand_is_lhs else fn(y, operand)
    out["y"] = y
    return out


def gather(data, indices, axis=0):
    """ONNX Gather as the reference computes it: output shape data.shape[:axis] +
    indices.shape + data.shape[axis+1:] (src/operators/gather.rs:59-151), a negative index
    taken from the end (gather.rs:89-114).  An index still outside [0, axis_len) is clamped,
    as the GPU kernels that the HIP path replaces do (gather_u8_kernel,
    src/cuda/ops/quantize_kernels.rs:203-224; the CPU forward would panic there).  The data
    dtype is kept, as on the GPU path (the CPU forward converts non-f32/i64 data to Float32
    first, gather.rs:203-207 — the same values).  Byte work: plain index arithmetic."""
    data = np.asarray(data)
    idx = np.asarray(indices).astype(np.int64)
    nd = data.ndim
    ax = axis + nd if axis < 0 else axis
    if nd < 1 or not 0 <= ax < nd:
        raise OracleError("Gather: axis %d out of range for rank %d" % (axis, nd))
    alen = data.shape[ax]
    out_shape = data.shape[:ax] + idx.shape + data.shape[ax + 1:]
    outer = int(np.prod(data.shape[:ax], dtype=np.int64))
    inner = int(np.prod(data.shape[ax + 1:], dtype=np.int64))
    flat = np.ascontiguousarray(data).reshape(outer, alen, inner)
    k = idx.reshape(-1).copy()
    k[k < 0] += alen
    k = np.clip(k, 0, max(alen - 1, 0))
    out = np.empty((outer, k.size, inner), data.dtype)
    for i, kk in enumerate(k.tolist()):
        out[:, i, :] = flat[:, kk, :]
    return out.reshape(out_shape)


# ---- encoder ops (fp32) ------------------------------------------------------------------
def _f32(x):
    return _contig(x, np.float32)


def sum_unrolled8(x):
    """f32 sum in ndarray 0.16's unrolled_fold order (eight strided partials)."""
    x = _f32(x).reshape(-1)
    return np.float32(_load().orc_sum_unrolled8(_ptr(x), x.size))


def _last_axis(x, axis):
    if axis not in (-1, x.ndim - 1):
        raise OracleError("only the last axis is supported (got axis %d of rank %d)"
                          % (axis, x.ndim))


def layer_norm(x, scale, bias, eps=1e-5, axis=-1):
    x = _f32(x)
    _last_axis(x, axis)
    cols = x.shape[-1]
    scale, bias = _f32(scale).reshape(-1), _f32(bias).reshape(-1)
    if scale.size != cols or bias.size != cols:
        raise OracleError("LayerNorm: cannot broadcast scale/bias to the last axis")
    y = np.empty_like(x)
    _load().orc_layer_norm(_ptr(x), x.size // max(cols, 1), cols, _ptr(scale), _ptr(bias),
                           ctypes.c_float(eps), _ptr(y))
    return y


def reduce_mean(x, axes=None, keepdims=True):
    """ReduceMean::forward (src/operators/reduce_mean.rs:19-105).  ``axes`` as the second
    input gives them (negative ones counted from the end); None or empty reduces every
    element (data.mean()).  Like the reference, only ``axes[0]`` is reduced.  keepdims keeps
    the reduced axis as 1; the full reduction returns the reference's rank-0 result (ONNX
    would keep every axis as 1: same value)."""
    x = _f32(x)
    lib = _load()
    if axes is None or len(axes) == 0:
        flat = x.reshape(-1)
        if flat.size == 0:
            raise OracleError("ReduceMean: mean of an empty tensor")
        y = np.empty((), np.float32)
        lib.orc_reduce_mean(_ptr(flat), 1, flat.size, 1, 0, _ptr(y))
        return y
    a = int(axes[0])
    a = a + x.ndim if a < 0 else a
    if not 0 <= a < x.ndim:
        raise OracleError("ReduceMean: axis %d out of range for rank %d" % (axes[0], x.ndim))
    outer = int(np.prod(x.shape[:a], dtype=np.int64))
    alen = x.shape[a]
    inner = int(np.prod(x.shape[a + 1:], dtype=np.int64))
    if alen == 0:
        raise OracleError("ReduceMean: mean_axis of an empty axis")
    sequential = 1 if (x.ndim > 1 and a != x.ndim - 1) else 0
    y = np.empty((outer, inner), np.float32)
    lib.orc_reduce_mean(_ptr(x), outer, alen, inner, sequential, _ptr(y))
    shape = list(x.shape)
    if keepdims:
        shape[a] = 1
    else:
        del shape[a]
    return y.reshape(shape)


def pow(x, e):
    """Pow::forward (src/operators/pow.rs:18-45): the exponent broadcast to the base's shape
    (the reference panics when it does not broadcast), powf per element."""
    x, e = _f32(x), _f32(e)
    try:
        eb = np.ascontiguousarray(np.broadcast_to(e, x.shape))
    except ValueError:
        raise OracleError("Pow: exponent %s does not broadcast to base %s"
                          % (list(e.shape), list(x.shape)))
    y = np.empty_like(x)
    _load().orc_pow_f32(_ptr(x), _ptr(eb), x.size, _ptr(y))
    return y


def sqrt(x):
    """Sqrt::forward (src/operators/sqrt.rs:18-30)."""
    x = _f32(x)
    y = np.empty_like(x)
    _load().orc_sqrt_f32(_ptr(x), x.size, _ptr(y))
    return y


def layer_norm_decomposed(x, scale, bias, eps, residual=None, square=False):
    """The LayerNorm an export below opset 17 writes, run node by node as the reference's
    GraphExecutor runs it (src/graph_executor.rs:356-432): [x = Add(x, residual)];
    mean = ReduceMean(x, [-1]); c = Sub(x, mean); v = ReduceMean(Pow(c, 2), [-1]);
    y = Div(c, Sqrt(Add(v, eps))) [; Mul(y, scale)] [; Add(y, bias)] (scale / bias None:
    absent).  ``square=True`` replaces Pow(c, 2) by Mul(c, c), the correctly rounded square
    (the LayerNormalization operator's arithmetic)."""
    x = _f32(x)
    if residual is not None:
        x = add(x, residual)
    mean = reduce_mean(x, [-1])
    c = sub(x, mean)
    sq = mul(c, c) if square else pow(c, np.float32(2.0))
    v = reduce_mean(sq, [-1])
    y = div(c, sqrt(add(v, np.float32(eps))))
    if scale is not None:
        y = mul(y, scale)
    if bias is not None:
        y = add(y, bias)
    return y


def softmax(x, axis=-1):
    x = _f32(x)
    _last_axis(x, axis)
    y = np.empty_like(x)
    cols = x.shape[-1]
    _load().orc_softmax_last(_ptr(x), x.size // max(cols, 1), cols, _ptr(y))
    return y


def erf(x):
    x = _f32(x)
    y = np.empty_like(x)
    _load().orc_erf(_ptr(x), x.size, _ptr(y))
    return y


def matmul_f32(a, b):
    """Batched a @ b with the reference's batch rules: equal batch dims, or one side
    without batch dims (matmul.rs:68-86)."""
    a, b = _f32(a), _f32(b)
    if a.ndim < 2 or b.ndim < 2 or a.shape[-1] != b.shape[-2]:
        raise OracleError("MatMul: inner dimensions must match")
    M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
    ab, bb = a.shape[:-2], b.shape[:-2]
    if not ab and bb:
        a = np.ascontiguousarray(np.broadcast_to(a, bb + (M, K)))
        batch, out_b, b_bcast = int(np.prod(bb)), bb, 0
    elif ab and not bb:
        batch, out_b, b_bcast = int(np.prod(ab)), ab, 1
    elif ab == bb:
        batch, out_b, b_bcast = int(np.prod(ab)) if ab else 1, ab, 0
    else:
        raise OracleError("MatMul: batch dimensions must be compatible")
    c = np.empty(out_b + (M, N), np.float32)
    _load().orc_matmul_f32(_ptr(a), _ptr(b), batch, b_bcast, M, K, N, _ptr(c))
    return c


def transpose(x, perm=None):
    x = np.ascontiguousarray(x)
    rank = x.ndim
    perm = list(range(rank))[::-1] if perm is None else [int(p) for p in perm]
    if sorted(perm) != list(range(rank)) or rank > 8:
        raise OracleError("Transpose: bad permutation %s" % perm)
    y = np.empty(tuple(x.shape[p] for p in perm), x.dtype)
    dims = np.array(x.shape, dtype=np.uintp)
    pm = np.array(perm, dtype=np.int32)
    _load().orc_transpose(_ptr(x), x.itemsize, rank, _ptr(dims), _ptr(pm), _ptr(y))
    return y
