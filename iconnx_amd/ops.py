"""Per-op GPU wrappers over the C ABI, mirroring the reference's ``gpu_*`` functions.

Device memory and streams come from PyTorch (plumbing only): tensors are ``torch`` CUDA
tensors, every call enqueues on ``torch.cuda.current_stream()``, and workspaces come from
torch's caching allocator, so steady-state calls do not reach ``hipMalloc``.  Errors raise
:class:`IconnxError`, the analogue of the reference's ``CudaError::Kernel(String)``; the
messages carry the op name as the reference's do.

Reference counterparts (ryanoneill/iconnx):
  gpu_dynamic_quantize_linear  src/cuda/ops/quantize.rs:296-377
  gpu_matmul_integer           src/cuda/ops/quantize.rs:398-615 (+ resolve_scalar_zp :625-679)
  gpu_dequantize_linear        src/cuda/ops/quantize.rs:24-267
  gpu_cast (Int32 -> Float32)  src/cuda/ops/cast.rs:134-148
  gpu_fused_mul_add            src/cuda/kernels/fused/wrappers.rs:495-581
  gpu_fused_add_mul / sub_mul  src/cuda/kernels/fused/wrappers.rs:583-650
  gpu_fused_div_mul            src/cuda/kernels/fused/wrappers.rs:652-683
  gpu_mul / gpu_add / gpu_div  src/cuda/kernels/mod.rs (+ broadcast, src/cuda/executor/elementwise.rs:54-200)
  gpu_gather_from_gpu          src/cuda/ops/layout/mod.rs:900-1020 (gather_u8_kernel,
                               src/cuda/ops/quantize_kernels.rs:203-224)
  gpu_reduce_mean_axis         src/cuda/reduction.rs:623-700 (CPU src/operators/reduce_mean.rs)
  gpu_pow / gpu_sqrt           src/cuda/kernels/mod.rs:1407 / the "Sqrt" arm of
                               src/cuda/executor/elementwise.rs:233-250
"""
import ctypes

import numpy as np
import torch

from ._lib import (BCAST_COL, BCAST_FULL, BCAST_ROW, BCAST_SCALAR, ICX_F32, ICX_I8, ICX_I32, ICX_I64,
                   ICX_U8, MAX_CHAIN, OP_ADD, OP_DIV, OP_ERF, OP_MUL, OP_MUL_SAVED, OP_SAVE,
                   OP_SUB, Chain, IconnxError, check, lib)

ERR_SHAPE, ERR_DTYPE, ERR_INVALID, ERR_UNSUPPORTED = 2, 3, 1, 6
_DT = {torch.int8: ICX_I8, torch.uint8: ICX_U8, torch.int32: ICX_I32, torch.float32: ICX_F32}
_DT_NAME = {torch.int8: "Int8", torch.uint8: "UInt8", torch.int32: "Int32",
            torch.float32: "Float32", torch.int64: "Int64", torch.float16: "Float16"}
_OPS = {"Add": OP_ADD, "Sub": OP_SUB, "Mul": OP_MUL, "Div": OP_DIV, "Erf": OP_ERF,
        "Save": OP_SAVE, "MulSaved": OP_MUL_SAVED}
_OPERAND_FREE = ("Erf", "Save", "MulSaved")


def _name(dt):
    return _DT_NAME.get(dt, str(dt))


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise IconnxError(ERR_INVALID, "expected a device (cuda) tensor")


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------------------
# DynamicQuantizeLinear
# ---------------------------------------------------------------------------------------
def gpu_dynamic_quantize_linear(x, rowsum_row_len=None):
    """[y u8 (x's shape), y_scale f32 [], y_zero_point u8 []]; with ``rowsum_row_len`` a
    fourth tensor holds the int32 row sums of y over rows of that length."""
    if x.dtype != torch.float32:
        raise IconnxError(ERR_DTYPE, "DynamicQuantizeLinear: input must be Float32, got %s"
                          % _name(x.dtype))
    _require_cuda(x)
    x = x.contiguous()
    n = x.numel()
    dev = x.device
    y = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    scale = torch.empty((), dtype=torch.float32, device=dev)
    zp = torch.empty((), dtype=torch.uint8, device=dev)
    rowsum = None
    if rowsum_row_len:
        rowsum = torch.empty(n // rowsum_row_len, dtype=torch.int32, device=dev)
    L = lib()
    ws = _workspace(L.icx_dql_workspace_size(n), dev)
    check(L.icx_dynamic_quantize_linear(_stream(), _p(x), n, _p(y), _p(scale), _p(zp),
                                        _p(rowsum), rowsum_row_len or 0, _p(ws), ws.numel()))
    out = [y, scale, zp]
    if rowsum is not None:
        out.append(rowsum)
    return out


# ---------------------------------------------------------------------------------------
# MatMulInteger
# ---------------------------------------------------------------------------------------
def _check_int8(t, label):
    if t.dtype not in (torch.int8, torch.uint8):
        raise IconnxError(ERR_DTYPE, "MatMulInteger: %s dtype %s unsupported (must be Int8 or UInt8)"
                          % (label, _name(t.dtype)))


def resolve_zero_point(zp, operand_dtype, label, n_cols=None):
    """Validate a zero point as resolve_scalar_zp does (quantize.rs:625-679): dtype equal to
    the operand's and scalar shape ([] or [1]).  ``n_cols`` additionally admits the ONNX
    per-column [N] form for b (the reference rejects it).  Returns (tensor|None, length)."""
    if zp is None:
        return None, 1
    if zp.dtype != operand_dtype:
        raise IconnxError(ERR_DTYPE, "MatMulInteger: %s_zero_point dtype %s must match operand dtype %s"
                          % (label, _name(zp.dtype), _name(operand_dtype)))
    shape = list(zp.shape)
    if len(shape) == 0 or shape == [1]:
        return zp.contiguous(), 1
    if n_cols is not None and len(shape) == 1 and shape[0] == n_cols:
        return zp.contiguous(), n_cols
    raise IconnxError(ERR_SHAPE, "MatMulInteger: %s_zero_point must be scalar (got shape %s); "
                      "per-axis zp is only supported for b as [N]" % (label, shape))


class PackedWeight:
    """A MatMulInteger B operand packed once for the MFMA kernel: B'^T [N,K] i8 plus its
    column sums.  Built when a weight initializer is uploaded."""

    def __init__(self, b):
        _check_int8(b, "b")
        _require_cuda(b)
        if b.dim() != 2:
            raise IconnxError(ERR_SHAPE, "MatMulInteger: b must be 2-D (got %s)" % list(b.shape))
        b = b.contiguous()
        self.K, self.N = b.shape
        self.dtype = b.dtype
        self.packed = torch.empty((self.N, self.K), dtype=torch.int8, device=b.device)
        self.colsum = torch.empty(self.N, dtype=torch.int32, device=b.device)
        check(lib().icx_pack_weight(_stream(), _p(b), _DT[b.dtype], self.K, self.N,
                                    _p(self.packed), _p(self.colsum)))

    @property
    def shape(self):
        return (self.K, self.N)


def _gemm_args(a, b, a_zp, b_zp):
    _require_cuda(a, a_zp, b_zp)
    _check_int8(a, "a")
    if isinstance(b, PackedWeight):
        b_dtype, K, N = b.dtype, b.K, b.N
    else:
        _check_int8(b, "b")
        _require_cuda(b)
        if b.dim() != 2:
            raise IconnxError(ERR_SHAPE, "MatMulInteger: 2-D inputs required (got a:%s, b:%s)"
                              % (list(a.shape), list(b.shape)))
        b_dtype = b.dtype
        K, N = b.shape
    if a.dim() != 2:
        raise IconnxError(ERR_SHAPE, "MatMulInteger: 2-D inputs required (got a:%s, b:%s)"
                          % (list(a.shape), [K, N]))
    M = a.shape[0]
    if a.shape[1] != K:
        raise IconnxError(ERR_SHAPE, "MatMulInteger: K mismatch — a is [%d,%d], b is [%d,%d]"
                          % (M, a.shape[1], K, N))
    azp, _ = resolve_zero_point(a_zp, a.dtype, "a")
    bzp, bzp_len = resolve_zero_point(b_zp, b_dtype, "b", n_cols=N)
    return a.contiguous(), b_dtype, M, K, N, azp, bzp, bzp_len


def gpu_matmul_integer(a, b, a_zp=None, b_zp=None, a_rowsum=None):
    """int32 [M,N] = (a - a_zp) @ (b - b_zp).  ``b`` is a [K,N] int8/uint8 tensor or a
    :class:`PackedWeight`."""
    a, b_dtype, M, K, N, azp, bzp, bzp_len = _gemm_args(a, b, a_zp, b_zp)
    packed = isinstance(b, PackedWeight)
    out = torch.empty((M, N), dtype=torch.int32, device=a.device)
    L = lib()
    ws = _workspace(L.icx_matmul_integer_workspace_size(M, K, N, int(packed)), a.device)
    bp = b.packed if packed else b.contiguous()
    cs = b.colsum if packed else None
    check(L.icx_matmul_integer(_stream(), _p(a), _DT[a.dtype], _p(bp), _DT[b_dtype], int(packed),
                               _p(cs), M, K, N, _p(azp), _p(bzp), bzp_len, _p(a_rowsum), _p(out),
                               _p(ws), ws.numel()))
    return out


# ---------------------------------------------------------------------------------------
# Elementwise chains
# ---------------------------------------------------------------------------------------
def _bcast_kind(t, rows, cols):
    if t.numel() == 1:
        return BCAST_SCALAR
    shape = list(t.shape)
    while shape and shape[0] == 1:
        shape = shape[1:]
    if shape == [cols]:
        return BCAST_COL
    if shape == [rows, 1] or (cols == 1 and shape == [rows]):
        return BCAST_ROW
    if t.numel() == rows * cols and (not shape or shape[-1] == cols):
        return BCAST_FULL
    return None


def build_chain(ops, rows, cols):
    """``ops``: sequence of (op_name, operand, operand_is_lhs); an operand is a float32
    device tensor or a pair (t0, t1) standing for a Mul node t0*t1 feeding this op.
    Returns (Chain, keepalive list)."""
    if len(ops) > MAX_CHAIN:
        raise IconnxError(ERR_INVALID, "chain of %d ops exceeds %d" % (len(ops), MAX_CHAIN))
    ch = Chain()
    ch.n_ops = len(ops)
    keep = []
    for i, (name, operand, is_lhs) in enumerate(ops):
        if name in _OPERAND_FREE:  # erf / save / multiply by the saved value
            o = ch.ops[i]
            o.op, o.operand_is_lhs, o.kind0, o.kind1, o.p0, o.p1 = _OPS[name], 0, 0, 0, None, None
            continue
        factors = operand if isinstance(operand, (tuple, list)) else (operand,)
        kinds, ptrs = [], []
        for f in factors:
            if f.dtype != torch.float32:
                raise IconnxError(ERR_DTYPE, "%s: operand must be Float32, got %s" % (name, _name(f.dtype)))
            _require_cuda(f)
            f = f.contiguous()
            k = _bcast_kind(f, rows, cols)
            if k is None:
                raise IconnxError(ERR_SHAPE, "%s: operand shape %s does not broadcast to [%d, %d]"
                                  % (name, list(f.shape), rows, cols))
            keep.append(f)
            kinds.append(k)
            ptrs.append(f.data_ptr())
        o = ch.ops[i]
        o.op = _OPS[name]
        o.operand_is_lhs = 1 if is_lhs else 0
        o.kind0, o.p0 = kinds[0], ptrs[0]
        if len(ptrs) > 1:
            o.kind1, o.p1 = kinds[1], ptrs[1]
        else:
            o.kind1, o.p1 = 0, None
    return ch, keep


def gpu_fused_chain(x, ops, out=None):
    """y = ops applied in order to x (float32), one rounding per op, [last-dim] broadcast."""
    if x.dtype != torch.float32:
        raise IconnxError(ERR_DTYPE, "fused_chain: input must be Float32, got %s" % _name(x.dtype))
    _require_cuda(x)
    x = x.contiguous()
    cols = x.shape[-1] if x.dim() > 0 else 1
    rows = x.numel() // cols if cols else 0
    ch, keep = build_chain(ops, rows, cols)
    y = out if out is not None else torch.empty_like(x)
    check(lib().icx_fused_chain_f32(_stream(), _p(x), rows, cols, ctypes.byref(ch), _p(y)))
    del keep
    return y


def _same_or_bcast(a, b, who):
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise IconnxError(ERR_DTYPE, "%s: Float32 operands required" % who)


def gpu_fused_mul_add(a, b, c):
    """a * b + c (two roundings; b, c same shape as a or broadcast along the last dim)."""
    _same_or_bcast(a, b, "fused_mul_add")
    return gpu_fused_chain(a, [("Mul", b, False), ("Add", c, False)])


def gpu_fused_add_mul(a, b, c):
    """(a + b) * c."""
    _same_or_bcast(a, b, "fused_add_mul")
    return gpu_fused_chain(a, [("Add", b, False), ("Mul", c, False)])


def gpu_fused_sub_mul(a, b, c):
    """(a - b) * c."""
    _same_or_bcast(a, b, "fused_sub_mul")
    return gpu_fused_chain(a, [("Sub", b, False), ("Mul", c, False)])


def gpu_fused_div_mul(a, b, c):
    """(a / b) * c with IEEE division; unlike the reference wrapper, [last-dim] broadcast
    operands are accepted."""
    _same_or_bcast(a, b, "fused_div_mul")
    return gpu_fused_chain(a, [("Div", b, False), ("Mul", c, False)])


def gpu_binary(op_name, a, b):
    """Broadcasting Add/Sub/Mul/Div where one operand has the output shape."""
    _same_or_bcast(a, b, op_name)
    out_shape = torch.broadcast_shapes(a.shape, b.shape)
    if tuple(a.shape) == tuple(out_shape):
        return gpu_fused_chain(a, [(op_name, b, False)])
    if tuple(b.shape) == tuple(out_shape):
        return gpu_fused_chain(b, [(op_name, a, True)])
    raise IconnxError(ERR_SHAPE, "%s: shapes %s and %s: neither operand has the broadcast shape"
                      % (op_name, list(a.shape), list(b.shape)))


def gpu_cast_i32_f32(x):
    if x.dtype != torch.int32:
        raise IconnxError(ERR_DTYPE, "Cast: expected Int32 input, got %s" % _name(x.dtype))
    _require_cuda(x)
    x = x.contiguous()
    y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    check(lib().icx_cast_i32_f32(_stream(), _p(x), x.numel(), _p(y)))
    return y


# ---------------------------------------------------------------------------------------
# Quantized linear (MatMulInteger + Cast + dequant Mul + bias Add + chain, one kernel)
# ---------------------------------------------------------------------------------------
def gpu_qlinear(a, b, a_zp=None, b_zp=None, epilogue=(), a_rowsum=None, out=None):
    """float32 [M,N] = epilogue(Cast(MatMulInteger(a, b, a_zp, b_zp))).  ``epilogue`` is a
    chain as in :func:`build_chain` (e.g. [("Mul", (x_scale, w_scale), False),
    ("Add", bias, False), ...])."""
    a, b_dtype, M, K, N, azp, bzp, bzp_len = _gemm_args(a, b, a_zp, b_zp)
    packed = isinstance(b, PackedWeight)
    ch, keep = build_chain(list(epilogue), M, N)
    y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=a.device)
    L = lib()
    ws = _workspace(L.icx_matmul_integer_workspace_size(M, K, N, int(packed)), a.device)
    bp = b.packed if packed else b.contiguous()
    cs = b.colsum if packed else None
    check(L.icx_qlinear_f32(_stream(), _p(a), _DT[a.dtype], _p(bp), _DT[b_dtype], int(packed),
                            _p(cs), M, K, N, _p(azp), _p(bzp), bzp_len, _p(a_rowsum),
                            ctypes.byref(ch), _p(y), _p(ws), ws.numel()))
    del keep
    return y


def exchange_buffer():
    """A zeroed exchange buffer (icx_exchange_buffer_size() bytes) for the single-launch
    entry points; keep it and pass it to every later call on the same stream."""
    return torch.zeros(lib().icx_exchange_buffer_size(), dtype=torch.uint8, device="cuda")


def gpu_dql_qlinear(x, b, epilogue, sync, out=None):
    """DynamicQuantizeLinear(x) and the quantized linear that reads it, as one launch:
    returns (y u8, y_scale, y_zp, Y f32), equal bit for bit to gpu_dynamic_quantize_linear(x)
    followed by gpu_qlinear(y, b, y_zp, epilogue=...).  ``b``: a PackedWeight of an Int8
    weight (no zero point); ``epilogue(y_scale)`` returns the chain (its reads of the scale,
    e.g. ("Mul", (y_scale, w_scale), False), see the DQL's output tensor); ``sync`` from
    exchange_buffer().  Raises IconnxError(ICX_ERR_UNSUPPORTED) for shapes outside the fused
    kernel."""
    if x.dtype != torch.float32 or x.dim() != 2:
        raise IconnxError(ERR_DTYPE, "DQL+QLinear: x must be a 2-D Float32 tensor")
    if not isinstance(b, PackedWeight):
        raise IconnxError(ERR_INVALID, "DQL+QLinear: the weight must be a PackedWeight")
    _require_cuda(x, sync)
    x = x.contiguous()
    M, K = x.shape
    N = b.shape[1]
    y = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    ys = torch.empty((), dtype=torch.float32, device=x.device)
    yz = torch.empty((), dtype=torch.uint8, device=x.device)
    ch, keep = build_chain(list(epilogue(ys)), M, N)
    Y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=x.device)
    check(lib().icx_dql_qlinear_f32(_stream(), _p(x), M, K, _p(y), _p(ys), _p(yz), _p(b.packed),
                                    _DT[b.dtype], _p(b.colsum), N, ctypes.byref(ch), _p(Y), _p(sync)))
    del keep
    return y, ys, yz, Y


# ---------------------------------------------------------------------------------------
# DequantizeLinear
# ---------------------------------------------------------------------------------------
def gpu_dequantize_linear(x, scale, zp=None, axis=1):
    """(x - zp) * scale as the CPU forward computes it; validation as quantize.rs:33-95."""
    if x.dtype not in (torch.int8, torch.uint8, torch.int32):
        raise IconnxError(ERR_DTYPE, "DequantizeLinear: input dtype %s unsupported" % _name(x.dtype))
    if scale.dtype != torch.float32:
        raise IconnxError(ERR_DTYPE, "DequantizeLinear: scale must be Float32, got %s"
                          % _name(scale.dtype))
    _require_cuda(x, scale, zp)
    shape = list(x.shape)
    n = x.numel()
    per_tensor = scale.dim() == 0 or (scale.dim() == 1 and scale.numel() == 1)
    if per_tensor:
        axis_size, inner = 1, max(n, 1)
    else:
        ax = axis + len(shape) if axis < 0 else axis
        if not 0 <= ax < len(shape):
            raise IconnxError(ERR_SHAPE, "DequantizeLinear: axis %d out of range for ndim %d"
                              % (axis, len(shape)))
        axis_size = shape[ax]
        if scale.numel() != axis_size:
            raise IconnxError(ERR_SHAPE, "DequantizeLinear: per-axis scale length %d doesn't match "
                              "input shape[%d] = %d" % (scale.numel(), ax, axis_size))
        inner = 1
        for d in shape[ax + 1:]:
            inner *= d
    if zp is not None:
        if zp.dtype != x.dtype:
            raise IconnxError(ERR_DTYPE, "DequantizeLinear: zero_point dtype %s must match input dtype %s"
                              % (_name(zp.dtype), _name(x.dtype)))
        if list(zp.shape) != list(scale.shape):
            raise IconnxError(ERR_SHAPE, "DequantizeLinear: zero_point shape %s must match scale shape %s"
                              % (list(zp.shape), list(scale.shape)))
        zp = zp.contiguous()
    x = x.contiguous()
    scale = scale.contiguous()
    y = torch.empty(shape, dtype=torch.float32, device=x.device)
    check(lib().icx_dequantize_linear_f32(_stream(), _p(x), _DT[x.dtype], _p(scale), _p(zp), n,
                                          axis_size, inner, _p(y)))
    return y


# ---------------------------------------------------------------------------------------
# Encoder ops (fp32)
# ---------------------------------------------------------------------------------------
def _f32_cuda(*ts):
    for t in ts:
        if t is not None:
            _require_cuda(t)
            if t.dtype != torch.float32:
                raise IconnxError(ERR_DTYPE, "expected Float32, got %s" % _name(t.dtype))


def gpu_layer_norm(x, scale, bias, eps=1e-5, residual=None):
    """LayerNormalization over the last axis of x (or of x + residual).  ``scale`` / ``bias``
    may be None: no Mul / Add (the node-by-node norm without its affine tail)."""
    _f32_cuda(x, scale, bias, residual)
    x = x.contiguous()
    cols = x.shape[-1]
    if (scale is not None and scale.numel() != cols) or (bias is not None and bias.numel() != cols):
        raise IconnxError(ERR_SHAPE, "LayerNorm: scale/bias must have %d elements" % cols)
    if residual is not None:
        if residual.shape != x.shape:
            raise IconnxError(ERR_SHAPE, "LayerNorm: residual shape differs from the input")
        residual = residual.contiguous()
    y = torch.empty_like(x)
    check(lib().icx_layer_norm_f32(_stream(), _p(x), _p(residual), x.numel() // cols, cols,
                                   _p(None if scale is None else scale.contiguous()),
                                   _p(None if bias is None else bias.contiguous()),
                                   ctypes.c_float(eps), _p(y)))
    return y


def gpu_reduce_mean(x, axes=None, keepdims=True):
    """ReduceMean (src/operators/reduce_mean.rs:19-105; the reference GPU's
    gpu_reduce_mean_axis, src/cuda/reduction.rs:623-700, is the last-axis case): one axis
    (negative from the end), or None / [] for every element; ndarray's summation order."""
    _f32_cuda(x)
    x = x.contiguous()
    r = x.dim()
    if not axes:
        y = torch.empty([1] * r if keepdims else [], dtype=torch.float32, device=x.device)
        check(lib().icx_reduce_mean_f32(_stream(), _p(x), 1, x.numel(), 1, 0, _p(y)))
        return y
    if len(axes) != 1:
        raise IconnxError(ERR_UNSUPPORTED, "ReduceMean: one axis is on this path")
    a = axes[0] + r if axes[0] < 0 else axes[0]
    if not 0 <= a < r:
        raise IconnxError(ERR_SHAPE, "ReduceMean: axis %d out of range for rank %d" % (axes[0], r))
    shape = list(x.shape)
    outer, alen = int(np.prod(shape[:a], dtype=np.int64)), shape[a]
    inner = int(np.prod(shape[a + 1:], dtype=np.int64))
    oshape = shape[:a] + ([1] if keepdims else []) + shape[a + 1:]
    y = torch.empty(oshape, dtype=torch.float32, device=x.device)
    check(lib().icx_reduce_mean_f32(_stream(), _p(x), outer, alen, inner, int(a != r - 1), _p(y)))
    return y


def gpu_reduce_mean_axis(x):
    """The reference GPU's last-axis ReduceMean (src/cuda/reduction.rs:623-700): [..., N] ->
    [...] (a 1-D input gives [1])."""
    y = gpu_reduce_mean(x, [-1], keepdims=False)
    return y.reshape(1) if y.dim() == 0 else y


def gpu_pow(base, exp):
    """Pow (src/operators/pow.rs:18-45; GPU gpu_pow, src/cuda/kernels/mod.rs:1407): the
    exponent broadcast over the base; exponent 2 is the correctly rounded square."""
    _f32_cuda(base, exp)
    base = base.contiguous()
    cols = base.shape[-1] if base.dim() else 1
    rows = base.numel() // max(cols, 1)
    kind = _bcast_kind(exp, rows, cols) if base.dim() else BCAST_SCALAR
    if kind is None or (exp.numel() != 1 and exp.dim() > base.dim()):
        raise IconnxError(ERR_SHAPE, "Pow: exponent %s does not broadcast over the base %s"
                          % (list(exp.shape), list(base.shape)))
    y = torch.empty_like(base)
    check(lib().icx_pow_f32(_stream(), _p(base), rows, cols, _p(exp.contiguous()), kind, _p(y)))
    return y


def gpu_sqrt(x):
    """Sqrt (src/operators/sqrt.rs:18-30): correctly rounded."""
    _f32_cuda(x)
    x = x.contiguous()
    y = torch.empty_like(x)
    check(lib().icx_sqrt_f32(_stream(), _p(x), x.numel(), _p(y)))
    return y


def gpu_softmax(x):
    _f32_cuda(x)
    x = x.contiguous()
    cols = x.shape[-1]
    y = torch.empty_like(x)
    check(lib().icx_softmax_f32(_stream(), _p(x), x.numel() // max(cols, 1), cols, _p(y)))
    return y


def gpu_erf(x):
    """Erf (the reference's Abramowitz-Stegun evaluation) as a one-step chain."""
    return gpu_fused_chain(x, [("Erf", None, False)])


def gpu_transpose(x, perm=None):
    _require_cuda(x)
    x = x.contiguous()
    rank = x.dim()
    perm = list(range(rank))[::-1] if perm is None else [int(p) for p in perm]
    y = torch.empty([x.shape[p] for p in perm], dtype=x.dtype, device=x.device)
    dims = (ctypes.c_int64 * max(rank, 1))(*x.shape)
    pm = (ctypes.c_int * max(rank, 1))(*perm)
    check(lib().icx_transpose(_stream(), _p(x), x.element_size(), rank, dims, pm, _p(y)))
    return y


def gpu_matmul_f32(a, b):
    """Batched a @ b with the reference's batch rules (equal batch dims or b without)."""
    _f32_cuda(a, b)
    a, b = a.contiguous(), b.contiguous()
    M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
    if b.shape[-2] != K:
        raise IconnxError(ERR_SHAPE, "MatMul: inner dimensions must match")
    ab, bb = tuple(a.shape[:-2]), tuple(b.shape[:-2])
    if bb and ab != bb:
        raise IconnxError(ERR_SHAPE, "MatMul: batch dimensions must be compatible")
    batch = 1
    for d in ab:
        batch *= d
    c = torch.empty(ab + (M, N), dtype=torch.float32, device=a.device)
    check(lib().icx_matmul_f32(_stream(), _p(a), _p(b), batch, 0 if bb else 1, M, K, N, _p(c)))
    return c


def gpu_attention(q, k, v, heads, scale, scale_div=True, scale_q=False):
    """Fused self-attention over [B, S, H*D] tensors (see icx_attention_f32)."""
    _f32_cuda(q, k, v)
    B, S, HD = q.shape
    D = HD // heads
    out = torch.empty_like(q)
    check(lib().icx_attention_f32(_stream(), _p(q.contiguous()), _p(k.contiguous()),
                                  _p(v.contiguous()), B, S, heads, D, HD, HD, HD, HD,
                                  ctypes.c_float(scale), 1 if scale_div else 0,
                                  1 if scale_q else 0, _p(out)))
    return out


# ---------------------------------------------------------------------------------------
# Gather
# ---------------------------------------------------------------------------------------
def gpu_gather_from_gpu(data, indices, axis=0):
    """ONNX Gather with device indices: ``data.shape[:axis] + indices.shape +
    data.shape[axis+1:]``, the data dtype kept (UInt8 for DistilBERT-INT8's embedding table);
    a negative index counts from the end and one still outside the axis is clamped, as the
    reference's gather kernels do (the reference wrapper takes axis 0 only and transposes for
    the others, src/cuda/executor/layout.rs:260-330)."""
    _require_cuda(data, indices)
    if indices.dtype not in (torch.int64, torch.int32):
        raise IconnxError(ERR_DTYPE, "Gather: indices must be Int64 or Int32, got %s" % _name(indices.dtype))
    nd = data.dim()
    ax = axis + nd if axis < 0 else axis
    if nd < 1 or not 0 <= ax < nd:
        raise IconnxError(ERR_SHAPE, "Gather: axis %d out of range for rank-%d data" % (axis, nd))
    data, indices = data.contiguous(), indices.contiguous()
    shape = list(data.shape)
    outer, inner = 1, 1
    for d in shape[:ax]:
        outer *= d
    for d in shape[ax + 1:]:
        inner *= d
    out = torch.empty(shape[:ax] + list(indices.shape) + shape[ax + 1:], dtype=data.dtype, device=data.device)
    check(lib().icx_gather(_stream(), _p(data), data.element_size(), outer, shape[ax], inner, _p(indices),
                           ICX_I64 if indices.dtype == torch.int64 else ICX_I32, indices.numel(), _p(out)))
    return out
