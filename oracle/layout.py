"""CPU oracle for the shape / mask plumbing of an exported encoder — TEST INFRASTRUCTURE ONLY.

Plain numpy index arithmetic (byte work: every result is exact), restating the reference's
operators for the ops an exported DistilBERT-INT8 uses around its quantized linears to build
reshape targets, position ids and the attention mask.  Only ``tests/`` may use it, as the
checker.

* :func:`shape` — ``src/operators/shape.rs`` (opset 15 start / end, clamped)
* :func:`unsqueeze` — ``src/operators/unsqueeze.rs:35-90``; :func:`squeeze` — GPU dispatch
  ``src/cuda/executor/layout.rs:579-613``
* :func:`concat` — ``src/operators/concat.rs``
* :func:`slice_` — the GPU Slice ``gpu_slice_nd`` (``src/cuda/ops/layout/mod.rs:2849-2939``)
  with the dispatch's parameter handling (``src/cuda/executor/layout.rs:345-456``)
* :func:`expand` — ``gpu_expand`` (``src/cuda/ops/layout/mod.rs:1624-1670``, bidirectional
  broadcast)
* :func:`equal` — ``src/operators/equal.rs``; :func:`where` — ``src/operators/where_op.rs``
* :func:`cast` — ``src/operators/cast.rs`` (Rust ``as`` semantics)

Pins (tests/test_oracle_layout.py): the ONNX 1.18 node goldens the reference vendors for each
op (tests/golden/onnx_node/test_{shape,unsqueeze,squeeze,concat,slice,expand,equal,where}_*),
numpy's own slicing / broadcasting / comparison on random cases (an independent
implementation of the same definitions), and Rust's documented ``as`` rules at the edges.
"""
import numpy as np

from . import OracleError


def _axis(a, rank, what):
    ax = a + rank if a < 0 else a
    if not 0 <= ax < rank:
        raise OracleError("%s: axis %d out of range for rank %d" % (what, a, rank))
    return ax


def shape(x_shape, start=0, end=None):
    """Int64 dims of a tensor of shape ``x_shape``, from ``start`` to ``end`` (negative ones
    counted from the rank, both clamped to [0, rank]), shape.rs."""
    r = len(x_shape)
    s = max(r + start, 0) if start < 0 else min(start, r)
    if end is None:
        e = r
    else:
        e = max(r + end, 0) if end < 0 else min(end, r)
    return np.array(list(x_shape)[s:max(e, s)], np.int64)


def unsqueeze(x, axes):
    """Insert unit dims at ``axes`` (positions in the output; negative ones counted from the
    output rank), unsqueeze.rs:57-90."""
    x = np.asarray(x)
    r = x.ndim + len(axes)
    pos = sorted(_axis(int(a), r, "Unsqueeze") for a in axes)
    if len(set(pos)) != len(pos):
        raise OracleError("Unsqueeze: repeated axis")
    shp, k = [], 0
    for d in range(r):
        if d in pos:
            shp.append(1)
        else:
            shp.append(x.shape[k])
            k += 1
    return x.reshape(shp)


def squeeze(x, axes=None):
    """Drop unit dims: all of them, or those of ``axes`` that are 1 (layout.rs:579-613)."""
    x = np.asarray(x)
    if axes is None:
        keep = [d for d in x.shape if d != 1]
    else:
        ax = {_axis(int(a), x.ndim, "Squeeze") for a in axes}
        keep = [d for i, d in enumerate(x.shape) if not (i in ax and d == 1)]
    return x.reshape(keep)


def concat(inputs, axis):
    xs = [np.asarray(t) for t in inputs]
    if not xs:
        raise OracleError("Concat requires at least 1 input tensor")
    ax = _axis(int(axis), xs[0].ndim, "Concat")
    for t in xs:
        if t.ndim != xs[0].ndim or t.dtype != xs[0].dtype or \
                any(t.shape[d] != xs[0].shape[d] for d in range(t.ndim) if d != ax):
            raise OracleError("Concat: shapes %s" % [u.shape for u in xs])
    total = sum(t.shape[ax] for t in xs)
    out = np.empty(xs[0].shape[:ax] + (total,) + xs[0].shape[ax + 1:], xs[0].dtype)
    at = 0
    for t in xs:
        idx = [slice(None)] * t.ndim
        idx[ax] = slice(at, at + t.shape[ax])
        out[tuple(idx)] = t
        at += t.shape[ax]
    return out


def slice_params(shape_, starts, ends, axes=None, steps=None):
    """Per dimension (first index, step, output length), as the reference's GPU Slice
    normalises them; starts / ends of different lengths broadcast or truncate first."""
    starts, ends = [int(v) for v in starts], [int(v) for v in ends]
    if len(starts) != len(ends):
        if len(starts) == 1 and len(ends) > 1:
            starts = starts * len(ends)
        elif len(ends) == 1 and len(starts) > 1:
            ends = ends * len(starts)
        else:
            n = min(len(starts), len(ends))
            starts, ends = starts[:n], ends[:n]
    ns = len(starts)
    axes = [int(a) for a in axes] if axes is not None and len(axes) == ns else list(range(ns))
    steps = [int(s) for s in steps] if steps is not None and len(steps) == ns else [1] * ns
    nd = len(shape_)
    first, step, end = [0] * nd, [1] * nd, list(shape_)
    for i in range(ns):
        ax = _axis(axes[i], nd, "Slice")
        if steps[i] == 0:
            raise OracleError("Slice: step cannot be 0")
        dim = shape_[ax]
        s = max(dim + starts[i], 0) if starts[i] < 0 else min(starts[i], dim)
        e = max(dim + ends[i], 0) if ends[i] < 0 else min(ends[i], dim)
        if steps[i] < 0:
            s, e = min(s, dim - 1), max(e, -1)
        else:
            s, e = max(s, 0), max(e, 0)
        first[ax], step[ax], end[ax] = s, steps[i], e
    length = []
    for d in range(nd):
        s, e, st = first[d], end[d], step[d]
        n = (e - s + st - 1) // st if st > 0 else (s - e - st - 1) // (-st)
        # Rust's `/` truncates toward zero; for a non-negative result the two agree, and a
        # negative one is clamped to 0 either way
        length.append(max(n, 0))
    return first, step, length


def slice_(x, starts, ends, axes=None, steps=None):
    """Output element i of each dimension d is input index first[d] + i * step[d]."""
    x = np.asarray(x)
    first, step, length = slice_params(x.shape, starts, ends, axes, steps)
    idx = [np.asarray([f + i * st for i in range(n)], np.int64) for f, st, n in zip(first, step, length)]
    if any(n == 0 for n in length):
        return np.empty(length, x.dtype)
    return x[np.ix_(*idx)] if x.ndim else x.copy()


def _bshape(*shapes):
    r = max(len(s) for s in shapes)
    out = []
    for d in range(r):
        dims = [s[d - (r - len(s))] if d >= r - len(s) else 1 for s in shapes]
        big = [v for v in dims if v != 1]
        if big and any(v != big[0] for v in big):
            raise OracleError("shapes %s are not broadcastable" % (shapes,))
        out.append(big[0] if big else 1)
    return out


def _read(x, out_shape):
    """x read at every index of out_shape, broadcast dims (size 1) repeated."""
    x = np.asarray(x)
    r = len(out_shape)
    xs = (1,) * (r - x.ndim) + x.shape
    x = x.reshape(xs)
    idx = [np.zeros(n, np.int64) if xs[d] == 1 else np.arange(n) for d, n in enumerate(out_shape)]
    return x[np.ix_(*idx)] if r else x.copy()


def expand(x, target):
    out = _bshape(np.asarray(x).shape, tuple(int(v) for v in target))
    return _read(x, out)


def equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype != b.dtype:
        raise OracleError("Equal: dtypes %s and %s" % (a.dtype, b.dtype))
    out = _bshape(a.shape, b.shape)
    return _read(a, out) == _read(b, out)


def where(c, x, y):
    """condition (any dtype, nonzero = true, as where_op.rs compares it as Float32) ? x : y."""
    c, x, y = np.asarray(c), np.asarray(x), np.asarray(y)
    if x.dtype != y.dtype:
        raise OracleError("Where: x and y dtypes differ")
    out = _bshape(c.shape, x.shape, y.shape)
    cc = _read(c, out) != 0
    xx, yy = _read(x, out), _read(y, out)
    res = yy.copy()
    res[cc] = xx[cc]
    return res


_ONNX = {1: np.float32, 6: np.int32, 7: np.int64, 9: np.bool_}


def cast(x, to):
    """Cast to ONNX FLOAT / INT32 / INT64 / BOOL with Rust's ``as``: integers wrap or widen,
    integer to Float32 rounds to nearest even, Float32 to an integer is NaN -> 0, saturating,
    else toward zero; to Bool is x != 0."""
    x = np.asarray(x)
    if to not in _ONNX:
        raise OracleError("Cast to %d unsupported" % to)
    dt = np.dtype(_ONNX[to])
    if dt == np.bool_:
        return x != 0
    if x.dtype == np.float32 and dt.kind == "i":
        info = np.iinfo(dt)
        out = np.zeros(x.shape, dt)
        f = x.astype(np.float64)
        ok = ~np.isnan(f)
        hi = f >= 2.0 ** (info.bits - 1)
        lo = f <= -(2.0 ** (info.bits - 1))
        mid = ok & ~hi & ~lo
        out[mid] = np.trunc(f[mid]).astype(dt)
        out[ok & hi] = info.max
        out[ok & lo] = info.min
        return out
    if dt.kind == "i" and x.dtype.kind in "iub":
        return x.astype(np.int64).astype(dt)  # wraps to the narrower type
    return x.astype(dt)
