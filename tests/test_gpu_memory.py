"""GPU tests of the memory half of the C ABI (streams, pool, pinned host buffers, stream-ordered
copies) and of a quantized linear driven through it alone, the way the reference's wrappers
would call the library once garboard is gone: every buffer from the pool
(src/cuda/memory_pool.rs get_* / return_tensor), host data in and out through stream-ordered
copies (src/cuda/context.rs:160-223), the DQL -> quantized-linear kernels on the context's
stream, one synchronisation at the end.  No torch anywhere in the path.

Parity: bit-exact against the oracle's op-by-op graph (DynamicQuantizeLinear, MatMulInteger,
Cast, Mul(x_scale * w_scale), Add(bias), chain), as the other epilogue tests.
"""
import ctypes

import numpy as np
import pytest

import oracle
from iconnx_amd import configs
from iconnx_amd._lib import (BCAST_COL, BCAST_SCALAR, ICX_I8, ICX_U8, OP_ADD, OP_DIV, OP_MUL,
                             OP_SUB, Chain, IconnxError, check, lib)
from iconnx_amd.memory import GpuMemoryPool, IconnxContext, PinnedArray
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def test_pool_reuses_buffers_by_size_class():
    pool = GpuMemoryPool()
    try:
        a = pool.get(1000)       # class 1024
        b = pool.get(5000)       # class 8192
        assert pool.stats() == (0, 2, 1024 + 8192)
        pool.return_buffer(a)
        c = pool.get(700)        # same class: the returned buffer, no hipMalloc
        assert c.ptr.value == a.ptr.value
        assert pool.stats() == (1, 2, 1024 + 8192)
        with pytest.raises(IconnxError):
            pool.return_buffer(a)  # already handed out again as c, then returned below
            pool.return_buffer(a)
        # at most eight free buffers are kept per class; the ninth returned is freed
        bufs = [pool.get(300) for _ in range(9)]
        held = pool.stats()[2]
        for x in bufs:
            pool.return_buffer(x)
        assert pool.stats()[2] == held - 512
        with pytest.raises(IconnxError):
            pool.return_buffer(type(b)(ctypes.c_void_p(0x1234), 8))  # not from this pool
        pool.return_buffer(b)
    finally:
        pool.destroy()


def _chain(ops):
    ch = Chain()
    ch.n_ops = len(ops)
    for i, (op, k0, p0, k1, p1) in enumerate(ops):
        o = ch.ops[i]
        o.op, o.operand_is_lhs, o.kind0, o.kind1, o.p0, o.p1 = op, 0, k0, k1, p0, p1
    return ch


@pytest.mark.parametrize("cfg,rows", [("cfg1", None), ("cfg2", [(0, 96), (2000, 2048), (4000, 4096)])])
def test_quantized_linear_through_the_memory_abi_only(cfg, rows):
    L = lib()
    d = configs.make(cfg)
    x = d["x"].reshape(-1, d["x"].shape[-1])
    M, K = x.shape
    N = d["w"].shape[1]
    ops_host = [("w_scale", np.asarray(d["w_scale"], np.float32).reshape(1)),
                ("bias", d["bias"])] + [("c%d" % i, np.asarray(c, np.float32)) for i, (_, c) in enumerate(d["chain"])]
    ctx, pool = IconnxContext(), GpuMemoryPool()
    pinned = []
    try:
        def upload(arr):
            h = PinnedArray(arr.shape, arr.dtype)
            h.array[...] = arr
            pinned.append(h)
            dbuf = pool.get(h.nbytes)
            ctx.htod_async(dbuf, h)
            return dbuf

        dx, dw = upload(x), upload(d["w"])
        dops = {name: upload(arr) for name, arr in ops_host}
        xq, xs, xzp = pool.get(M * K), pool.get(4), pool.get(1)
        ws = pool.get(L.icx_dql_workspace_size(M * K))
        s = ctx.stream
        check(L.icx_dynamic_quantize_linear(s, dx.ptr, M * K, xq.ptr, xs.ptr, xzp.ptr, None, 0, ws.ptr,
                                            ws.nbytes))
        packed, colsum = pool.get(L.icx_packed_weight_bytes(K, N)), pool.get(4 * N)
        check(L.icx_pack_weight(s, dw.ptr, ICX_I8, K, N, packed.ptr, colsum.ptr))
        opc = {"Mul": OP_MUL, "Add": OP_ADD, "Div": OP_DIV, "Sub": OP_SUB}
        chain = _chain([(OP_MUL, BCAST_SCALAR, xs.ptr, BCAST_SCALAR, dops["w_scale"].ptr),
                        (OP_ADD, BCAST_COL, dops["bias"].ptr, 0, None)]
                       + [(opc[op], BCAST_COL, dops["c%d" % i].ptr, 0, None) for i, (op, _) in enumerate(d["chain"])])
        y = pool.get(4 * M * N)
        gws = pool.get(max(1, L.icx_matmul_integer_workspace_size(M, K, N, 1)))
        check(L.icx_qlinear_f32(s, xq.ptr, ICX_U8, packed.ptr, ICX_I8, 1, colsum.ptr, M, K, N, xzp.ptr, None, 1,
                                None, ctypes.byref(chain), y.ptr, gws.ptr, gws.nbytes))
        # the dequantized output and the DQL's outputs back to pinned host memory
        hy, hq = PinnedArray((M, N), np.float32), PinnedArray((M, K), np.uint8)
        hs, hz = PinnedArray((), np.float32), PinnedArray((), np.uint8)
        pinned += [hy, hq, hs, hz]
        for h, dbuf in ((hy, y), (hq, xq), (hs, xs), (hz, xzp)):
            ctx.dtoh_async(h, dbuf)
        ctx.sync()
        assert pool.stats()[0] == 0  # every buffer fresh so far
        for dbuf in (dx, dw, xq, xs, xzp, ws, packed, colsum, y, gws, *dops.values()):
            pool.return_buffer(dbuf)

        chain_ops = [(op, c, False) for op, c in d["chain"]]
        for r0, r1 in rows or [(0, M)]:
            want = oracle.qlinear_graph(x, d["w"], d["w_zp"], d["w_scale"], d["bias"], chain_ops, rows=(r0, r1))
            assert np.array_equal(hq.array, want["xq"])
            assert bits(hs.array) == bits(np.float32(want["x_scale"])) and int(hz.array) == int(want["x_zp"])
            got, exp = hy.array[r0:r1], want["y"][r0:r1]
            bad = int(np.count_nonzero(bits(got) != bits(exp)))
            assert bad == 0, "%s rows %d:%d: %d of %d differ" % (cfg, r0, r1, bad, exp.size)
        # a second pass takes every buffer from the pool: no new hipMalloc
        misses = pool.stats()[1]
        for nbytes in (M * K, 4, 1, 4 * M * N):
            pool.return_buffer(pool.get(nbytes))
        assert pool.stats()[1] == misses
    finally:
        pool.destroy()
        for h in pinned:
            h.free()
        ctx.close()
