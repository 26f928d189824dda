"""GPU: a caller that uses nothing but the C ABI sees a device-side failure of a run as an
error status, the reference's CudaError::Kernel (src/cuda/executor/mod.rs:169-186).

The sequence is a drop-in binding's ``run``: icx_graph_run, the outputs'
device pointers from icx_graph_get_output, icx_memcpy_d2h_async into pinned host memory,
icx_stream_synchronize, then icx_graph_status.  A DynamicQuantizeLinear of a batch-1
activation ([1, 128, 768]) runs as the single-launch exchange, whose blocks wait for one
another; the host-side test hook (icx_debug_qout_fault) makes every wait expect a tag no
block publishes, with a 64 us bound, so every block takes the failure path and exits
normally.  The status must be ICX_ERR_KERNEL — also when the check is given another stream
than the run's — and a normal run afterwards must be correct.
"""
import ctypes

import numpy as np
import pytest

import oracle
from iconnx_amd._lib import ICX_F32, lib

pytestmark = pytest.mark.gpu
P = ctypes.c_void_p


def cstrs(names):
    return (ctypes.c_char_p * len(names))(*[n.encode() for n in names])


def dims(shape):
    return (ctypes.c_int64 * max(len(shape), 1))(*shape)


def build(L):
    g = L.icx_graph_create()
    assert g
    assert L.icx_graph_add_input(g, b"x", 3, dims([1, 128, 768])) == 0
    outs = ["y", "s", "zp"]
    assert L.icx_graph_add_node(g, b"dql", b"DynamicQuantizeLinear", 1, cstrs(["x"]), 3, cstrs(outs), 0,
                                None, None) == 0
    for o in outs:
        assert L.icx_graph_add_output(g, o.encode()) == 0
    return g


def run_and_copy(L, g, stream, x, host):
    """The binding's run: enqueue, copy every output to pinned host memory, synchronise."""
    assert L.icx_graph_set_input(g, b"x", ICX_F32, 3, dims(x.shape), x.ctypes.data_as(P), 0) == 0
    assert L.icx_graph_run(g, stream) == 0
    for name, (buf, nbytes) in host.items():
        dt, rk = ctypes.c_int(), ctypes.c_int()
        dd = (ctypes.c_int64 * 8)()
        ptr = ctypes.c_void_p()
        assert L.icx_graph_get_output(g, name.encode(), ctypes.byref(dt), ctypes.byref(rk), dd,
                                      ctypes.byref(ptr)) == 0
        assert L.icx_memcpy_d2h_async(stream, buf, ptr, nbytes) == 0
    assert L.icx_stream_synchronize(stream) == 0
    out = {}
    for name, (buf, nbytes) in host.items():
        out[name] = bytes((ctypes.c_ubyte * nbytes).from_address(buf.value))
    return out


def test_failed_exchange_is_an_error_status_through_the_c_abi_only():
    L = lib()
    stream, other = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.icx_stream_create(ctypes.byref(stream)) == 0
    assert L.icx_stream_create(ctypes.byref(other)) == 0
    x = np.random.default_rng(12).standard_normal((1, 128, 768)).astype(np.float32)
    n = x.size
    host = {}
    for name, nbytes in (("y", n), ("s", 4), ("zp", 1)):
        buf = ctypes.c_void_p()
        assert L.icx_host_alloc(nbytes, ctypes.byref(buf)) == 0
        host[name] = (buf, nbytes)
    g = build(L)
    try:
        assert L.icx_graph_compile(g, stream) == 0
        L.icx_debug_qout_fault(64)
        try:
            got = run_and_copy(L, g, stream, x, host)
        finally:
            L.icx_debug_qout_fault(0)
        assert np.isnan(np.frombuffer(got["s"], np.float32)[0])
        assert not np.frombuffer(got["y"], np.uint8).any()
        assert L.icx_graph_status(g, stream) == 7  # ICX_ERR_KERNEL
        assert b"range exchange" in L.icx_last_error()
        assert L.icx_graph_status(g, stream) == 0  # the record is cleared by the check
        # the check waits for the run's own stream when given another one
        L.icx_debug_qout_fault(64)
        try:
            assert L.icx_graph_set_input(g, b"x", ICX_F32, 3, dims(x.shape), x.ctypes.data_as(P), 0) == 0
            assert L.icx_graph_run(g, stream) == 0
        finally:
            L.icx_debug_qout_fault(0)
        assert L.icx_graph_status(g, other) == 7
        # a normal run is correct and clean
        got = run_and_copy(L, g, stream, x, host)
        assert L.icx_graph_status(g, stream) == 0
        yq, ys, yz = oracle.dynamic_quantize_linear(x)
        assert np.array_equal(np.frombuffer(got["y"], np.uint8), yq.reshape(-1))
        assert np.frombuffer(got["s"], np.uint32)[0] == np.float32(ys).view(np.uint32)
        assert np.frombuffer(got["zp"], np.uint8)[0] == int(yz)
    finally:
        L.icx_graph_destroy(g)
        for buf, _ in host.values():
            L.icx_host_free(buf)
        L.icx_stream_destroy(stream)
        L.icx_stream_destroy(other)
