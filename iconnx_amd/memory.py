"""Streams, the device memory pool and host transfers over the C ABI, without torch.

Mirrors what the reference's per-op wrappers get from garboard and its context / pool
(src/cuda/context.rs, src/cuda/memory_pool.rs): one stream per context, a size-class pool
whose buffers the wrappers take their outputs from, and host <-> device copies.  The
copies here are stream-ordered (the reference's dtoh blocks, context.rs:214-223); host
buffers come from pinned memory so they really run asynchronously.
"""
import ctypes

import numpy as np

from ._lib import check, lib


class DeviceBuffer:
    """A device allocation handed out by a GpuMemoryPool (``ptr`` is a c_void_p)."""

    def __init__(self, ptr, nbytes):
        self.ptr = ptr
        self.nbytes = nbytes


class PinnedArray:
    """A numpy array over pinned host memory (icx_host_alloc)."""

    def __init__(self, shape, dtype):
        self._L = lib()
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        self.ptr = ctypes.c_void_p()
        check(self._L.icx_host_alloc(max(nbytes, 1), ctypes.byref(self.ptr)))
        buf = (ctypes.c_char * max(nbytes, 1)).from_address(self.ptr.value)
        self.array = np.frombuffer(buf, dtype=np.uint8, count=nbytes).view(dtype).reshape(shape)
        self.nbytes = nbytes

    def free(self):
        if self.ptr:
            self.array = None
            check(self._L.icx_host_free(self.ptr))
            self.ptr = None


class IconnxContext:
    """The context's one stream (IconnxCudaContext, src/cuda/context.rs:22-31)."""

    def __init__(self):
        self._L = lib()
        self.stream = ctypes.c_void_p()
        check(self._L.icx_stream_create(ctypes.byref(self.stream)))

    def htod_async(self, dst, src):
        """Enqueue a copy of PinnedArray ``src`` into DeviceBuffer ``dst`` (htod, :160)."""
        assert src.nbytes <= dst.nbytes
        check(self._L.icx_memcpy_h2d_async(self.stream, dst.ptr, src.ptr, src.nbytes))

    def dtoh_async(self, dst, src):
        """Enqueue a copy of DeviceBuffer ``src`` into PinnedArray ``dst`` (dtoh, :214);
        ``dst.array`` holds the data after :meth:`sync`."""
        assert dst.nbytes <= src.nbytes
        check(self._L.icx_memcpy_d2h_async(self.stream, dst.ptr, src.ptr, dst.nbytes))

    def sync(self):
        check(self._L.icx_stream_synchronize(self.stream))

    def close(self):
        if self.stream:
            check(self._L.icx_stream_destroy(self.stream))
            self.stream = None


class GpuMemoryPool:
    """GpuMemoryPool (src/cuda/memory_pool.rs:47-545) on hipMalloc: ``get`` is the
    get_f32 / get_u8 / ... family (buffers are not zero-filled), ``return_buffer`` is
    return_tensor, ``stats`` is (hits, misses, bytes held)."""

    def __init__(self):
        self._L = lib()
        self._p = self._L.icx_pool_create()
        if not self._p:
            raise MemoryError("icx_pool_create failed")

    def get(self, nbytes):
        ptr = ctypes.c_void_p()
        check(self._L.icx_pool_alloc(self._p, nbytes, ctypes.byref(ptr)))
        return DeviceBuffer(ptr, nbytes)

    def return_buffer(self, buf):
        check(self._L.icx_pool_free(self._p, buf.ptr))

    def stats(self):
        h, m, b = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        check(self._L.icx_pool_stats(self._p, ctypes.byref(h), ctypes.byref(m), ctypes.byref(b)))
        return h.value, m.value, b.value

    def destroy(self):
        if self._p:
            self._L.icx_pool_destroy(self._p)
            self._p = None
