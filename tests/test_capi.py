"""CPU-side checks of the C ABI: the library loads and exports every declared symbol.
No compute entry point is called here (there is no GPU in the build container)."""
import ctypes
import os

import pytest

from iconnx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libiconnx_hip.so not built; run `python -m iconnx_amd.build`")
    return _lib.lib()


def test_every_header_symbol_is_exported(L):
    names = _lib.header_symbols()
    assert len(names) >= 13
    for name in names:
        assert hasattr(L, name), name
    # and every exported entry point has a ctypes signature
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_status_strings_and_version(L):
    assert L.icx_status_str(0) == b"ok"
    assert L.icx_status_str(4) == b"workspace too small"
    assert b"gfx950" in L.icx_version()
    assert L.icx_last_error() == b""


def test_chain_struct_layout_matches_header():
    # icx_chain_op: 4 x int32 + 2 pointers; icx_chain: 2 x int32 + 8 ops
    assert ctypes.sizeof(_lib.ChainOp) == 32
    assert ctypes.sizeof(_lib.Chain) == 8 + 8 * 32


def test_workspace_queries_are_host_only(L):
    assert L.icx_dql_workspace_size(1 << 20) >= 8
    assert L.icx_packed_weight_bytes(768, 3072) == 768 * 3072
    ws_packed = L.icx_matmul_integer_workspace_size(4096, 768, 3072, 1)
    ws_raw = L.icx_matmul_integer_workspace_size(4096, 768, 3072, 0)
    assert ws_raw >= ws_packed + 768 * 3072 + 4 * 3072


def test_library_is_gfx950_only():
    """The shared object carries a gfx950 code object and no other GPU target."""
    with open(_lib.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in blob


def test_noalloc_matmul_rejects_an_oversized_workspace_before_any_gpu_work(L):
    """icx_matmul_integer_noalloc checks the shape's workspace against its static array
    (32 MiB) first: an unpacked 8192 x 8192 weight is refused with ICX_ERR_WORKSPACE and a
    message, without touching the (here fake) pointers or the GPU."""
    assert L.icx_matmul_integer_noalloc_max_bytes() == 32 << 20
    fake = ctypes.c_void_p(0x1000)
    rc = L.icx_matmul_integer_noalloc(None, fake, 0, fake, 0, 0, None, 16, 8192, 8192,
                                      None, None, 1, None, fake)
    assert rc == 4
    assert b"static scratch" in L.icx_last_error()


def test_pool_bookkeeping_is_host_only(L):
    """An empty pool is created, queried and destroyed without a GPU; returning a pointer it
    never handed out is an error, as the reference pool only takes back its own slices."""
    p = L.icx_pool_create()
    assert p
    h, m, b = ctypes.c_int64(-1), ctypes.c_int64(-1), ctypes.c_int64(-1)
    assert L.icx_pool_stats(p, ctypes.byref(h), ctypes.byref(m), ctypes.byref(b)) == 0
    assert (h.value, m.value, b.value) == (0, 0, 0)
    assert L.icx_pool_free(p, ctypes.c_void_p(0x1000)) == 1
    assert b"not handed out" in L.icx_last_error()
    assert L.icx_pool_free(p, None) == 0
    L.icx_pool_destroy(p)


def test_pool_rejects_a_size_without_a_size_class(L):
    """A request above the largest power-of-two class (2^63 bytes), e.g. (size_t)-1 from a bad
    size computation, is ICX_ERR_INVALID_ARG before any device call, not an endless doubling."""
    p = L.icx_pool_create()
    out = ctypes.c_void_p(0)
    try:
        for n in ((1 << 64) - 1, (1 << 63) + 1):
            assert L.icx_pool_alloc(p, n, ctypes.byref(out)) == 1
            assert out.value is None
            assert b"largest size class" in L.icx_last_error()
    finally:
        L.icx_pool_destroy(p)
