"""GPU parity of icx_matmul_integer_noalloc, the MatMulInteger entry point that allocates
nothing (its workspace is a static device array), against icx_matmul_integer with a
caller-provided workspace, through the C ABI: bit-exact int32, two calls in a row with the
second on a smaller input (the array keeps the first call's contents), packed and unpacked
weights, scalar and per-column zero points (so the row sums live in the array too), and the
size limit reported as ICX_ERR_WORKSPACE before any GPU work.

No reference counterpart: the reference's gpu_matmul_integer (src/cuda/ops/quantize.rs:398)
always allocates its output and zero-point buffers from its pool.
"""
import ctypes

import numpy as np
import pytest
import torch

from iconnx_amd import ops
from iconnx_amd._lib import ICX_I8, ICX_U8, IconnxError, check, lib

pytestmark = pytest.mark.gpu

_DT = {torch.int8: ICX_I8, torch.uint8: ICX_U8}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def noalloc(a, b, azp, bzp, packed=None, out=None):
    """icx_matmul_integer_noalloc; ``packed``: an ops.PackedWeight of ``b`` or None."""
    L = lib()
    M, K = a.shape
    N = b.shape[1]
    if out is None:
        out = torch.full((M, N), -7, dtype=torch.int32, device="cuda")
    bp = packed.packed if packed is not None else b
    cs = packed.colsum if packed is not None else None
    check(L.icx_matmul_integer_noalloc(_stream(), _p(a), _DT[a.dtype], _p(bp), _DT[b.dtype],
                                       int(packed is not None), _p(cs), M, K, N, _p(azp), _p(bzp),
                                       1 if bzp is None else bzp.numel(), None, _p(out)))
    return out


def case(rng, M, K, N, adt, bdt, per_col):
    a = torch.from_numpy(rng.integers(np.iinfo(adt).min, np.iinfo(adt).max + 1, (M, K)).astype(adt)).cuda()
    b = torch.from_numpy(rng.integers(np.iinfo(bdt).min, np.iinfo(bdt).max + 1, (K, N)).astype(bdt)).cuda()
    azp = torch.tensor(int(rng.integers(0, 20)), dtype=a.dtype).cuda()
    bzp = torch.from_numpy(rng.integers(-5, 6, N if per_col else 1).astype(bdt)).cuda()
    return a, b, azp, bzp


@pytest.mark.parametrize("packed", [False, True])
def test_noalloc_matches_the_workspace_entry_point(packed):
    rng = np.random.default_rng(71)
    shapes = [(2048, 1024, 3072, np.uint8, np.int8, True),   # 3 MiB packed weight + row sums
              (130, 96, 200, np.int8, np.int8, False)]       # smaller, ragged, right after
    for i, (M, K, N, adt, bdt, per_col) in enumerate(shapes):
        a, b, azp, bzp = case(rng, M, K, N, adt, bdt, per_col)
        pw = ops.PackedWeight(b) if packed else None
        want = ops.gpu_matmul_integer(a, pw if packed else b, azp, bzp)
        got = noalloc(a, b, azp, bzp, pw)
        torch.cuda.synchronize()
        assert torch.equal(got, want), "call %d (M=%d K=%d N=%d packed=%s): %d elements differ" % (
            i, M, K, N, packed, int((got != want).sum()))


def test_noalloc_rejects_a_workspace_beyond_its_array():
    L = lib()
    cap = L.icx_matmul_integer_noalloc_max_bytes()
    assert cap == 32 << 20
    K = N = 8192  # an unpacked 64 MiB weight would have to be packed into the array
    assert L.icx_matmul_integer_workspace_size(16, K, N, 0) > cap
    t = torch.zeros(16, dtype=torch.int8, device="cuda")
    with pytest.raises(IconnxError) as e:
        check(L.icx_matmul_integer_noalloc(_stream(), _p(t), ICX_I8, _p(t), ICX_I8, 0, None, 16, K, N,
                                           None, None, 1, None, _p(t)))
    assert e.value.status == 4 and "static scratch" in str(e.value)


def test_noalloc_allocates_nothing():
    """After a warm-up call (which resolves the static array's device address once and loads
    the kernels), further calls leave the device's free memory exactly as it was: no
    hipMalloc, no allocating library routine — for the packed and the unpacked weight."""
    rng = np.random.default_rng(72)
    a, b, azp, bzp = case(rng, 1024, 768, 3072, np.uint8, np.int8, True)
    pw = ops.PackedWeight(b)
    out = torch.empty((1024, 3072), dtype=torch.int32, device="cuda")
    want = ops.gpu_matmul_integer(a, pw, azp, bzp)
    for packed in (pw, None):  # warm-up of both forms
        noalloc(a, b, azp, bzp, packed, out)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        for packed in (pw, None):
            noalloc(a, b, azp, bzp, packed, out)
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, "packed=%s" % (packed is not None)
    assert torch.equal(out, want)
