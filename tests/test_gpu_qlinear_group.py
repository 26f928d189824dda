"""GPU: sibling quantized linears (several heads over one DynamicQuantizeLinear, like an
attention block's Q / K / V projections) run as one GEMM over the column-concatenated
weight, each head's output written as its own tensor.

Every head's output must equal, bit for bit, the oracle's op-by-op evaluation of that head
(oracle.qlinear_graph follows src/graph_executor.rs:356-432) — or, for GELU heads, the same
head run on its own through the executor, whose single-head path the other GPU tests pin to
the oracle.  Heads differ in weights, scalar / per-column scales, biases and chain
constants, so a segment that read another head's operands or weights would show.  The
cases reach each GEMM main loop: LDS-DMA (K % 64 == 0), register-staged (K = 72), the
256 x 256 tile (many tiles) and the persistent producer / consumer kernel (K >= 2048, few
tiles)."""
import numpy as np
import pytest
import torch

import oracle
from iconnx_amd import graphs
from iconnx_amd.executor import GpuGraphExecutor
from tests.golden_util import bits

pytestmark = pytest.mark.gpu


def assert_bits_equal(got, want, what):
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = int(np.count_nonzero(bits(got) != bits(want)))
    assert bad == 0, "%s: %d of %d elements differ" % (what, bad, want.size)


def head_params(rng, K, N, i, per_col_scale):
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    sc = rng.uniform(2e-4, 9e-4, N).astype(np.float32) if per_col_scale else np.float32(rng.uniform(2e-4, 9e-4))
    b = (0.02 * rng.standard_normal(N)).astype(np.float32)
    chain = [("Mul", np.float32(0.5 + 0.25 * i)), ("Add", rng.standard_normal(N).astype(np.float32))]
    return w, sc, b, chain


def build(rows, K, N, n_heads, seed, per_col=(), gelu=False, chain=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, K])
    dql = graphs.add_dynamic_quantize(ex, "x", "sib")
    params, outs = [], []
    for i in range(n_heads):
        w, sc, b, ch = head_params(rng, K, N, i, i in per_col)
        ch = ch if chain else []
        params.append((w, sc, b, ch))
        outs.append(graphs.add_quantized_linear(ex, "x", w, np.int8(0), sc, b, ch, prefix="h%d" % i,
                                                dql=dql, gelu=gelu))
    return ex, x, params, outs


def groups_of(ex):
    entries, _ = ex.plan()
    return {e.node: e.group for e in entries if e.pattern == "QuantizedLinear" and e.kind == "FusedHead"}


def check_vs_oracle(got, x, params, outs, rows=None):
    for i, (o, (w, sc, b, ch)) in enumerate(zip(outs, params)):
        ref = oracle.qlinear_graph(x, w, np.int8(0), sc, b, [(op, c, False) for op, c in ch], rows=rows)
        g = got[o]
        if rows is not None:
            assert_bits_equal(g[rows[0]:rows[1]], ref["y"][rows[0]:rows[1]], "head %d rows %s" % (i, rows))
        else:
            assert_bits_equal(g, ref["y"], "head %d" % i)


@pytest.mark.parametrize("rows,K,N", [(300, 256, 256), (129, 768, 512), (64, 72, 256)],
                         ids=["dma-ragged", "dma-768", "reg-K72"])
def test_three_siblings_one_launch(rows, K, N):
    ex, x, params, outs = build(rows, K, N, 3, seed=rows + K, per_col=(1,))
    got = ex.run({"x": torch.from_numpy(x).cuda()}, outs)
    g = groups_of(ex)
    assert g == {"h0.mmi": "h0.mmi", "h1.mmi": "h0.mmi", "h2.mmi": "h0.mmi"}
    check_vs_oracle(got, x, params, outs)


def test_five_siblings_split_four_plus_one():
    ex, x, params, outs = build(200, 128, 256, 5, seed=51, per_col=(0, 3))
    got = ex.run({"x": torch.from_numpy(x).cuda()}, outs)
    g = groups_of(ex)
    assert [g["h%d.mmi" % i] for i in range(5)] == ["h0.mmi"] * 4 + [None]
    check_vs_oracle(got, x, params, outs)
    # a second run reuses the packed group weight and pooled buffers
    x2 = np.random.default_rng(52).standard_normal((77, 128)).astype(np.float32)
    got2 = ex.run({"x": x2}, outs)
    check_vs_oracle(got2, x2, params, outs)


def test_big_tile_path_sampled_rows():
    # 16384 x (3 x 512): 64 x 6 256-wide tiles >= 512 -> the 256 x 256 kernel.  The DQL
    # range is over all of x; the rest of each head is row-wise, so the oracle runs its
    # ops (the same ones qlinear_graph chains) on the sampled rows only.
    ex, x, params, outs = build(16384, 128, 512, 3, seed=61)
    got = ex.run({"x": torch.from_numpy(x).cuda()}, outs)
    assert set(groups_of(ex).values()) == {"h0.mmi"}
    xq, xs, xzp = oracle.dynamic_quantize_linear(x)
    for i, (o, (w, sc, b, ch)) in enumerate(zip(outs, params)):
        for r0, r1 in ((0, 300), (8000, 8300), (16384 - 260, 16384)):
            y = oracle.mul(oracle.cast_i32_f32(oracle.matmul_integer(xq[r0:r1], w, xzp, np.int8(0))),
                           oracle.mul(xs, sc))
            y = oracle.add(y, b)
            for op, c in ch:
                y = {"Mul": oracle.mul, "Add": oracle.add}[op](y, c)
            assert_bits_equal(got[o][r0:r1], y, "head %d rows %d:%d" % (i, r0, r1))


def test_stream_kernel_path():
    # K = 2048, 8 x 12 64-wide tiles < CUs -> the persistent producer / consumer kernel
    ex, x, params, outs = build(512, 2048, 256, 3, seed=71)
    got = ex.run({"x": torch.from_numpy(x).cuda()}, outs)
    assert set(groups_of(ex).values()) == {"h0.mmi"}
    check_vs_oracle(got, x, params, outs)


def test_gelu_siblings_match_single_heads():
    ex, x, params, outs = build(257, 256, 512, 2, seed=81, gelu=True, chain=False)
    xd = torch.from_numpy(x).cuda()
    got = ex.run({"x": xd}, outs)
    assert set(groups_of(ex).values()) == {"h0.mmi"}
    for i, (w, sc, b, _) in enumerate(params):
        solo = GpuGraphExecutor()
        solo.add_input("x", [None, 256])
        o = graphs.add_quantized_linear(solo, "x", w, np.int8(0), sc, b, prefix="h%d" % i, gelu=True)
        assert groups_of(solo) == {"h%d.mmi" % i: None}
        want = solo.run({"x": xd}, [o])[o]
        assert_bits_equal(got[outs[i]], want, "gelu head %d" % i)
