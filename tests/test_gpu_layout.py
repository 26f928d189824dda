"""GPU: the shape and mask plumbing of an exported encoder through GpuGraphExecutor, at the
DistilBERT-INT8 sizes (batch 32, seq 128, 12 heads), every result exact against the oracle
(oracle/layout.py, pinned by the ONNX node goldens in tests/test_oracle_layout.py):

* the attention mask as the export builds it — Equal(mask, 0), a reshape target assembled from
  Shape / Gather / Unsqueeze / Concat (computed on the host), Reshape, Expand to the scores'
  Shape, Where(mask, finfo.min, scores) — eager, and captured with replays on new data;
* the position ids — Slice of a [1, 512] constant up to Shape(input_ids)[1], Gather of the
  position table, added to [B, S, D] embeddings under [1, S, D] broadcasting;
* device Concat / Slice (negative steps) / Equal (NaN) / Cast (Rust `as` edges) on tensors
  that are never host-known;
* a shape that would have to be read back from the device while the run is captured is an
  error, not a silent wrong replay.
"""
import numpy as np
import pytest
import torch

from iconnx_amd._lib import IconnxError
from iconnx_amd.executor import GpuGraphExecutor
from oracle import layout as L
from tests.golden_util import bits

pytestmark = pytest.mark.gpu
B, H, S = 32, 12, 128
FMIN = np.float32(np.finfo(np.float32).min)


def mask_graph():
    ex = GpuGraphExecutor()
    ex.add_input("scores", [None, H, None, None])
    ex.add_input("mask", [None, None])
    ex.add_initializer("zero", np.array(0, np.int64))
    ex.add_initializer("i0", np.array(0, np.int64))
    ex.add_initializer("i3", np.array(3, np.int64))
    ex.add_initializer("ax0", np.array([0], np.int64))
    ex.add_initializer("one", np.array([1], np.int64))
    ex.add_initializer("fill", FMIN)
    ex.add_node("eq", "Equal", ["mask", "zero"], ["eqo"])
    ex.add_node("shp", "Shape", ["scores"], ["sh"])
    ex.add_node("g0", "Gather", ["sh", "i0"], ["bs"])
    ex.add_node("g3", "Gather", ["sh", "i3"], ["kl"])
    ex.add_node("u0", "Unsqueeze", ["bs", "ax0"], ["bsu"])           # axes as an input (opset 13)
    ex.add_node("u3", "Unsqueeze", ["kl"], ["klu"], {"axes": [0]})   # axes as an attribute
    ex.add_node("cat", "Concat", ["bsu", "one", "one", "klu"], ["tgt"], {"axis": 0})
    ex.add_node("rs", "Reshape", ["eqo", "tgt"], ["m4"])
    ex.add_node("ex", "Expand", ["m4", "sh"], ["mx"])
    ex.add_node("wh", "Where", ["mx", "fill", "scores"], ["out"])
    return ex


def mask_ref(scores, mask):
    m4 = L.equal(mask, np.array(0, np.int64)).reshape(mask.shape[0], 1, 1, mask.shape[1])
    return L.where(L.expand(m4, scores.shape), FMIN, scores), m4


def inputs(seed, b=B, s=S):
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((b, H, s, s)).astype(np.float32)
    lens = rng.integers(1, s + 1, b)
    mask = (np.arange(s)[None, :] < lens[:, None]).astype(np.int64)
    return scores, mask


def test_attention_mask_plumbing():
    scores, mask = inputs(1)
    ex = mask_graph()
    got = ex.run({"scores": torch.from_numpy(scores).cuda(), "mask": torch.from_numpy(mask).cuda()},
                 ["out", "mx", "tgt", "sh"])
    want, m4 = mask_ref(scores, mask)
    assert got["sh"].dtype == np.int64 and got["sh"].tolist() == [B, H, S, S]
    assert got["tgt"].tolist() == [B, 1, 1, S]
    assert got["mx"].dtype == np.bool_ and np.array_equal(got["mx"], np.broadcast_to(m4, scores.shape))
    assert np.array_equal(bits(got["out"]), bits(want))
    # host-bound inputs: the Equal (int64 [B, S] = 4096 elements) is larger than what is folded
    # on the host, so it still runs on the device; same result
    got2 = ex.run({"scores": scores, "mask": mask}, ["out"])
    assert np.array_equal(bits(got2["out"]), bits(want))
    # another batch and sequence length through the same executor (shapes recomputed)
    scores3, mask3 = inputs(2, b=3, s=77)
    got3 = ex.run({"scores": torch.from_numpy(scores3).cuda(), "mask": torch.from_numpy(mask3).cuda()}, ["out"])
    assert np.array_equal(bits(got3["out"]), bits(mask_ref(scores3, mask3)[0]))


def test_attention_mask_capture_and_replay():
    data = [inputs(10 + i) for i in range(3)]
    ex = mask_graph()
    sc = torch.from_numpy(data[0][0]).cuda()
    mk = torch.from_numpy(data[0][1]).cuda()
    ex.capture({"scores": sc, "mask": mk}, ["out"])
    for rep in range(6):
        scores, mask = data[rep % 3]
        sc.copy_(torch.from_numpy(scores))
        mk.copy_(torch.from_numpy(mask))
        ex.replay()
        got = ex.outputs(["out"])["out"].cpu().numpy()
        assert np.array_equal(bits(got), bits(mask_ref(scores, mask)[0])), rep
        _ = (sc * 2.0).sum().item()
        torch.cuda.synchronize()


def test_position_ids_and_broadcast_add():
    rng = np.random.default_rng(3)
    D, P = 768, 512
    ex = GpuGraphExecutor()
    ex.add_input("ids", [None, None])
    ex.add_input("emb", [None, None, D])
    ex.add_initializer("pos_ids", np.arange(P, dtype=np.int64).reshape(1, P))
    table = rng.standard_normal((P, D)).astype(np.float32)
    ex.add_initializer("pos_table", table)
    ex.add_initializer("i1", np.array(1, np.int64))
    ex.add_initializer("z", np.array([0], np.int64))
    ex.add_initializer("ax1", np.array([1], np.int64))
    ex.add_node("shp", "Shape", ["ids"], ["sh"])
    ex.add_node("g", "Gather", ["sh", "i1"], ["slen"])
    ex.add_node("u", "Unsqueeze", ["slen", "z"], ["end"])
    ex.add_node("sl", "Slice", ["pos_ids", "z", "end", "ax1"], ["pid"])
    ex.add_node("pe", "Gather", ["pos_table", "pid"], ["pemb"])
    ex.add_node("add", "Add", ["emb", "pemb"], ["out"])
    ids = rng.integers(0, 30522, (B, S)).astype(np.int64)
    emb = rng.standard_normal((B, S, D)).astype(np.float32)
    got = ex.run({"ids": torch.from_numpy(ids).cuda(), "emb": torch.from_numpy(emb).cuda()}, ["out", "pid"])
    pid = L.slice_(np.arange(P, dtype=np.int64).reshape(1, P), [0], [S], [1])
    assert np.array_equal(got["pid"], pid)
    want = (emb + table[:S][None]).astype(np.float32)  # one f32 rounding per element
    assert np.array_equal(bits(got["out"]), bits(want))


def test_device_concat_slice_equal_cast():
    rng = np.random.default_rng(4)
    parts = [rng.standard_normal((64, n, 24)).astype(np.float32) for n in (100, 50, 7)]
    ex = GpuGraphExecutor()
    for i in range(3):
        ex.add_input("p%d" % i, [64, None, 24])
    ex.add_input("st", [3])
    ex.add_input("en", [3])
    ex.add_input("ax", [3])
    ex.add_input("sp", [3])
    ex.add_node("cat", "Concat", ["p0", "p1", "p2"], ["c"], {"axis": -2})
    ex.add_node("sl", "Slice", ["c", "st", "en", "ax", "sp"], ["s"])
    ex.add_node("eq", "Equal", ["c", "c"], ["e"])
    ex.add_node("c1", "Cast", ["e"], ["ef"], {"to": 1})
    dev = {"p%d" % i: torch.from_numpy(p).cuda() for i, p in enumerate(parts)}
    st, en, ax, sp = (np.array(v, np.int64) for v in ([150, -3, 20], [2, 0, 60], [1, 2, 0], [-3, -2, 1]))
    for k, v in (("st", st), ("en", en), ("ax", ax), ("sp", sp)):
        dev[k] = torch.from_numpy(v).cuda()  # read back to the host for the Slice bounds
    parts[1][5, 7, 3] = np.nan
    dev["p1"] = torch.from_numpy(parts[1]).cuda()
    got = ex.run(dev, ["c", "s", "e", "ef"])
    c = L.concat(parts, -2)
    assert np.array_equal(bits(got["c"]), bits(c))
    assert np.array_equal(bits(got["s"]), bits(L.slice_(c, st, en, ax, sp)))
    assert np.array_equal(got["e"], L.equal(c, c)) and not got["e"][5, 100 + 7, 3]  # NaN != NaN
    assert np.array_equal(got["ef"], L.cast(L.equal(c, c), 1))


@pytest.mark.parametrize("src,to", [("f32", 7), ("f32", 6), ("f32", 9), ("i64", 1), ("i64", 6), ("i32", 7),
                                    ("bool", 1), ("i64", 9)])
def test_device_cast(src, to):
    rng = np.random.default_rng(5)
    if src == "f32":
        x = (rng.standard_normal(5000) * 1e10).astype(np.float32)
        x[:8] = [np.nan, np.inf, -np.inf, 2.9, -2.9, 3e9, -3e9, -0.0]
    elif src == "i64":
        x = rng.integers(-2**62, 2**62, 5000, dtype=np.int64)
        x[:4] = [16777217, 16777219, 0, -1]
    elif src == "i32":
        x = rng.integers(-2**31, 2**31, 5000, dtype=np.int64).astype(np.int32)
    else:
        x = rng.integers(0, 2, 5000).astype(np.bool_)
    ex = GpuGraphExecutor()
    ex.add_input("x", [None])
    ex.add_node("c", "Cast", ["x"], ["y"], {"to": to})
    got = ex.run({"x": torch.from_numpy(x).cuda()}, ["y"])["y"]
    want = L.cast(x, to)
    assert got.dtype == want.dtype and np.array_equal(got, want)


def test_shape_read_back_while_capturing_is_an_error():
    ex = GpuGraphExecutor()
    ex.add_input("x", [None, None])
    ex.add_input("shape", [2])
    ex.add_node("rs", "Reshape", ["x", "shape"], ["y"])
    x = torch.arange(12, dtype=torch.float32, device="cuda").reshape(3, 4)
    shp = torch.tensor([2, 6], dtype=torch.int64, device="cuda")
    assert ex.run({"x": x, "shape": shp}, ["y"])["y"].shape == (2, 6)  # eager: read back
    with pytest.raises(IconnxError, match="captured"):
        ex.capture({"x": x, "shape": shp}, ["y"])
    # a host-bound shape is known without a read-back, also under capture
    ex2 = GpuGraphExecutor()
    ex2.add_input("x", [None, None])
    ex2.add_initializer("shape", np.array([2, 6], np.int64))
    ex2.add_node("rs", "Reshape", ["x", "shape"], ["y"])
    ex2.capture({"x": x}, ["y"])
    ex2.replay()
    assert ex2.outputs(["y"])["y"].shape == (2, 6)
