"""Benchmark of the int8 dynamic-quantized linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2]

A step is one pass of the hot path over one batch of synthetic, HBM-resident input.  The
default workload is BASELINE configs[1] (cfg2): x [32,128,768] f32 ->
DynamicQuantizeLinear -> MatMulInteger with W int8 [768,3072] -> Cast -> Mul(x_scale *
w_scale) -> Add(bias) -> Mul/Add/Div/Mul chain, as ONE kernel launch (icx_dql_qlinear_f32):
the GEMM's blocks compute the range of their slices of x, trade it through an exchange buffer
kept from step to step, quantize their rows and multiply once their row panel is complete.
Where that kernel does not take the shape, the DQL is its own launch
(icx_dynamic_quantize_linear_exchange) before the fused GEMM; where a GEMM needs the DQL's
row sums (cfg4's weight zero points) or the input is past that launch's limit, the DQL is
the two launches of icx_dynamic_quantize_linear (min/max, quantize).  The same run also reports the metric's second part,
encoder seq/s (cfg3: the 6-layer DistilBERT-int8-shaped encoder at batch 32, seq 128, one
captured forward replayed per step), and next to it the same encoder in the form a
DistilBERT-INT8 export writes it (Int64 ids and mask, embeddings, runtime shapes, padding mask).
--config cfg3 makes the encoder the primary line; the other configs (cfg1|cfg4|cfg5a|cfg5b)
are for the per-kernel roofline figures.

Timing: W untimed warmup steps, then exactly K steps launched back to back on one stream
(each step's host-side launch overlaps the previous step's kernels), bracketed by
synchronize; the same K steps as replays of a HIP graph holding one step are timed too and
reported beside (--graph makes those the primary figure).  The encoder (cfg3) is one
captured forward replayed per step.  The dominant kernel's average duration is measured live
with HIP events around a graph of R back-to-back launches of that kernel on the same stream.
Prints ONE JSON line.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MatMulInteger int8 TOPS (% MFMA peak); encoder seq/s, DistilBERT-int8 shape b32 s128"
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0       # MI355X dense int8 MFMA (no sparsity)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2",
                    choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5a", "cfg5b", "copy"],
                    help="copy: the chain kernel with no ops over f32[65536,768] — a plain copy "
                         "of known size, the scale for the rocprofv3 FETCH_SIZE/WRITE_SIZE counters")
    ap.add_argument("--kernel-reps", type=int, default=100,
                    help="back-to-back launches of the dominant kernel for its average duration")
    ap.add_argument("--cpu-rows", type=int, default=None,
                    help="rows of the CPU-baseline sample (default: config-specific)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time each step as the replay of a HIP graph holding that step instead of "
                         "launching it directly (the other figure is reported beside it either way)")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the steps directly (the default; kept for older command lines)")
    ap.add_argument("--no-encoder", action="store_true",
                    help="cfg2: skip the secondary encoder seq/s measurement")
    return ap.parse_args()


# ---------------------------------------------------------------------------------------
# GPU runners: buffers allocated once, C entry points called directly (no per-step alloc)
# ---------------------------------------------------------------------------------------
class Runner:
    def __init__(self, cfg):
        import numpy as np
        import torch

        from iconnx_amd import configs, ops
        from iconnx_amd._lib import ICX_I8, ICX_U8, check, lib

        self.cfg = cfg
        self.torch = torch
        self.L = lib()
        self.check = check
        d = configs.make("cfg5b" if cfg == "copy" else cfg)
        if cfg == "copy":
            d = dict(d, chain=[])
        self.d = d
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        self.keep = []
        if cfg in ("cfg1", "cfg2", "cfg4"):
            x = d["x"].reshape(-1, d["x"].shape[-1])
            self.M, self.K = x.shape
            self.N = d["w"].shape[1]
            self.x = dev(x)
            self.w = ops.PackedWeight(dev(d["w"]))
            # A weight zero point is an initializer: when it is all zeros (and the weight is
            # int8) its row term is multiplied by exactly 0, so it is folded away at plan time,
            # as the executor does (the kernel then needs no row sums).
            self.w_zp = None if not np.any(d["w_zp"]) else dev(d["w_zp"])
            self.bzp_len = int(np.asarray(d["w_zp"]).size)
            self.xq = torch.empty((self.M, self.K), dtype=torch.uint8, device="cuda")
            self.xs = torch.empty((), dtype=torch.float32, device="cuda")
            self.xzp = torch.empty((), dtype=torch.uint8, device="cuda")
            self.rs = torch.empty(self.M, dtype=torch.int32, device="cuda")
            self.y = torch.empty((self.M, self.N), dtype=torch.float32, device="cuda")
            self.dql_ws = torch.empty(self.L.icx_dql_workspace_size(self.x.numel()), dtype=torch.uint8, device="cuda")
            # the single-launch DQL's exchange buffer: zeroed once, kept for every later call
            self.sync = torch.zeros(self.L.icx_exchange_buffer_size(), dtype=torch.uint8, device="cuda")
            self.dql_launches = 2
            if self.w_zp is None:  # no row sums wanted: try the single launch once, eagerly
                from iconnx_amd._lib import ICX_ERR_UNSUPPORTED
                h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                rc = self.L.icx_dynamic_quantize_linear_exchange(
                    h, self._p(self.x), self.x.numel(), self._p(self.xq), self._p(self.xs), self._p(self.xzp),
                    self._p(self.sync))
                if rc == 0:
                    self.check(self.L.icx_exchange_status(h, self._p(self.sync)))
                    self.dql_launches = 1
                elif rc != ICX_ERR_UNSUPPORTED:
                    self.check(rc)
            self.gemm_ws = torch.empty(max(1, self.L.icx_matmul_integer_workspace_size(self.M, self.K, self.N, 1)),
                                       dtype=torch.uint8, device="cuda")
            epi = [("Mul", (self.xs, dev(d["w_scale"])), False), ("Add", dev(d["bias"]), False)]
            epi += [(op, dev(c), False) for op, c in d["chain"]]
            self.chain, k = ops.build_chain(epi, self.M, self.N)
            self.keep += k
            # the DQL and the quantized linear as one launch where the fused kernel takes the
            # shape (cfg2): tried once, eagerly
            self.fused = False
            if self.w_zp is None and self.dql_launches == 1:
                from iconnx_amd._lib import ICX_ERR_UNSUPPORTED
                h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                self.y = torch.empty((self.M, self.N), dtype=torch.float32, device="cuda")
                rc = self.L.icx_dql_qlinear_f32(
                    h, self._p(self.x), self.M, self.K, self._p(self.xq), self._p(self.xs), self._p(self.xzp),
                    self._p(self.w.packed), ICX_I8, self._p(self.w.colsum), self.N, ctypes.byref(self.chain),
                    self._p(self.y), self._p(self.sync))
                if rc == 0:
                    self.check(self.L.icx_exchange_status(h, self._p(self.sync)))
                    self.fused = True
                elif rc != ICX_ERR_UNSUPPORTED:
                    self.check(rc)
            self.a_dtype, self.b_dtype = ICX_U8, ICX_I8
            self.ops_count = 2.0 * self.M * self.N * self.K
            # cfg2 (256x192 tiles) and cfg4 (256x256) take the 128-byte-row kernel, cfg1 the
            # 64x64-tile one
            self.dominant = "gemm_i8_dma128_kernel" if cfg in ("cfg2", "cfg4") else "gemm_i8_dma_kernel"
            if self.fused:
                self.dominant = "gemm_i8_dma128_kernel (DQL + GEMM + epilogue, one launch)"
        elif cfg == "cfg5a":
            self.M, self.K = d["a"].shape
            self.N = d["b"].shape[1]
            self.a = dev(d["a"])
            self.a_zp = dev(d["a_zp"])
            self.w = ops.PackedWeight(dev(d["b"]))
            self.w_zp = None if not np.any(d["b_zp"]) else dev(d["b_zp"])  # folded when all-zero
            self.bzp_len = 1
            self.y = torch.empty((self.M, self.N), dtype=torch.float32, device="cuda")
            self.gemm_ws = torch.empty(max(1, self.L.icx_matmul_integer_workspace_size(self.M, self.K, self.N, 1)),
                                       dtype=torch.uint8, device="cuda")
            self.chain, k = ops.build_chain([("Mul", (dev(d["a_scale"]), dev(d["b_scale"])), False)],
                                            self.M, self.N)
            self.keep += k
            self.a_dtype, self.b_dtype = ICX_U8, ICX_I8
            self.ops_count = 2.0 * self.M * self.N * self.K
            self.dominant = "gemm_i8_dma128_kernel"
        else:  # cfg5b, copy
            self.x = dev(d["x"])
            self.M, self.N = d["x"].shape
            self.y = torch.empty_like(self.x)
            chain = [] if cfg == "copy" else [(op, dev(c), False) for op, c in d["chain"]]
            self.chain, k = ops.build_chain(chain, self.M, self.N)
            self.keep += k
            self.ops_count = None
            self.dominant = "chain_cols_kernel"
        torch.cuda.synchronize()

    def _p(self, t):
        return ctypes.c_void_p(t.data_ptr())

    def dql(self, stream):
        if self.dql_launches == 1:
            self.check(self.L.icx_dynamic_quantize_linear_exchange(
                stream, self._p(self.x), self.x.numel(), self._p(self.xq), self._p(self.xs),
                self._p(self.xzp), self._p(self.sync)))
            return
        self.check(self.L.icx_dynamic_quantize_linear(
            stream, self._p(self.x), self.x.numel(), self._p(self.xq), self._p(self.xs),
            self._p(self.xzp), self._p(self.rs) if self.w_zp is not None else None, self.K,
            self._p(self.dql_ws), self.dql_ws.numel()))

    def gemm(self, stream):
        if self.cfg == "cfg5a":
            a, azp, rs = self.a, self.a_zp, None
        else:
            a, azp, rs = self.xq, self.xzp, self.rs
        self.check(self.L.icx_qlinear_f32(
            stream, self._p(a), self.a_dtype, self._p(self.w.packed), self.b_dtype, 1,
            self._p(self.w.colsum), self.M, self.K, self.N, self._p(azp),
            self._p(self.w_zp) if self.w_zp is not None else None,
            self.bzp_len, self._p(rs) if (rs is not None and self.w_zp is not None) else None,
            ctypes.byref(self.chain),
            self._p(self.y), self._p(self.gemm_ws), self.gemm_ws.numel()))

    def dql_gemm(self, stream):
        self.check(self.L.icx_dql_qlinear_f32(
            stream, self._p(self.x), self.M, self.K, self._p(self.xq), self._p(self.xs), self._p(self.xzp),
            self._p(self.w.packed), self.b_dtype, self._p(self.w.colsum), self.N, ctypes.byref(self.chain),
            self._p(self.y), self._p(self.sync)))

    def chain_only(self, stream):
        self.check(self.L.icx_fused_chain_f32(stream, self._p(self.x), self.M, self.N,
                                              ctypes.byref(self.chain), self._p(self.y)))

    def step(self, stream):
        if self.cfg in ("cfg5b", "copy"):
            self.chain_only(stream)
        elif self.cfg == "cfg5a":
            self.gemm(stream)
        elif getattr(self, "fused", False):
            self.dql_gemm(stream)
        else:
            self.dql(stream)
            self.gemm(stream)

    def dominant_launch(self, stream):
        if self.cfg in ("cfg5b", "copy"):
            self.chain_only(stream)
        elif getattr(self, "fused", False):
            self.dql_gemm(stream)
        else:
            self.gemm(stream)

    def algorithmic_bytes(self):
        """HBM bytes one launch of the dominant kernel must move at minimum."""
        import numpy as np

        M, N = self.M, self.N
        if self.cfg in ("cfg5b", "copy"):
            return 8.0 * M * N + sum(4.0 * N for _ in self.d["chain"])
        K = self.K
        b = M * K + K * N + 4.0 * M * N  # A u8, packed B i8, Y f32
        if getattr(self, "fused", False):
            b += 4.0 * M * K  # the launch also reads x f32 (and writes A, counted once above)
        b += 4.0 * N  # colsum
        if self.cfg != "cfg5a":
            b += 4.0 * M  # row sums from DQL
            b += 4.0 * N * (1 + len(self.d["chain"])) + 4.0 * N * (self.bzp_len > 1)  # bias, chain, per-col zp
            b += 4.0 * N if np.size(self.d["w_scale"]) > 1 else 0
        return b


class EncoderRunner:
    """cfg3: the DistilBERT-int8-shaped encoder (6 layers, hidden 768, 12 heads, FFN 3072)
    through GpuGraphExecutor with random-init weights, input [32, 128, 768] ~ N(0, 1) on the
    device; one forward is recorded once (icx_graph_capture) and a step is one replay."""

    def __init__(self):
        import torch

        from iconnx_amd import graphs
        from iconnx_amd.executor import GpuGraphExecutor

        cfg = graphs.ENCODER
        self.B, self.S = cfg["batch"], cfg["seq"]
        self.ex = GpuGraphExecutor()
        self.out, _, self.params = graphs.encoder_graph(self.ex, layers=cfg["layers"], heads=cfg["heads"])
        self.x = torch.from_numpy(graphs.encoder_input(self.B, self.S)).cuda()
        self.ex.capture({"x": self.x}, [self.out])
        torch.cuda.synchronize()
        # int8 work of one forward: 4 x (M x 768 x 768) + 2 x (M x 768 x 3072) per layer
        M = self.B * self.S
        self.int8_ops = cfg["layers"] * 2.0 * M * (4 * 768 * 768 + 2 * 768 * 3072)

    def step(self):
        self.ex.replay()


class ExportEncoderRunner:
    """The same encoder in the form a DistilBERT-INT8 export writes it (graphs.
    export_encoder_graph): Int64 input_ids / attention_mask [32, 128] (seeded lengths, one row
    unpadded), the UINT8 word-embedding lookup, position embeddings, runtime reshape targets,
    the padding mask and node-by-node LayerNorms; one forward captured, a step is one replay."""

    def __init__(self):
        import torch

        from iconnx_amd import graphs
        from iconnx_amd.executor import GpuGraphExecutor

        cfg = graphs.ENCODER
        self.B, self.S = cfg["batch"], cfg["seq"]
        self.ex = GpuGraphExecutor()
        self.out, _, _, _ = graphs.export_encoder_graph(self.ex, layers=cfg["layers"], heads=cfg["heads"])
        ids, mask = graphs.export_inputs(self.B, self.S)
        self.feeds = {"input_ids": torch.from_numpy(ids).cuda(), "attention_mask": torch.from_numpy(mask).cuda()}
        self.ex.capture(self.feeds, [self.out])
        torch.cuda.synchronize()

    def step(self):
        self.ex.replay()


def export_form_line(torch):
    """seq/s of the exported form (a reported extra next to the encoder line)."""
    exp = ExportEncoderRunner()
    ms, _ = time_replays(exp.step, 50, 5, torch)
    exp.ex.check_status()
    return {"metric": "encoder seq/s, exported form", "value": round(exp.B / (ms * 1e-3), 1), "unit": "seq/s",
            "ms_per_forward": round(ms, 4), "workload": EXPORT_WORKLOAD, "graph_replay": True}


class FfnUpGeluRunner:
    """The encoder's largest kernel on its own: the FFN-up quantized linear (x [4096, 768]
    -> [4096, 3072]) with the dequant, bias and erf-GELU in the GEMM store."""

    def __init__(self, params):
        import numpy as np
        import torch

        from iconnx_amd import graphs, ops
        from iconnx_amd._lib import ICX_I8, ICX_U8, check, lib

        self.L, self.check, self.torch = lib(), check, torch
        p = params["ff1"]
        x = graphs.encoder_input(32, 128).reshape(-1, 768)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        self.M, self.K, self.N = 4096, 768, 3072
        self.xq, xs, self.xzp = ops.gpu_dynamic_quantize_linear(dev(x))
        self.w = ops.PackedWeight(dev(p["w"]))
        c = [dev(np.array(v, np.float32)) for v in (1.4142135381698608, 1.0, 0.5)]
        epi = [("Mul", (xs, dev(p["w_scale"])), False), ("Add", dev(p["bias"]), False),
               ("Save", None, False), ("Div", c[0], False), ("Erf", None, False),
               ("Add", c[1], False), ("MulSaved", None, False), ("Mul", c[2], False)]
        self.chain, self.keep = ops.build_chain(epi, self.M, self.N)
        self.y = torch.empty((self.M, self.N), dtype=torch.float32, device="cuda")
        self.ws = torch.empty(max(1, self.L.icx_matmul_integer_workspace_size(self.M, self.K, self.N, 1)),
                              dtype=torch.uint8, device="cuda")
        self.a_dtype, self.b_dtype = ICX_U8, ICX_I8
        torch.cuda.synchronize()

    def launch(self, stream):
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.check(self.L.icx_qlinear_f32(
            stream, p(self.xq), self.a_dtype, p(self.w.packed), self.b_dtype, 1, p(self.w.colsum),
            self.M, self.K, self.N, p(self.xzp), None, 1, None, ctypes.byref(self.chain), p(self.y),
            p(self.ws), self.ws.numel()))

    def algorithmic_bytes(self):
        return self.M * self.K + self.K * self.N + 4.0 * self.M * self.N + 4.0 * self.N * 2


def time_replays(step, steps, warmup, torch):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, time.perf_counter() - t0


def host_info():
    """The CPU the baseline ran on: logical CPUs this process may use (nproc) and the model
    name from /proc/cpuinfo (what lscpu prints as 'Model name')."""
    try:
        cores = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cores = os.cpu_count()
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cores": cores, "cpu_model": model, "threads_used": 1}


def encoder_cpu_baseline():
    """The oracle (single-threaded C restatement of the reference CPU ops, composed op by op)
    running the same 6-layer encoder on one sequence [1, 128, 768] — a bounded sample of the
    batch-32 workload (per-tensor quantization then spans that sequence only)."""
    import numpy as npx

    from iconnx_amd import graphs
    from oracle.encoder import layer_ref

    cfg = graphs.ENCODER
    x = graphs.encoder_input(1, cfg["seq"])
    params = [graphs.encoder_layer_params(l) for l in range(cfg["layers"])]
    t0 = time.perf_counter()
    for l in range(cfg["layers"]):
        x = layer_ref(x, params[l], cfg["heads"], cfg["eps"])["out"]
    dt = time.perf_counter() - t0
    assert npx.all(npx.isfinite(x))
    return {"value": round(1.0 / dt, 4), "unit": "seq/s", "cores": 1, "kind": "port",
            "sample": "one sequence [1,128,768] through the 6 layers op by op (%.1f s measured)" % dt,
            **host_info()}


def measured_traffic(cfg):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the plain-copy calibration), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_hbm_pmc.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and parts[0] == "traffic" and parts[1] == cfg:
                return float(parts[5])
    return None


def graph_of(fn, reps, torch):
    """Capture `reps` calls of fn(stream) into one HIP graph (default-priority stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(ctypes.c_void_p(s.cuda_stream))  # warm the path on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(reps):
            fn(h)
    torch.cuda.synchronize()
    return g


# ---------------------------------------------------------------------------------------
# CPU baseline: the oracle (single-threaded C restatement of the reference CPU ops)
# ---------------------------------------------------------------------------------------
def cpu_baseline(cfg, rows_arg):
    import numpy as npx

    import oracle
    from iconnx_amd import configs

    d = configs.make(cfg)
    t = {}
    if cfg == "cfg5b":
        rows = rows_arg or 16384
        x = d["x"][:rows]
        t0 = time.perf_counter()
        y = x
        for op, c in d["chain"]:
            y = {"Mul": oracle.mul, "Add": oracle.add, "Div": oracle.div}[op](y, c)
        dt = time.perf_counter() - t0
        full = dt * d["x"].shape[0] / rows
        gbs = 8.0 * d["x"].size / full / 1e9
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": "Mul/Add/Div/Mul op by op on rows [0,%d) of 65536, extrapolated linearly"
                          " in rows (%.2f s measured)" % (rows, dt)}
    if cfg == "cfg5a":
        rows = rows_arg or 16
        a, b = d["a"], d["b"]
        M, K = a.shape
        N = b.shape[1]
        t0 = time.perf_counter()
        acc = oracle.matmul_integer(a[:rows], b, d["a_zp"], d["b_zp"])
        t["MatMulInteger"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        s = oracle.mul(d["a_scale"], d["b_scale"])
        oracle.mul(oracle.cast_i32_f32(acc), s)
        t["Cast+Mul"] = time.perf_counter() - t0
        full = sum(t.values()) * M / rows
        return {"value": round(2.0 * M * N * K / full / 1e12, 6), "unit": "TOPS", "cores": 1,
                "kind": "port", "per_op_s": {k: round(v * M / rows, 3) for k, v in t.items()},
                "sample": "MatMulInteger + Cast + Mul on rows [0,%d) of %d, extrapolated linearly "
                          "in M (%.2f s measured)" % (rows, M, sum(t.values()))}
    rows = rows_arg or {"cfg1": 128, "cfg2": 1024, "cfg4": 192}[cfg]
    x = d["x"].reshape(-1, d["x"].shape[-1])
    M, K = x.shape
    N = d["w"].shape[1]
    rows = min(rows, M)
    t0 = time.perf_counter()
    xq, xs, xzp = oracle.dynamic_quantize_linear(x)  # needs the whole tensor (global min/max)
    t_dql = time.perf_counter() - t0
    per_col = npx.asarray(d["w_zp"]).ndim == 1
    t0 = time.perf_counter()
    acc = oracle.matmul_integer(xq[:rows], d["w"], xzp, d["w_zp"], per_column_b_zp=per_col)
    t["MatMulInteger"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    c = oracle.cast_i32_f32(acc)
    t["Cast"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    s = oracle.mul(xs, d["w_scale"])
    y = oracle.mul(c, s)
    t["Mul"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    y = oracle.add(y, d["bias"])
    t["Add"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    for op, cc in d["chain"]:
        y = {"Mul": oracle.mul, "Add": oracle.add, "Div": oracle.div}[op](y, cc)
    if d["chain"]:
        t["chain"] = time.perf_counter() - t0
    scale = M / rows
    per_op = {"DynamicQuantizeLinear": round(t_dql, 4)}
    per_op.update({k: round(v * scale, 3) for k, v in t.items()})
    full = t_dql + sum(t.values()) * scale
    return {"value": round(2.0 * M * N * K / full / 1e12, 6), "unit": "TOPS", "cores": 1,
            "kind": "port", "per_op_s": per_op,
            "sample": "DynamicQuantizeLinear on all %d rows; MatMulInteger + epilogue on rows [0,%d),"
                      " extrapolated linearly in M (%.2f s measured)" % (M, rows, t_dql + sum(t.values()))}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); --gpus %d is not "
              "supported" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch

    torch.cuda.set_device(0)
    if args.config == "cfg3":
        return main_encoder(args, torch)
    r = Runner(args.config)
    sync = torch.cuda.synchronize

    # ---- timed steps -------------------------------------------------------------------
    # Steps are launched directly, back to back on one stream: each is one call of the C
    # entry points (one kernel for cfg2), whose host-side launch overlaps the previous step's
    # kernel.  The same K steps as replays of a HIP graph holding one step are timed too and
    # reported beside (a graph launch per step leaves the GPU idle ~6 us between steps).
    eager = lambda: r.step(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))  # noqa: E731
    g_step = graph_of(r.step, 1, torch)

    def timed(run_step):
        for _ in range(args.warmup):
            run_step()
        sync()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record()
        for _ in range(args.steps):
            run_step()
        ev1.record()
        sync()
        return ev0.elapsed_time(ev1) / args.steps, time.perf_counter() - t0

    use_graph = args.graph and not args.no_graph
    ms_step, wall = timed(g_step.replay if use_graph else eager)
    ms_other, _ = timed(eager if use_graph else g_step.replay)

    # ---- dominant kernel: average launch duration over R back-to-back launches --------
    reps = args.kernel_reps
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def time_launches(fn):
        """Average duration of `reps` back-to-back launches of fn on the current stream."""
        g = graph_of(fn, reps, torch)
        g.replay()
        sync()
        k0.record()
        g.replay()
        k1.record()
        sync()
        return k0.elapsed_time(k1) * 1e3 / reps

    k_us = time_launches(r.dominant_launch)

    # the DQL on its own, for the breakdown
    extra = {}
    if args.config in ("cfg1", "cfg2", "cfg4"):
        dql_us = time_launches(r.dql)
        n = r.x.numel()
        # a single-launch DQL whose blocks gave up waiting (not all resident) wrote y = 0:
        # the timed steps would then be invalid, so that raises here
        r.check(r.L.icx_exchange_status(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                        r._p(r.sync)))
        extra["dql_launches"] = 0 if r.fused else r.dql_launches
        extra["launches_per_step"] = 1 if r.fused else r.dql_launches + 1
        extra["dql_us"] = round(dql_us, 3)
        extra["dql_algorithmic_GBps"] = round(5.0 * n / (dql_us * 1e-6) / 1e9, 1)
        if r.fused:
            extra["dql_us_standalone"] = extra.pop("dql_us")

    alg_bytes = r.algorithmic_bytes()
    if r.ops_count is not None:
        value = r.ops_count / (ms_step * 1e-3) / 1e12
        unit = "TOPS"
    else:
        value = 8.0 * r.M * r.N / (ms_step * 1e-3) / 1e9
        unit = "GB/s"
    if args.config == "cfg5a":
        ach = r.ops_count / (k_us * 1e-6) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS,
                "unit": "TFLOP/s", "op_kind": "int8 ops (2*M*N*K)", "frac": round(ach / PEAK_INT8_TOPS, 4),
                "traffic": measured_traffic(args.config), "kernel": r.dominant,
                "kernel_avg_us": round(k_us, 3), "algorithmic_bytes": alg_bytes}
    else:
        ach = alg_bytes / (k_us * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": measured_traffic(args.config),
                "kernel": r.dominant,
                "kernel_avg_us": round(k_us, 3), "algorithmic_bytes": alg_bytes}
        if r.ops_count is not None:
            roof["kernel_int8_TOPS"] = round(r.ops_count / (k_us * 1e-6) / 1e12, 2)
    mfma = None
    if r.ops_count is not None:  # the metric's "% MFMA peak": step and dominant kernel
        k_tops = r.ops_count / (k_us * 1e-6) / 1e12
        mfma = {"peak_TOPS": PEAK_INT8_TOPS, "step_TOPS": round(value, 2),
                "step_frac": round(value / PEAK_INT8_TOPS, 4), "kernel_TOPS": round(k_tops, 2),
                "kernel_frac": round(k_tops / PEAK_INT8_TOPS, 4)}

    workload = {
        "cfg1": "cfg1: DQL + quantized linear x[1,128,768] W[768,768] + bias",
        "cfg2": "cfg2: DQL + MatMulInteger + dequant Mul + bias Add + Mul/Add/Div/Mul chain, "
                "x[32,128,768] W[768,3072] (DistilBERT-int8 FFN-up shape, b32 s128)",
        "cfg4": "cfg4: DQL + per-channel quantized linear x[64,384,1024] W[1024,4096]",
        "cfg5a": "cfg5a: MatMulInteger A u8[16384,4096] x B i8[4096,4096] + fused fp32 dequant",
        "cfg5b": "cfg5b: fused Mul/Add/Div/Mul chain on f32[65536,768] with [768] operands",
        "copy": "copy calibration: chain kernel with no ops (plain copy) on f32[65536,768]",
    }[args.config]
    cfg = {"workload": workload, "M": r.M, "N": r.N}
    if hasattr(r, "K"):
        cfg["K"] = r.K
    out = {
        "metric": METRIC, "value": round(value, 4), "unit": unit, "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded N(0,1) activations (SplitMix64 + Box-Muller), random-init int8 weights",
        "config": cfg, "roofline": roof,
        "timing": {"launch": "graph replay per step" if use_graph else "direct, back to back",
                   "wall_s": round(wall, 4),
                   ("direct_ms_per_step" if use_graph else "graph_replay_ms_per_step"): round(ms_other, 6),
                   **extra},
        **({"mfma": mfma} if mfma else {}),
        "traffic_source": "profiles/traffic_hbm_pmc.txt (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)",
    }
    if args.config in ("cfg5b", "copy"):
        out["dtype"] = "f32"
    if args.config == "cfg2" and not args.no_encoder:
        # the metric's second part, encoder seq/s, measured in the same run
        enc = EncoderRunner()
        ms_e, _ = time_replays(enc.step, 50, 5, torch)
        enc.ex.check_status()  # a quantized-output launch that failed on the device raises
        e_tops = enc.int8_ops / (ms_e * 1e-3) / 1e12
        out["encoder"] = {"metric": "encoder seq/s", "value": round(enc.B / (ms_e * 1e-3), 1),
                          "unit": "seq/s", "ms_per_forward": round(ms_e, 4),
                          "int8_TOPS": round(e_tops, 2), "int8_frac_of_mfma_peak": round(e_tops / PEAK_INT8_TOPS, 4),
                          "workload": ENCODER_WORKLOAD, "graph_replay": True}
        out["encoder"]["export_form"] = export_form_line(torch)
        if not args.no_cpu_baseline:
            out["encoder"]["cpu_baseline"] = encoder_cpu_baseline()
    if not args.no_cpu_baseline and args.config != "copy":
        cb = cpu_baseline(args.config, args.cpu_rows)
        cb["cores"] = 1
        cb.update(host_info())
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


ENCODER_WORKLOAD = ("cfg3: 6-layer DistilBERT-int8-shaped encoder, hidden 768, 12 heads, FFN 3072, "
                    "batch 32, seq 128; every linear DQL + MatMulInteger + dequant Mul + bias Add, "
                    "LayerNorm / Softmax / erf-GELU in fp32")
EXPORT_WORKLOAD = ("cfg3 as a DistilBERT-INT8 export writes it: Int64 input_ids / attention_mask [32, 128], "
                   "UINT8 word-embedding Gather + DequantizeLinear, position embeddings, reshape targets from "
                   "Shape / Gather / Unsqueeze / Concat, padding mask Equal / Reshape / Expand / Where, "
                   "node-by-node LayerNorms (embeddings and mask included in the forward)")


def main_encoder(args, torch):
    enc = EncoderRunner()
    ms_step, wall = time_replays(enc.step, args.steps, args.warmup, torch)
    enc.ex.check_status()
    seq_s = enc.B / (ms_step * 1e-3)
    # dominant kernel: the FFN-up GEMM with its erf-GELU epilogue, R launches in one graph
    ffn = FfnUpGeluRunner(enc.params[0])
    g = graph_of(ffn.launch, args.kernel_reps, torch)
    g.replay()
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record()
    g.replay()
    k1.record()
    torch.cuda.synchronize()
    k_us = k0.elapsed_time(k1) * 1e3 / args.kernel_reps
    alg = ffn.algorithmic_bytes()
    ach = alg / (k_us * 1e-6) / 1e9
    out = {
        "metric": METRIC, "value": round(seq_s, 2), "unit": "seq/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: input embeddings ~ N(0,1) (SplitMix64 + Box-Muller), random-init int8 "
                "weights (per-tensor scale), N(0,0.02) biases",
        "config": {"workload": ENCODER_WORKLOAD, "batch": enc.B, "seq": enc.S, "layers": 6},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "gemm_i8_dma128_kernel<256,192> (FFN-up 4096x768x3072, erf-GELU epilogue, "
                               "f32 output; inside the encoder it runs in its quantized-output form)",
                     "kernel_avg_us": round(k_us, 3), "algorithmic_bytes": alg,
                     "kernel_int8_TOPS": round(2.0 * ffn.M * ffn.N * ffn.K / (k_us * 1e-6) / 1e12, 2)},
        "timing": {"graph_replay": True, "wall_s": round(wall, 4),
                   "encoder_int8_TOPS": round(enc.int8_ops / (ms_step * 1e-3) / 1e12, 2)},
        "export_form": export_form_line(torch),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = encoder_cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
