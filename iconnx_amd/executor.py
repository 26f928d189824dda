"""GpuGraphExecutor over the C ABI graph executor (``icx_graph_*`` in include/iconnx_hip.h).

Mirrors the reference's shim (src/cuda/inference/mod.rs:208-659): ``add_input`` (:306),
``add_initializer`` (:317), ``add_node`` (:331), ``compile`` (:487), ``run`` (:428) with the
input-shape guard (:441-460) and ``pool_stats`` (:381).  Lowering, fusion, weight packing,
the memory pool and per-op dispatch all live in the native library
(iconnx_amd/csrc/executor.cpp); this class only marshals names, host arrays and torch
device tensors across the boundary.

Differences from the reference that a caller can see:
  * only the ops of the quantized-linear path and the encoder around it dispatch
    (DynamicQuantizeLinear, MatMulInteger, DequantizeLinear, Cast to FLOAT, Mul/Add/Sub/Div,
    LayerNormalization, ReduceMean, Pow, Sqrt, Softmax, Erf, Transpose, Reshape, Gather,
    f32 MatMul); any other op raises IconnxError at run naming the node;
  * ``MatMulInteger -> Cast -> Mul(scale) [-> Add(bias)] [-> chain] [-> erf-GELU]`` runs as
    one fused GEMM (pattern ``QuantizedLinear``), a BERT self-attention subgraph as one
    kernel (``Attention``), ``LayerNormalization(Add(a, b))`` as one (``AddLayerNorm``) and
    the node-by-node LayerNorm ``ReduceMean -> Sub -> Pow -> ReduceMean -> Add -> Sqrt ->
    Div [-> Mul -> Add]`` as the same kernel (``DecomposedLayerNorm``); the reference leaves
    these unfused (it fuses only the Add -> Sqrt -> Div tail, ``DivRsqrt``);
  * ``run_device`` returns device tensors without the host round trip.
"""
import ctypes
from collections import namedtuple

import numpy as np

from ._lib import ICX_BOOL, ICX_F32, ICX_I8, ICX_I32, ICX_I64, ICX_U8, IconnxError, OpProfile, check, lib

_NP_DT = {np.dtype(np.int8): ICX_I8, np.dtype(np.uint8): ICX_U8,
          np.dtype(np.int32): ICX_I32, np.dtype(np.float32): ICX_F32,
          np.dtype(np.int64): ICX_I64, np.dtype(np.bool_): ICX_BOOL}
_INIT_DT = {**_NP_DT, np.dtype(np.int64): ICX_I64}
_DT_NP = {v: k for k, v in _NP_DT.items()}

# group: for a quantized linear run as one launch with its siblings, the lead's node name
PlanEntry = namedtuple("PlanEntry", "node op_type kind pattern steps out wzp_folded group",
                       defaults=(None,))


def _torch():
    import torch
    return torch


def _torch_dt(code):
    torch = _torch()
    return {ICX_I8: torch.int8, ICX_U8: torch.uint8, ICX_I32: torch.int32,
            ICX_F32: torch.float32, ICX_I64: torch.int64, ICX_BOOL: torch.bool}[code]


def _dims(shape):
    arr = (ctypes.c_int64 * max(len(shape), 1))(*[int(d) for d in shape])
    return arr


def _cstrs(names):
    arr = (ctypes.c_char_p * max(len(names), 1))(*[n.encode() for n in names])
    return arr


_hip = None


def _hip_memcpy_d2d(dst, src, nbytes, stream):
    """hipMemcpyAsync device-to-device on `stream` (the HIP runtime torch already loaded)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                        ctypes.c_int, ctypes.c_void_p]
        _hip.hipMemcpyAsync.restype = ctypes.c_int
    rc = _hip.hipMemcpyAsync(dst, src, nbytes, 3, stream)  # 3 = hipMemcpyDeviceToDevice
    if rc != 0:
        raise IconnxError(5, "hipMemcpyAsync of an output failed (hipError %d)" % rc)


class ProfileData:
    """Result of :meth:`GpuGraphExecutor.run_with_profiling` — the reference's ProfileData
    (src/cuda/inference/mod.rs:89-164).  Times are microseconds, as floats (the reference
    truncates to whole microseconds, which rounds short kernels to 0).

    * ``gpu_op_times`` {label: (us, calls)}: device time between the hipEvents that bracket
      each op on the stream;
    * ``op_times`` {label: (us, calls)}: host time to validate and enqueue each op;
    * ``ops``: (node, label, gpu_us, cpu_us) per executed op, in execution order;
    * ``input_upload_us`` (device time of the input copies), ``node_execution_us`` (host
      enqueue time of all ops), ``output_download_us``, ``total_us``."""

    def __init__(self):
        self.input_upload_us = self.node_execution_us = 0.0
        self.output_download_us = self.total_us = 0.0
        self.op_times, self.gpu_op_times, self.ops = {}, {}, []

    def summary(self, top=15):
        """The reference's print_summary as a string: the labels by GPU time."""
        lines = ["=== GPU Inference Profile ===",
                 "  Input upload:     %10.1f us" % self.input_upload_us,
                 "  Node execution:   %10.1f us (host enqueue)" % self.node_execution_us,
                 "  Output download:  %10.1f us" % self.output_download_us,
                 "  TOTAL:            %10.1f us" % self.total_us,
                 "=== Top Operators by GPU-Side Time (HIP events) ==="]
        for label, (us, calls) in sorted(self.gpu_op_times.items(), key=lambda kv: -kv[1][0])[:top]:
            cpu = self.op_times.get(label, (0.0, 0))[0]
            lines.append("  %-28s gpu=%10.1f us cpu=%9.1f us (%4d calls, %8.2f us/call)"
                         % (label, us, cpu, calls, us / max(calls, 1)))
        return "\n".join(lines)


def constant_value(node):
    """The static tensor of a promotable ``Constant`` node (one non-empty output), else None:
    the ``value`` tensor, else ``value_int`` / ``value_ints`` as Int64, ``value_float`` /
    ``value_floats`` as Float32 (src/attributes.rs:103-133)."""
    if node.op_type != "Constant" or len(node.outputs) != 1 or not node.outputs[0]:
        return None
    a = node.attributes
    if isinstance(a.get("value"), np.ndarray):
        return a["value"]
    if isinstance(a.get("value_int"), (int, np.integer)):
        return np.array(a["value_int"], np.int64)
    if isinstance(a.get("value_ints"), list):
        return np.array(a["value_ints"], np.int64).reshape(-1)
    if isinstance(a.get("value_float"), (float, np.floating)):
        return np.array(a["value_float"], np.float32)
    if isinstance(a.get("value_floats"), list):
        return np.array(a["value_floats"], np.float32).reshape(-1)
    return None


class GpuGraphExecutor:
    """Build a graph, then ``run`` it on the GPU (one executor per thread, as in the
    reference)."""

    def __init__(self):
        self._L = lib()
        self._g = self._L.icx_graph_create()
        if not self._g:
            raise IconnxError(1, "icx_graph_create failed")
        self._outputs = []
        self._keep = []  # device inputs bound in place, alive until the next run
        self._n_nodes = 0

    def __del__(self):
        g, self._g = getattr(self, "_g", None), None
        if g:
            self._L.icx_graph_destroy(g)

    # ---- construction -------------------------------------------------------------------
    @classmethod
    def from_model(cls, model):
        """Seed inputs, initializers and nodes from a parsed model
        (src/cuda/inference/mod.rs:250-271): node names are synthesised as ``n{i}``.  A
        ``Constant`` node with one output and a static value becomes an initializer of that
        name, as the reference's constant-promotion pass does
        (src/ir/passes/constant_promotion.rs:1-160, values resolved as
        src/attributes.rs:103-133): exporters write the exponent and epsilon of a
        node-by-node LayerNorm that way."""
        exec_ = cls()
        for name, shape in model.input_shapes():
            exec_.add_input(name, shape)
        for name, arr in model.extract_weights().items():
            exec_.add_initializer(name, arr)
        for i, node in enumerate(model.computation_graph()):
            value = constant_value(node)
            if value is not None:
                exec_.add_initializer(node.outputs[0], value)
                continue
            exec_.add_node("n%d" % i, node.op_type, node.inputs, node.outputs, node.attributes)
        return exec_

    def add_input(self, name, shape, elem_type=None):
        """``shape[i] is None`` marks a dynamic dimension.  ``elem_type`` (an ONNX element
        type, as a model file declares it) is accepted for the builders' sake and not
        needed: the dtype comes with the tensor bound at run."""
        dims = [-1 if d is None else int(d) for d in shape]
        check(self._L.icx_graph_add_input(self._g, name.encode(), len(dims), _dims(dims)))

    def add_initializer(self, name, tensor):
        """Host array (numpy or CPU torch).  Int8 / UInt8 / Int32 / Float32 / Int64 / Bool
        are kept (small integer ones are also read on the host as shape constants); other
        dtypes are skipped, so a node reading one fails at run (as the reference does)."""
        arr = tensor.numpy() if hasattr(tensor, "numpy") and not isinstance(tensor, np.ndarray) \
            else np.asarray(tensor)
        code = _INIT_DT.get(arr.dtype)
        if code is None:
            return
        if not arr.flags.c_contiguous:  # (np.ascontiguousarray would make a 0-d array 1-d)
            arr = arr.copy(order="C")
        check(self._L.icx_graph_add_initializer(
            self._g, name.encode(), code, arr.ndim, _dims(arr.shape),
            arr.ctypes.data_as(ctypes.c_void_p)))

    def add_node(self, name, op_type, inputs, outputs, attributes=None):
        """Attributes: ints (``to``, ``axis``), floats (``epsilon``) and int lists
        (``perm``); others are not read by any op here and are ignored."""
        attributes = attributes or {}
        attrs = {k: int(v) for k, v in attributes.items()
                 if isinstance(v, (int, np.integer)) and not isinstance(v, bool)}
        keys = list(attrs)
        vals = (ctypes.c_int64 * max(len(keys), 1))(*[attrs[k] for k in keys])
        check(self._L.icx_graph_add_node(
            self._g, name.encode(), op_type.encode(), len(inputs), _cstrs(list(inputs)),
            len(outputs), _cstrs(list(outputs)), len(keys), _cstrs(keys), vals))
        self._n_nodes += 1
        for k, v in attributes.items():
            if isinstance(v, (float, np.floating)):
                check(self._L.icx_graph_set_node_attr_float(self._g, name.encode(), k.encode(),
                                                            float(v)))
            elif isinstance(v, (list, tuple)) and all(isinstance(x, (int, np.integer)) for x in v):
                arr = (ctypes.c_int64 * max(len(v), 1))(*[int(x) for x in v])
                check(self._L.icx_graph_set_node_attr_ints(self._g, name.encode(), k.encode(),
                                                           len(v), arr))

    def add_output(self, name):
        if name not in self._outputs:
            self._outputs.append(name)
        check(self._L.icx_graph_add_output(self._g, name.encode()))

    def set_option(self, name, value):
        """Planner option; ``"quantized_outputs"``: True (default) lets a head whose output
        only a DynamicQuantizeLinear reads write that DQL's outputs in the same launch, False
        runs every DQL as its own launch (bit-identical results), also the DQL that a quantized
        linear's launch would run for its own input; ``"quantized_inputs"`` turns off that
        second fusion alone.  Replans at the next run."""
        check(self._L.icx_graph_set_option(self._g, name.encode(), int(value)))

    # ---- lowering -------------------------------------------------------------------------
    def plan(self):
        """Fusion decision and op order (host only, no GPU work): a list of PlanEntry, plus
        the DQL outputs whose row sums the fused GEMMs read."""
        size = 1 << 16
        while True:
            buf = ctypes.create_string_buffer(size)
            rc = self._L.icx_graph_plan(self._g, buf, size)
            if rc == 0:
                break
            msg = self._L.icx_last_error().decode()
            if "buffer has" not in msg or size > (1 << 26):
                check(rc)
            size *= 4
        entries, rowsums, ranges, quant_out, quant_in = [], [], [], {}, {}
        self._quant_launches = self._dql_single = self._qin_launches = 0
        for line in buf.value.decode().splitlines():
            parts = line.split()
            if parts[0] == "rowsum":
                rowsums.append(parts[1])
                continue
            if parts[0] == "range":
                ranges.append(parts[1])
                continue
            if parts[0] == "quantout":
                quant_out[parts[1]] = parts[2]
                continue
            if parts[0] == "quantout-launches":
                self._quant_launches = int(parts[1])
                continue
            if parts[0] == "quantin":
                quant_in[parts[1]] = parts[2]
                continue
            if parts[0] == "quantin-launches":
                self._qin_launches = int(parts[1])
                continue
            if parts[0] == "dql-single-launches":
                self._dql_single = int(parts[1])
                continue
            extra = dict(p.split("=", 1) for p in parts[4:])
            entries.append(PlanEntry(parts[0], parts[1], parts[2], parts[3],
                                     int(extra.get("steps", 0)), extra.get("out"),
                                     extra.get("wzp") == "folded", extra.get("group")))
        self._range_inputs = ranges
        self._quant_out = quant_out
        self._quant_in = quant_in
        return entries, rowsums

    def quantized_outputs(self):
        """Head outputs (quantized linear, attention) read only by a DynamicQuantizeLinear,
        mapped to that node: the head's kernel writes the DQL's outputs itself when the shape
        allows, and the f32 tensor is never formed.  Second value: how many head launches so
        far did that."""
        self.plan()
        return dict(self._quant_out), self._quant_launches

    def quantized_inputs(self):
        """Quantized-linear head outputs whose input's DynamicQuantizeLinear (read by that head
        alone) the head's GEMM launch runs too, mapped to that DQL node; second value: how many
        head launches so far did that (the others ran the DQL on its own first)."""
        self.plan()
        return dict(self._quant_in), self._qin_launches

    def single_launch_dqls(self):
        """How many DynamicQuantizeLinear runs so far were one launch (the blocks trading
        their ranges through the graph's exchange buffer) rather than two."""
        self.plan()
        return self._dql_single

    def range_inputs(self):
        """DynamicQuantizeLinear inputs whose producing kernel (LayerNorm, attention, a
        quantized linear) leaves their min / max, so that DQL runs its quantize pass only."""
        self.plan()
        return list(self._range_inputs)

    def compile(self):
        torch = _torch()
        check(self._L.icx_graph_compile(self._g, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))

    # ---- execution ------------------------------------------------------------------------
    def _bind(self, inputs):
        torch = _torch()
        self._keep = []
        for name, t in inputs.items():
            if isinstance(t, torch.Tensor) and t.is_cuda:
                t = t.contiguous()
                code = _NP_DT.get(np.dtype(str(t.dtype).replace("torch.", "")))
                if code is None:
                    raise IconnxError(3, "input '%s': dtype %s unsupported" % (name, t.dtype))
                self._keep.append(t)
                check(self._L.icx_graph_set_input(self._g, name.encode(), code, t.dim(),
                                                  _dims(t.shape), ctypes.c_void_p(t.data_ptr()), 1))
                continue
            arr = np.asarray(t.numpy() if isinstance(t, torch.Tensor) else t)
            if not arr.flags.c_contiguous:  # (np.ascontiguousarray would make a 0-d input 1-d)
                arr = arr.copy(order="C")
            code = _NP_DT.get(arr.dtype)
            if code is None:
                raise IconnxError(3, "input '%s': dtype %s unsupported" % (name, arr.dtype))
            check(self._L.icx_graph_set_input(self._g, name.encode(), code, arr.ndim,
                                              _dims(arr.shape), arr.ctypes.data_as(ctypes.c_void_p), 0))

    def run_device(self, inputs, output_names):
        """Run on ``torch.cuda.current_stream()``; returns {name: device tensor} (copies that
        outlive the next run).  Nothing synchronises the host."""
        torch = _torch()
        for n in output_names:
            self.add_output(n)
        self._bind(inputs)
        stream = torch.cuda.current_stream().cuda_stream
        check(self._L.icx_graph_run(self._g, ctypes.c_void_p(stream)))
        return self._fetch(output_names, stream)

    def _fetch(self, output_names, stream):
        torch = _torch()
        out = {}
        for n in output_names:
            dt, rank = ctypes.c_int(), ctypes.c_int()
            dims = (ctypes.c_int64 * 8)()
            ptr = ctypes.c_void_p()
            check(self._L.icx_graph_get_output(self._g, n.encode(), ctypes.byref(dt),
                                               ctypes.byref(rank), dims, ctypes.byref(ptr)))
            t = torch.empty([dims[i] for i in range(rank.value)], dtype=_torch_dt(dt.value),
                            device="cuda")
            nbytes = t.numel() * t.element_size()
            if nbytes:
                _hip_memcpy_d2d(ctypes.c_void_p(t.data_ptr()), ptr, nbytes, ctypes.c_void_p(stream))
            out[n] = t
        return out

    def run(self, inputs, output_names):
        """As the reference's ``run``: host arrays in (device tensors also accepted), host
        arrays (numpy) out."""
        dev = self.run_device(inputs, output_names)
        out = {k: v.cpu().numpy() for k, v in dev.items()}
        self.check_status()
        return out

    def run_with_profiling(self, inputs, output_names):
        """``run`` with per-op timing (GpuGraphExecutor::run_with_profiling,
        src/cuda/inference/mod.rs:649-658): every executed op of one eager run is bracketed by
        hipEvents on the launch stream.  Returns (host outputs, :class:`ProfileData`), whose
        ``gpu_op_times`` / ``op_times`` map each label — the op type, or ``Fused_<pattern>``
        for a fused head, as the reference labels them — to (microseconds, calls)."""
        import time

        torch = _torch()
        t0 = time.perf_counter()
        for n in output_names:
            self.add_output(n)
        self._bind(inputs)
        stream = torch.cuda.current_stream().cuda_stream
        cap = self._n_nodes + 8  # at most one executed op per node
        recs = (OpProfile * cap)()
        n_ops, up = ctypes.c_int(), ctypes.c_float()
        check(self._L.icx_graph_run_profiled(self._g, ctypes.c_void_p(stream), recs, cap,
                                             ctypes.byref(n_ops), ctypes.byref(up)))
        t1 = time.perf_counter()
        dev = self._fetch(output_names, stream)
        out = {k: v.cpu().numpy() for k, v in dev.items()}
        self.check_status()
        t2 = time.perf_counter()
        prof = ProfileData()
        prof.input_upload_us = float(up.value)
        for r in recs[:min(n_ops.value, cap)]:
            label, node = r.label.decode(), r.node.decode()
            prof.ops.append((node, label, float(r.gpu_us), float(r.cpu_us)))
            for m, v in ((prof.gpu_op_times, r.gpu_us), (prof.op_times, r.cpu_us)):
                us, calls = m.get(label, (0.0, 0))
                m[label] = (us + float(v), calls + 1)
        prof.node_execution_us = sum(o[3] for o in prof.ops)
        prof.output_download_us = (t2 - t1) * 1e6
        prof.total_us = (t2 - t0) * 1e6
        return out, prof

    def check_status(self):
        """Synchronise the current stream, then raise IconnxError (ICX_ERR_KERNEL) if a
        kernel of an earlier run or replay recorded a failure on the device — the reference
        surfaces failed launches as CudaError::Kernel (src/cuda/executor/mod.rs:169-186).
        ``run`` calls this; after ``run_device`` or ``replay`` a caller calls it before
        trusting the outputs."""
        torch = _torch()
        check(self._L.icx_graph_status(self._g, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))

    def capture(self, inputs, output_names):
        """Record one run into a HIP graph on ``torch.cuda.current_stream()``.  ``inputs``
        must be device tensors: the graph reads them in place, so a caller writes new data
        into the same tensors before :meth:`replay`.  A warm-up run executes first; the
        recorded run does not."""
        torch = _torch()
        for n, t in inputs.items():
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous()):
                raise IconnxError(1, "capture: input '%s' must be a contiguous device tensor" % n)
        for n in output_names:
            self.add_output(n)
        self._bind(inputs)
        # recorded on a stream of the executor's own (the legacy default stream cannot be
        # captured), ordered after and before the caller's stream
        if getattr(self, "_stream", None) is None:
            self._stream = torch.cuda.Stream()
        cur = torch.cuda.current_stream()
        self._stream.wait_stream(cur)
        check(self._L.icx_graph_capture(self._g, ctypes.c_void_p(self._stream.cuda_stream)))
        cur.wait_stream(self._stream)

    def replay(self):
        """Launch the recorded run, ordered after the current stream's work and before its
        later work (asynchronous)."""
        torch = _torch()
        if getattr(self, "_stream", None) is None:
            raise IconnxError(1, "replay: nothing captured (call capture first)")
        cur = torch.cuda.current_stream()
        self._stream.wait_stream(cur)
        check(self._L.icx_graph_replay(self._g, ctypes.c_void_p(self._stream.cuda_stream)))
        cur.wait_stream(self._stream)

    def outputs(self, output_names):
        """{name: device tensor}: copies of the outputs of the last run or replay (ordered
        after it on the current stream)."""
        torch = _torch()
        out = {}
        for n in output_names:
            dt, rank = ctypes.c_int(), ctypes.c_int()
            dims = (ctypes.c_int64 * 8)()
            ptr = ctypes.c_void_p()
            check(self._L.icx_graph_get_output(self._g, n.encode(), ctypes.byref(dt),
                                               ctypes.byref(rank), dims, ctypes.byref(ptr)))
            shape = [dims[i] for i in range(rank.value)]
            t = torch.empty(shape, dtype=_torch_dt(dt.value), device="cuda")
            nbytes = t.numel() * t.element_size()
            if nbytes:
                _hip_memcpy_d2d(ctypes.c_void_p(t.data_ptr()), ptr, nbytes,
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            out[n] = t
        return out

    def pool_stats(self):
        """(hipMalloc calls, pool hits, bytes held by the pool)."""
        a, b, c = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        check(self._L.icx_graph_pool_stats(self._g, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
        return a.value, b.value, c.value
