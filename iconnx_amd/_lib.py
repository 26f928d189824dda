"""ctypes binding of libiconnx_hip.so (the C ABI declared in include/iconnx_hip.h).

The library is built ahead of time (``python -m iconnx_amd.build``).  Loading fails loudly
when it is missing: there is no fallback implementation anywhere in this package.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libiconnx_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "iconnx_hip.h")

ICX_I8, ICX_U8, ICX_I32, ICX_F32, ICX_I64, ICX_BOOL = 0, 1, 2, 3, 4, 5
# status codes (include/iconnx_hip.h)
ICX_OK, ICX_ERR_INVALID_ARG, ICX_ERR_SHAPE, ICX_ERR_DTYPE, ICX_ERR_WORKSPACE, ICX_ERR_HIP = 0, 1, 2, 3, 4, 5
ICX_ERR_UNSUPPORTED, ICX_ERR_KERNEL = 6, 7
OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3
OP_ERF, OP_SAVE, OP_MUL_SAVED = 4, 5, 6
BCAST_SCALAR, BCAST_COL, BCAST_ROW, BCAST_FULL = 0, 1, 2, 3
MAX_CHAIN = 8


class IconnxError(RuntimeError):
    """A failed library call (the reference's CudaError::Kernel(String))."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


class ChainOp(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("operand_is_lhs", ctypes.c_int32),
                ("kind0", ctypes.c_int32), ("kind1", ctypes.c_int32),
                ("p0", ctypes.c_void_p), ("p1", ctypes.c_void_p)]


class OpProfile(ctypes.Structure):
    _fields_ = [("label", ctypes.c_char * 48), ("node", ctypes.c_char * 80),
                ("gpu_us", ctypes.c_float), ("cpu_us", ctypes.c_float)]


class Chain(ctypes.Structure):
    _fields_ = [("n_ops", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("ops", ChainOp * MAX_CHAIN)]


_lib = None

P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
C, CP = ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)
SIGNATURES = {
    "icx_status_str": ([I], ctypes.c_char_p),
    "icx_last_error": ([], ctypes.c_char_p),
    "icx_version": ([], ctypes.c_char_p),
    "icx_stream_create": ([ctypes.POINTER(P)], I),
    "icx_stream_destroy": ([P], I),
    "icx_stream_synchronize": ([P], I),
    "icx_pool_create": ([], P),
    "icx_pool_destroy": ([P], None),
    "icx_pool_alloc": ([P, S, ctypes.POINTER(P)], I),
    "icx_pool_free": ([P, P], I),
    "icx_pool_stats": ([P, P, P, P], I),
    "icx_host_alloc": ([S, ctypes.POINTER(P)], I),
    "icx_host_free": ([P], I),
    "icx_memcpy_h2d_async": ([P, P, P, S], I),
    "icx_memcpy_d2h_async": ([P, P, P, S], I),
    "icx_dql_workspace_size": ([S], S),
    "icx_dynamic_quantize_linear": ([P, P, S, P, P, P, P, S, P, S], I),
    "icx_packed_weight_bytes": ([S, S], S),
    "icx_pack_weight": ([P, P, I, S, S, P, P], I),
    "icx_matmul_integer_workspace_size": ([S, S, S, I], S),
    "icx_matmul_integer": ([P, P, I, P, I, I, P, S, S, S, P, P, S, P, P, P, S], I),
    "icx_matmul_integer_noalloc_max_bytes": ([], S),
    "icx_matmul_integer_noalloc": ([P, P, I, P, I, I, P, S, S, S, P, P, S, P, P], I),
    "icx_fused_chain_f32": ([P, P, S, S, ctypes.POINTER(Chain), P], I),
    "icx_qlinear_f32": ([P, P, I, P, I, I, P, S, S, S, P, P, S, P, ctypes.POINTER(Chain), P, P, S], I),
    "icx_dql_qlinear_f32": ([P, P, S, S, P, P, P, P, I, P, S, ctypes.POINTER(Chain), P, P], I),
    "icx_cast_i32_f32": ([P, P, S, P], I),
    "icx_dequantize_linear_f32": ([P, P, I, P, P, S, S, S, P], I),
    "icx_gather": ([P, P, S, S, S, S, P, I, S, P], I),
    "icx_layer_norm_f32": ([P, P, P, S, S, P, P, ctypes.c_float, P], I),
    "icx_softmax_f32": ([P, P, S, S, P], I),
    "icx_reduce_mean_f32": ([P, P, S, S, S, I, P], I),
    "icx_pow_f32": ([P, P, S, S, P, I, P], I),
    "icx_sqrt_f32": ([P, P, S, P], I),
    "icx_transpose": ([P, P, S, I, P, P, P], I),
    "icx_matmul_f32": ([P, P, P, S, I, S, S, S, P], I),
    "icx_attention_f32": ([P, P, P, P, S, S, S, S, S, S, S, S, ctypes.c_float, I, I, P], I),
    "icx_graph_create": ([], P),
    "icx_graph_destroy": ([P], None),
    "icx_graph_add_input": ([P, C, I, P], I),
    "icx_graph_add_initializer": ([P, C, I, I, P, P], I),
    "icx_graph_add_node": ([P, C, C, I, CP, I, CP, I, CP, P], I),
    "icx_graph_add_output": ([P, C], I),
    "icx_exchange_buffer_size": ([], ctypes.c_size_t),
    "icx_dynamic_quantize_linear_exchange": ([P, P, ctypes.c_size_t, P, P, P, P], I),
    "icx_exchange_status": ([P, P], I),
    "icx_graph_set_option": ([P, C, ctypes.c_int64], I),
    "icx_graph_set_node_attr_float": ([P, C, C, ctypes.c_double], I),
    "icx_graph_set_node_attr_ints": ([P, C, C, I, P], I),
    "icx_graph_plan": ([P, P, S], I),
    "icx_graph_compile": ([P, P], I),
    "icx_graph_set_input": ([P, C, I, I, P, P, I], I),
    "icx_graph_run": ([P, P], I),
    "icx_graph_run_profiled": ([P, P, ctypes.POINTER(OpProfile), I, ctypes.POINTER(I),
                                ctypes.POINTER(ctypes.c_float)], I),
    "icx_graph_get_output": ([P, C, ctypes.POINTER(I), ctypes.POINTER(I), P, ctypes.POINTER(P)], I),
    "icx_graph_pool_stats": ([P, P, P, P], I),
    "icx_graph_capture": ([P, P], I),
    "icx_graph_replay": ([P, P], I),
    "icx_graph_status": ([P, P], I),
    "icx_debug_qout_fault": ([I], None),
}


def header_symbols():
    """Function names declared in include/iconnx_hip.h."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(icx_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError("libiconnx_hip.so is not built (%s); run `python -m iconnx_amd.build`"
                          % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def check(status):
    if status != 0:
        L = lib()
        msg = L.icx_last_error().decode() or L.icx_status_str(status).decode()
        raise IconnxError(status, msg)
