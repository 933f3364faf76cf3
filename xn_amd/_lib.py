"""ctypes binding of libxnq.so, the C ABI declared in include/xnq.h.

Loading fails loudly: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("XNQ_LIB_PATH") or os.path.join(_HERE, "libxnq.so")

_lock = threading.Lock()
_lib = None

c_size = ctypes.c_size_t
c_u32 = ctypes.c_uint32
c_int = ctypes.c_int
c_void = ctypes.c_void_p

# name -> (restype, argtypes), one line per declaration in include/xnq.h
SIGNATURES = {
    "xnq_last_error": (ctypes.c_char_p, []),
    "xnq_abi_version": (c_int, []),
    "xnq_type_size": (c_size, [c_u32]),
    "xnq_block_size": (c_size, [c_u32]),
    "xnq_qtensor_upload": (c_int, [c_int, c_u32, c_void, c_size, c_size, c_void, ctypes.POINTER(c_void)]),
    "xnq_qtensor_upload_device": (c_int, [c_int, c_u32, c_void, c_size, c_size, c_void, ctypes.POINTER(c_void)]),
    "xnq_qtensor_quantize": (c_int, [c_int, c_u32, c_void, c_size, c_size, c_void, ctypes.POINTER(c_void)]),
    "xnq_qtensor_free": (None, [c_void]),
    "xnq_qtensor_dtype": (c_u32, [c_void]),
    "xnq_qtensor_rows": (c_size, [c_void]),
    "xnq_qtensor_cols": (c_size, [c_void]),
    "xnq_qtensor_device": (c_int, [c_void]),
    "xnq_qtensor_storage_size": (c_size, [c_void]),
    "xnq_qtensor_device_bytes": (c_size, [c_void]),
    "xnq_qtensor_matmul_t": (c_int, [c_void, c_size, c_size, c_size, c_void, c_void, c_void]),
    "xnq_qtensor_matmul_t_workspace_size": (c_size, [c_void, c_size]),
    "xnq_qtensor_matmul_t_ws": (c_int, [c_void, c_size, c_size, c_size, c_void, c_void, c_size, c_void, c_void]),
    "xnq_qtensor_matmul_t_noalloc": (c_int, [c_void, c_size, c_size, c_size, c_void, c_void, c_void]),
    "xnq_matmul_t_silu_gate_workspace_size": (c_size, [c_void, c_void, c_size]),
    "xnq_matmul_t_silu_gate": (c_int, [c_void, c_void, c_size, c_size, c_size, c_void, c_void, c_size, c_void, c_void]),
    "xnq_mlp_t_workspace_size": (c_size, [c_void, c_void, c_void, c_size]),
    "xnq_mlp_t": (c_int, [c_void, c_void, c_void, c_size, c_size, c_size, c_void, c_void, c_size, c_void, c_void,
                          c_void]),
    "xnq_matmul_t_group_workspace_size": (c_size, [ctypes.POINTER(c_void), c_size, c_size]),
    "xnq_matmul_t_group": (c_int, [ctypes.POINTER(c_void), c_size, c_size, c_size, c_void, ctypes.POINTER(c_void), c_void,
                                   c_size, c_void]),
    "xnq_capture_begin": (c_int, [c_void]),
    "xnq_capture_end": (c_int, [c_void, ctypes.POINTER(c_void)]),
    "xnq_capture_abort": (None, [c_void]),
    "xnq_graph_launch": (c_int, [c_void, c_void]),
    "xnq_graph_free": (None, [c_void]),
    "xnq_lhs_workspace_size": (c_size, [c_u32, c_size, c_size]),
    "xnq_qtensor_workspace_size": (c_size, [c_void, c_size]),
    "xnq_quantize_lhs": (c_int, [c_u32, c_size, c_size, c_void, c_void, c_void]),
    "xnq_qtensor_matmul_preq": (c_int, [c_void, c_size, c_size, c_size, c_void, c_size, c_void, c_void]),
    "xnq_set_route": (c_int, [c_int]),
    "xnq_qtensor_dequantize": (c_int, [c_void, c_void, c_size, c_void]),
    "xnq_qtensor_raw_data": (c_int, [c_void, c_void, c_size, c_void]),
    "xnq_quantize_act_blocks": (c_int, [c_u32, c_size, c_size, c_void, c_void, c_void]),
    "xnq_qtensor_block_ints": (c_int, [c_void, c_size, c_void, c_void, c_void]),
}

STATUS = {0: "XNQ_OK", 1: "XNQ_ERR_INVALID", 2: "XNQ_ERR_UNSUPPORTED", 3: "XNQ_ERR_HIP", 4: "XNQ_ERR_OOM"}


class XnqError(RuntimeError):
    """A libxnq call failed; `status` is the xnq_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.message = message


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libxnq.so (built in-tree by __graft_entry__.build()) and declare its ABI."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise ImportError(
                f"libxnq.so not found at {p}: build it first (python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().xnq_last_error().decode("utf-8", "replace")
        raise XnqError(status, msg)
