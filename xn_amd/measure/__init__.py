"""Measurement library (libxnq_measure.so): the bare HBM read the decode
matvec's weight stream is judged against.  Not part of the product: only
bench.py's `--only stream` leg and its GPU test load it."""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libxnq_measure.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        lib.xnqm_stream_read.restype = ctypes.c_int
        lib.xnqm_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        _lib = lib
    return _lib


def stream_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """Read every byte of the device buffer `buf` (XOR-folded into the int32
    device tensor `sink`) on the current stream."""
    if buf.device.type != "cuda" or not buf.is_contiguous() or sink.dtype != torch.int32:
        raise ValueError("stream_read: contiguous device buffer and an int32 device sink")
    nbytes = buf.numel() * buf.element_size()
    st = _load().xnqm_stream_read(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                  ctypes.c_void_p(torch.cuda.current_stream(buf.device).cuda_stream))
    if st:
        raise RuntimeError(f"xnqm_stream_read failed with status {st}")
