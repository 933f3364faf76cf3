"""Device-resident quantized tensors: the host-side mirror of xn's quantized API.

Mirrors gradium-ai/xn xn-core/src/quantized/mod.rs:
  GgmlDType            mod.rs:77-196   (ids, type_size, block_size)
  QStorage / QTensor   mod.rs:27-75, 305-340 (device storage instead of Cpu)
  QLinear              mod.rs:342-406
  backend_q instances  mod.rs:408-455  (Q40Hip, Q80Hip, Q4kHip, Q6kHip)
Every numerical operation runs in libxnq (HIP kernels for gfx950); torch only
provides device memory and the stream.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import XnqError, check


class GgmlDType(enum.IntEnum):
    """GGML dtype ids (mod.rs:97-137)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    Q8K = 15
    BF16 = 30

    @classmethod
    def from_u32(cls, u: int) -> "GgmlDType":
        try:
            return cls(u)
        except ValueError:
            raise XnqError(1, f"unknown dtype for tensor {u}") from None

    def to_u32(self) -> int:
        return int(self)

    def type_size(self) -> int:
        """Bytes per block (mod.rs:160-179)."""
        return _TYPE_SIZE[self]

    def block_size(self) -> int:
        """Elements per block (mod.rs:182-195)."""
        return _BLOCK_SIZE[self]


_TYPE_SIZE = {
    GgmlDType.F32: 4, GgmlDType.F16: 2, GgmlDType.BF16: 2, GgmlDType.Q4_0: 18, GgmlDType.Q4_1: 20,
    GgmlDType.Q5_0: 22, GgmlDType.Q5_1: 24, GgmlDType.Q8_0: 34, GgmlDType.Q8_1: 36,
    GgmlDType.Q2K: 84, GgmlDType.Q3K: 110, GgmlDType.Q4K: 144, GgmlDType.Q5K: 176,
    GgmlDType.Q6K: 210, GgmlDType.Q8K: 292,
}
_BLOCK_SIZE = {
    GgmlDType.F32: 1, GgmlDType.F16: 1, GgmlDType.BF16: 1, GgmlDType.Q4_0: 32, GgmlDType.Q4_1: 32,
    GgmlDType.Q5_0: 32, GgmlDType.Q5_1: 32, GgmlDType.Q8_0: 32, GgmlDType.Q8_1: 32,
    GgmlDType.Q2K: 256, GgmlDType.Q3K: 256, GgmlDType.Q4K: 256, GgmlDType.Q5K: 256,
    GgmlDType.Q6K: 256, GgmlDType.Q8K: 256,
}

# dtypes with a device implementation
DEVICE_DTYPES = (GgmlDType.Q4_0, GgmlDType.Q4_1, GgmlDType.Q5_0, GgmlDType.Q5_1, GgmlDType.Q8_0,
                 GgmlDType.Q2K, GgmlDType.Q3K, GgmlDType.Q4K, GgmlDType.Q5K, GgmlDType.Q6K)
# dtypes the device also quantizes from f32 (QTensor.quantize_f32 / QLinear.from_linear)
DEVICE_QUANTIZE_DTYPES = (GgmlDType.Q4_0, GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K)


def vec_dot_type(dtype: GgmlDType) -> GgmlDType:
    """Activation block type a weight dtype dots against (the VecDotType of
    k_quants.rs:210, 310, 405, 507, 615, 883, 1059, 1321, 1510, 1727)."""
    if dtype in (GgmlDType.Q4_0, GgmlDType.Q5_0, GgmlDType.Q8_0):
        return GgmlDType.Q8_0
    if dtype in (GgmlDType.Q4_1, GgmlDType.Q5_1):
        return GgmlDType.Q8_1
    return GgmlDType.Q8K


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _check_shape(dims: Tuple[int, ...], block_size: int) -> None:
    """mod.rs:262-274 check_shape."""
    if len(dims) == 0:
        raise XnqError(1, f"scalar tensor cannot be quantized {dims}")
    if dims[-1] % block_size != 0:
        raise XnqError(
            1, f"quantized tensor must have their last dim divisible by block size {dims} {block_size}"
        )


class QStorage:
    """Device storage of a quantized tensor (the HIP variant of mod.rs:32-34).

    Owns one libxnq qtensor handle: the GGUF blocks repacked into planes in HBM.
    """

    def __init__(self, handle: int, device: torch.device):
        self._h = ctypes.c_void_p(handle)
        self.device = device

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def dtype(self) -> GgmlDType:
        return GgmlDType(_lib.load().xnq_qtensor_dtype(self._h))

    def block_size(self) -> int:
        return self.dtype().block_size()

    def size_in_bytes(self) -> int:
        return _lib.load().xnq_qtensor_storage_size(self._h)

    def device_bytes(self) -> int:
        return _lib.load().xnq_qtensor_device_bytes(self._h)

    def rows(self) -> int:
        return _lib.load().xnq_qtensor_rows(self._h)

    def cols(self) -> int:
        return _lib.load().xnq_qtensor_cols(self._h)

    def close(self) -> None:
        if self._h is not None and self._h.value:
            _lib.load().xnq_qtensor_free(self._h)
            self._h = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _as_2d(dims: Tuple[int, ...]) -> Tuple[int, int]:
    k = dims[-1]
    n = int(np.prod(dims[:-1])) if len(dims) > 1 else 1
    return n, k


class QTensor:
    """A quantized tensor on a HIP device (mod.rs:27-30, 305-340)."""

    def __init__(self, storage: QStorage, shape: Sequence[int]):
        shape = tuple(int(s) for s in shape)
        _check_shape(shape, storage.block_size())
        self.storage = storage
        self._shape = shape

    # -- constructors -----------------------------------------------------
    @classmethod
    def from_gguf_bytes(cls, data, shape: Sequence[int], dtype: GgmlDType,
                        device: torch.device | str | int = "cuda") -> "QTensor":
        """Upload canonical GGUF block bytes (the on-disk layout) and repack them
        on the device (ggml_file.rs:128-163 qtensor_from_ggml, HIP variant)."""
        dtype = GgmlDType(dtype)
        shape = tuple(int(s) for s in shape)
        _check_shape(shape, dtype.block_size())
        device = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        if device.type != "cuda":
            raise XnqError(2, f"{dtype.name} QTensor requires a HIP device, got {device}")
        idx = device.index if device.index is not None else torch.cuda.current_device()
        n, k = _as_2d(shape)
        expect = n * (k // dtype.block_size()) * dtype.type_size()
        buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray)
                                   else data.view(np.uint8).reshape(-1))
        if buf.nbytes != expect:
            raise XnqError(1, f"{dtype.name} tensor {shape}: expected {expect} bytes, got {buf.nbytes}")
        out = ctypes.c_void_p()
        dev = torch.device("cuda", idx)
        check(_lib.load().xnq_qtensor_upload(idx, int(dtype), buf.ctypes.data, n, k, _stream(dev),
                                             ctypes.byref(out)))
        return cls(QStorage(out.value, dev), shape)

    @classmethod
    def quantize_f32(cls, src: torch.Tensor, shape: Optional[Sequence[int]] = None,
                     dtype: GgmlDType = GgmlDType.Q4K) -> "QTensor":
        """Quantize a device f32 tensor (mod.rs:283-303), on the device."""
        dtype = GgmlDType(dtype)
        shape = tuple(src.shape) if shape is None else tuple(int(s) for s in shape)
        _check_shape(shape, dtype.block_size())
        if src.device.type != "cuda" or src.dtype != torch.float32:
            raise XnqError(1, "quantize_f32 expects a float32 tensor on a HIP device")
        src = src.contiguous()
        if src.numel() != int(np.prod(shape)):
            raise XnqError(1, f"tensor size {src.numel()} does not match shape {shape}")
        n, k = _as_2d(shape)
        out = ctypes.c_void_p()
        check(_lib.load().xnq_qtensor_quantize(src.device.index, int(dtype), _ptr(src), n, k,
                                               _stream(src.device), ctypes.byref(out)))
        return cls(QStorage(out.value, src.device), shape)

    # -- accessors --------------------------------------------------------
    def dtype(self) -> GgmlDType:
        return self.storage.dtype()

    def rank(self) -> int:
        return len(self._shape)

    def shape(self) -> Tuple[int, ...]:
        return self._shape

    @property
    def device(self) -> torch.device:
        return self.storage.device

    def storage_size_in_bytes(self) -> int:
        return self.storage.size_in_bytes()

    def __repr__(self) -> str:
        return f"QTensor[{list(self._shape)}; {self.dtype().name}]"

    # -- operations -------------------------------------------------------
    def dequantize(self) -> torch.Tensor:
        """f32 values on the device, in `shape` (mod.rs:316-318)."""
        out = torch.empty(self._shape, dtype=torch.float32, device=self.device)
        check(_lib.load().xnq_qtensor_dequantize(self.storage.handle, _ptr(out), out.numel(),
                                                 _stream(self.device)))
        return out

    def to_tensor(self) -> torch.Tensor:
        return self.dequantize()

    def data(self) -> bytes:
        """Canonical GGUF block bytes (mod.rs:206-214 raw_data)."""
        nbytes = self.storage_size_in_bytes()
        host = np.empty(nbytes, dtype=np.uint8)
        check(_lib.load().xnq_qtensor_raw_data(self.storage.handle, host.ctypes.data, nbytes,
                                               _stream(self.device)))
        return host.tobytes()

    def _check_mm(self, mkn, lhs: torch.Tensor, dst: torch.Tensor) -> Tuple[int, int, int]:
        m, k, n = (int(v) for v in mkn)
        if m * k != lhs.numel():
            raise XnqError(1, f"unexpected lhs length {lhs.numel()} {(m, k, n)}")
        if dst.numel() < m * n:
            raise XnqError(1, f"dst too small ({dst.numel()} < {m * n})")
        for t, name in ((lhs, "lhs"), (dst, "dst")):
            if t.device != self.device or t.dtype != torch.float32 or not t.is_contiguous():
                raise XnqError(1, f"{name} must be a contiguous float32 tensor on {self.device}")
        return m, k, n

    def matmul_t(self, mkn: Tuple[int, int, int], lhs: torch.Tensor, dst: torch.Tensor) -> None:
        """dst[m, n] = quantize(lhs[m, k]) . W^T (mod.rs:334-339, k_quants.rs:1996-2011).

        Decode-sized m on small weights is one kernel that quantizes the
        rows in LDS; otherwise the quantized activation goes to a workspace
        from torch's caching allocator (graph-capture safe, no per-call
        device allocation) and the library runs quantize_lhs + T::matmul, as
        k_quants::matmul does.  Runs on the current stream."""
        m, k, n = self._check_mm(mkn, lhs, dst)
        if m == 0 or n == 0:
            return
        L = _lib.load()
        h = self.storage.handle
        nbytes = L.xnq_qtensor_matmul_t_workspace_size(h, m)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device) if nbytes else None
        check(L.xnq_qtensor_matmul_t_ws(h, m, k, n, _ptr(lhs), _ptr(ws) if ws is not None else None, nbytes,
                                        _ptr(dst), _stream(self.device)))

    def matmul_t_workspace_size(self, m: int) -> int:
        """Bytes of caller scratch matmul_t_ws needs for m rows (0 on the fused decode route)."""
        return int(_lib.load().xnq_qtensor_matmul_t_workspace_size(self.storage.handle, int(m)))

    def matmul_t_ws(self, mkn: Tuple[int, int, int], lhs: torch.Tensor, ws: Optional[torch.Tensor],
                    dst: torch.Tensor) -> None:
        """matmul_t with caller-owned scratch `ws` (uint8, at least
        matmul_t_workspace_size(m) bytes): allocates nothing, so it can be
        captured into a graph."""
        m, k, n = self._check_mm(mkn, lhs, dst)
        nbytes = ws.numel() if ws is not None else 0
        check(_lib.load().xnq_qtensor_matmul_t_ws(self.storage.handle, m, k, n, _ptr(lhs),
                                                  _ptr(ws) if ws is not None else None, nbytes, _ptr(dst),
                                                  _stream(self.device)))

    def matmul_t_noalloc(self, mkn: Tuple[int, int, int], lhs: torch.Tensor, dst: torch.Tensor) -> None:
        """matmul_t with the library's static per-GPU scratch
        (xnq_qtensor_matmul_t_noalloc): allocates nothing; calls on one GPU
        must not overlap."""
        m, k, n = self._check_mm(mkn, lhs, dst)
        check(_lib.load().xnq_qtensor_matmul_t_noalloc(self.storage.handle, m, k, n, _ptr(lhs), _ptr(dst),
                                                       _stream(self.device)))

    def matmul_t_split(self, mkn: Tuple[int, int, int], lhs: torch.Tensor, dst: torch.Tensor) -> None:
        """quantize_lhs then matmul_preq as two library calls, for every m
        (k_quants.rs:2014-2026: quantize_lhs, then T::matmul)."""
        m, k, n = self._check_mm(mkn, lhs, dst)
        if m == 0 or n == 0:
            return
        ws = self.workspace(m)
        L = _lib.load()
        st = _stream(self.device)
        check(L.xnq_quantize_lhs(int(self.dtype()), m, k, _ptr(lhs), _ptr(ws), st))
        check(L.xnq_qtensor_matmul_preq(self.storage.handle, m, k, n, _ptr(ws), ws.numel(), _ptr(dst), st))

    def workspace(self, m: int) -> torch.Tensor:
        """Scratch for quantize_lhs + matmul_preq of m rows on this weight."""
        nbytes = _lib.load().xnq_qtensor_workspace_size(self.storage.handle, int(m))
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)

    def matmul_t_abi(self, mkn: Tuple[int, int, int], lhs: torch.Tensor, dst: torch.Tensor) -> None:
        """The same product through the single C entry point xnq_qtensor_matmul_t
        (what a foreign caller binds): m == 1 on small weights quantizes inside
        the matvec kernel, other calls use a stream-ordered workspace."""
        m, k, n = self._check_mm(mkn, lhs, dst)
        check(_lib.load().xnq_qtensor_matmul_t(self.storage.handle, m, k, n, _ptr(lhs), _ptr(dst),
                                               _stream(self.device)))


class QLinear:
    """A linear layer with a device quantized weight (mod.rs:342-406)."""

    def __init__(self, weight: QTensor, bias: Optional[torch.Tensor] = None):
        self.weight = weight
        self.bias = bias

    def with_bias(self, bias: torch.Tensor) -> "QLinear":
        self.bias = bias
        return self

    @classmethod
    def from_linear(cls, weight: torch.Tensor, bias: Optional[torch.Tensor], dtype: GgmlDType) -> "QLinear":
        """mod.rs:397-405: quantize an f32 [out, in] weight (on the device)."""
        return cls(QTensor.quantize_f32(weight.contiguous(), tuple(weight.shape), dtype), bias)

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        """mod.rs:352-384: (..., k) -> (..., n), then + bias."""
        dims = self.weight.shape()
        if len(dims) != 2:
            raise XnqError(1, f"unexpected rank, expected: 2, got: {len(dims)} ({dims})")
        n, k = dims
        if xs.dim() < 2:
            raise XnqError(1, f"input tensor has only one dimension {tuple(xs.shape)}")
        if xs.shape[-1] != k:
            raise XnqError(1, f"input tensor {tuple(xs.shape)} incompatible with {list(dims)}")
        dst_shape = tuple(xs.shape[:-1]) + (n,)
        dst = torch.empty(dst_shape, dtype=torch.float32, device=self.weight.device)
        xs = xs.contiguous()
        m = xs.numel() // k
        self.weight.matmul_t((m, k, n), xs, dst)
        if self.bias is not None:
            dst = dst + self.bias
        return dst

    __call__ = forward


def _backend_q(name: str, dtype: GgmlDType):
    """The BackendQ instances of mod.rs:408-455, for the HIP device."""

    @dataclass(frozen=True)
    class _B:
        DTYPE = dtype

        @staticmethod
        def from_linear(weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> QLinear:
            return QLinear.from_linear(weight, bias, dtype)

        @staticmethod
        def linear_load(vb, in_features: int, out_features: int) -> QLinear:
            """Use the GGUF tensor `weight` when the builder has one, else quantize
            the f32 `weight` (mod.rs:422-439)."""
            qt = vb.qtensor("weight")
            bias = vb.get_optional("bias") if hasattr(vb, "get_optional") else None
            if qt is not None:
                if list(qt.shape()) != [out_features, in_features]:
                    raise XnqError(1, f"quantized weight tensor has wrong shape {list(qt.shape())}, "
                                      f"expected [{out_features}, {in_features}]")
                return QLinear(qt, bias)
            w = vb.get("weight", (out_features, in_features))
            return QLinear.from_linear(w, bias, dtype)

    _B.__name__ = name
    return _B


Q40Hip = _backend_q("Q40Hip", GgmlDType.Q4_0)
Q41Hip = _backend_q("Q41Hip", GgmlDType.Q4_1)
Q50Hip = _backend_q("Q50Hip", GgmlDType.Q5_0)
Q51Hip = _backend_q("Q51Hip", GgmlDType.Q5_1)
Q80Hip = _backend_q("Q80Hip", GgmlDType.Q8_0)
Q2kHip = _backend_q("Q2kHip", GgmlDType.Q2K)
Q3kHip = _backend_q("Q3kHip", GgmlDType.Q3K)
Q4kHip = _backend_q("Q4kHip", GgmlDType.Q4K)
Q5kHip = _backend_q("Q5kHip", GgmlDType.Q5K)
Q6kHip = _backend_q("Q6kHip", GgmlDType.Q6K)


# -- decode-step groups: weights that read one activation ----------------------

def matmul_t_silu_gate(gate: QTensor, up: QTensor, mkn: Tuple[int, int, int], lhs: torch.Tensor,
                       dst: torch.Tensor) -> None:
    """dst = silu(lhs . gate^T) * (lhs . up^T): the SwiGLU of llama.rs:258-264
    (silu(s) = s / (1 + exp(0 - s)), cpu_backend.rs:354-356); one kernel at
    m = 1.  Runs on the current stream."""
    m, k, n = gate._check_mm(mkn, lhs, dst)
    L = _lib.load()
    nbytes = L.xnq_matmul_t_silu_gate_workspace_size(gate.storage.handle, up.storage.handle, m)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gate.device) if nbytes else None
    check(L.xnq_matmul_t_silu_gate(gate.storage.handle, up.storage.handle, m, k, n, _ptr(lhs),
                                   _ptr(ws) if ws is not None else None, nbytes, _ptr(dst), _stream(gate.device)))


def mlp_t(gate: QTensor, up: QTensor, down: QTensor, m: int, lhs: torch.Tensor, h: torch.Tensor,
          dst: torch.Tensor) -> None:
    """The SwiGLU MLP of llama.rs:236-264: h = silu(lhs . gate^T) * (lhs . up^T),
    dst = h . down^T; h [m, f] and dst [m, down rows] are both written.  Runs
    on the current stream."""
    k, f = gate.shape()[1], gate.shape()[0]
    gate._check_mm((m, k, f), lhs, h)
    down._check_mm((m, f, down.shape()[0]), h, dst)
    L = _lib.load()
    nbytes = L.xnq_mlp_t_workspace_size(gate.storage.handle, up.storage.handle, down.storage.handle, m)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gate.device) if nbytes else None
    check(L.xnq_mlp_t(gate.storage.handle, up.storage.handle, down.storage.handle, m, k, f, _ptr(lhs),
                      _ptr(ws) if ws is not None else None, nbytes, _ptr(h), _ptr(dst), _stream(gate.device)))


def matmul_t_group(qts, m: int, k: int, lhs: torch.Tensor, dsts) -> None:
    """dsts[i][m, n_i] = lhs . qts[i]^T for weights of one dtype and K (the q,
    k, v projections of llama.rs:156-158); one kernel at m = 1."""
    qts = list(qts)
    dsts = list(dsts)
    if len(qts) != len(dsts):
        raise XnqError(1, f"{len(qts)} weights but {len(dsts)} destinations")
    for qt, d in zip(qts, dsts):
        qt._check_mm((m, k, qt.shape()[0]), lhs, d)
    L = _lib.load()
    hs = (ctypes.c_void_p * max(len(qts), 1))(*[qt.storage.handle for qt in qts])
    ds = (ctypes.c_void_p * max(len(dsts), 1))(*[d.data_ptr() for d in dsts])
    nbytes = L.xnq_matmul_t_group_workspace_size(hs, len(qts), m)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=lhs.device) if nbytes else None
    check(L.xnq_matmul_t_group(hs, len(qts), m, k, _ptr(lhs), ds, _ptr(ws) if ws is not None else None, nbytes,
                               _stream(lhs.device)))


# -- stream capture (cuda_backend/mod.rs:251-283: capture_begin / capture_end) --

class CaptureGraph:
    """A captured sequence of library launches, replayed with launch()."""

    def __init__(self, handle: int, device):
        self.handle = handle
        self.device = device

    def launch(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        s = stream.cuda_stream if stream is not None else _stream(self.device)
        check(_lib.load().xnq_graph_launch(self.handle, s))

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            _lib.load().xnq_graph_free(h)


class capture:
    """with capture(stream) as c: <library calls on stream>; then c.graph.launch().

    The calls inside are recorded, not run (Device::capture_begin /
    capture_end); use the entry points that allocate nothing (matmul_t on the
    decode route, matmul_t_ws, the group / gate entries with workspaces)."""

    def __init__(self, stream: torch.cuda.Stream):
        self.stream = stream
        self.graph: Optional[CaptureGraph] = None

    def __enter__(self) -> "capture":
        self._ctx = torch.cuda.stream(self.stream)
        self._ctx.__enter__()
        check(_lib.load().xnq_capture_begin(self.stream.cuda_stream))
        return self

    def __exit__(self, exc_type, exc, tb) -> bool:
        L = _lib.load()
        try:
            if exc_type is not None:
                L.xnq_capture_abort(self.stream.cuda_stream)
                return False
            out = ctypes.c_void_p()
            check(L.xnq_capture_end(self.stream.cuda_stream, ctypes.byref(out)))
            self.graph = CaptureGraph(out.value, self.stream.device)
            return False
        finally:
            self._ctx.__exit__(exc_type, exc, tb)


# -- lower-level entry points used by tests and the benchmark ------------------

def set_route(route: int) -> None:
    """0 = route by m, 1 = force the matvec kernel, 2 = force the MFMA kernel,
    3 = force the skinny MFMA kernel (m <= 64, Q4_K / Q6_K)."""
    check(_lib.load().xnq_set_route(int(route)))


def lhs_workspace(dtype: GgmlDType, m: int, k: int, device) -> torch.Tensor:
    nbytes = _lib.load().xnq_lhs_workspace_size(int(dtype), m, k)
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def quantize_lhs(dtype: GgmlDType, lhs: torch.Tensor, ws: torch.Tensor, m: int, k: int) -> None:
    check(_lib.load().xnq_quantize_lhs(int(dtype), m, k, _ptr(lhs), _ptr(ws), _stream(lhs.device)))


def matmul_preq(qt: QTensor, m: int, ws: torch.Tensor, dst: torch.Tensor) -> None:
    n, k = qt.storage.rows(), qt.storage.cols()
    check(_lib.load().xnq_qtensor_matmul_preq(qt.storage.handle, m, k, n, _ptr(ws), ws.numel(), _ptr(dst),
                                              _stream(dst.device)))


def quantize_act_blocks(act_dtype: GgmlDType, x: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """Canonical BlockQ8_0 / BlockQ8K bytes of m rows of k floats, on the device."""
    act_dtype = GgmlDType(act_dtype)
    nbytes = m * (k // act_dtype.block_size()) * act_dtype.type_size()
    out = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    check(_lib.load().xnq_quantize_act_blocks(int(act_dtype), m, k, _ptr(x), _ptr(out),
                                              _stream(x.device)))
    return out[:nbytes]


def block_ints(qt: QTensor, m: int, ws: torch.Tensor) -> torch.Tensor:
    """int32 [m, n, blocks, 2] integer parts of every block dot (see xnq.h)."""
    n, k = qt.storage.rows(), qt.storage.cols()
    nb = k // qt.dtype().block_size()
    out = torch.empty((m, n, nb, 2), dtype=torch.int32, device=ws.device)
    check(_lib.load().xnq_qtensor_block_ints(qt.storage.handle, m, _ptr(ws), _ptr(out),
                                             _stream(ws.device)))
    return out
