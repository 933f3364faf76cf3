"""One decode step's quantized matmuls, captured into a replayable graph.

xn's llama decode step (xn-core/src/models/llama.rs:145-160 the q/k/v/o
projections, 236-264 the SwiGLU MLP, plus the lm_head) runs every weight
through QMatMul; its CUDA backend records the step once and replays it
(cuda_backend/mod.rs:236-300, Device::capture_begin / capture_end /
CaptureGraph::launch).  DecodeStep does that for the quantized-matmul part of
the step on this library:

  per layer  q, k, v = x . Wq^T, x . Wk^T, x . Wv^T      one grouped call
             o       = attn . Wo^T
             h       = silu(o' . Wg^T) * (o' . Wu^T)     one MLP call
             x_next  = h . Wd^T
  then       logits  = x_L . Wlm^T

Every activation lives in a buffer the step owns (one per layer and role, so
each product can be checked afterwards), and every call gets a slice of one
preallocated workspace, so capture makes no allocation.  The non-matmul
parts of the model (rmsnorm, RoPE, attention, residual adds) are outside
the quantized path: `glue(point, layer, bufs)` is called at "attention"
(write bufs["attn"] from q/k/v), "post_attention" (may rewrite bufs["o"] in
place) and "post_mlp" (write bufs["x_next"]) and may enqueue
non-allocating work on the current stream.  Without glue the chain feeds
each product forward: attn = q, and the next layer's input is the down
projection's output.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Sequence

import torch

from . import _lib
from ._lib import XnqError, check
from .quantized import CaptureGraph, GgmlDType, QTensor, _ptr, _stream, capture


@dataclass
class LayerWeights:
    """The seven quantized weights of one transformer block (llama.rs Attention + Mlp)."""

    q: QTensor
    k: QTensor
    v: QTensor
    o: QTensor
    gate: QTensor
    up: QTensor
    down: QTensor

    def all(self) -> List[QTensor]:
        return [self.q, self.k, self.v, self.o, self.gate, self.up, self.down]


@dataclass
class DecoderWeights:
    layers: List[LayerWeights]
    lm_head: QTensor

    @property
    def hidden(self) -> int:
        return self.layers[0].q.shape()[1]

    @property
    def kv_dim(self) -> int:
        return self.layers[0].k.shape()[0]

    @property
    def ffn(self) -> int:
        return self.layers[0].gate.shape()[0]

    @property
    def vocab(self) -> int:
        return self.lm_head.shape()[0]

    def weight_bytes(self) -> int:
        """GGUF bytes streamed by one step (every weight once)."""
        qts = [w for lw in self.layers for w in lw.all()] + [self.lm_head]
        return sum(qt.storage_size_in_bytes() for qt in qts)

    @classmethod
    def random(cls, layers: int, hidden: int, kv_dim: int, ffn: int, vocab: int, device,
               generator: Optional[torch.Generator] = None, attn_dtype=GgmlDType.Q4K, down_dtype=GgmlDType.Q6K,
               head_dtype=GgmlDType.Q6K, std: float = 0.02) -> "DecoderWeights":
        """N(0, std) weights quantized on the device: Q4_K attention and
        gate/up, Q6_K down and lm_head by default (a Q4_K_M-style mix)."""

        def make(n, k, dt):
            w = torch.randn((n, k), generator=generator, device=device, dtype=torch.float32) * std
            q = QTensor.quantize_f32(w, (n, k), dt)
            del w
            return q

        ls = [LayerWeights(make(hidden, hidden, attn_dtype), make(kv_dim, hidden, attn_dtype),
                           make(kv_dim, hidden, attn_dtype), make(hidden, hidden, attn_dtype),
                           make(ffn, hidden, attn_dtype), make(ffn, hidden, attn_dtype),
                           make(hidden, ffn, down_dtype)) for _ in range(layers)]
        return cls(ls, make(vocab, hidden, head_dtype))

    @classmethod
    def from_gguf(cls, weights, layers: int) -> "DecoderWeights":
        """From a llama GGUF file opened as xn_amd.gguf.GgufWeights, with the
        llama.cpp tensor names (blk.{i}.attn_q.weight, ..., output.weight)."""

        def get(name):
            qt = weights.qtensor(name)
            if not isinstance(qt, QTensor):
                raise XnqError(1, f"{name} is not a quantized tensor")
            return qt

        ls = [LayerWeights(*(get(f"blk.{i}.{n}.weight") for n in
                             ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")))
              for i in range(layers)]
        return cls(ls, get("output.weight"))


Glue = Callable[[str, int, Dict[str, torch.Tensor]], None]


class DecodeStep:
    """All quantized matmuls of one decode step for `batch` rows.

    `x` is the step's input (batch, hidden); after `run()` or a replay of
    `capture()`'s graph, `logits` holds (batch, vocab) and `bufs[l]` every
    layer's intermediate activations."""

    def __init__(self, weights: DecoderWeights, batch: int, device=None, glue: Optional[Glue] = None):
        self.w = weights
        self.b = int(batch)
        if self.b < 1:
            raise XnqError(1, "batch must be at least 1")
        self.device = torch.device(device) if device is not None else weights.lm_head.device
        self.glue = glue
        d, kv, ff, vocab = weights.hidden, weights.kv_dim, weights.ffn, weights.vocab
        for i, lw in enumerate(weights.layers):
            for name, qt, shape in (("q", lw.q, (d, d)), ("k", lw.k, (kv, d)), ("v", lw.v, (kv, d)),
                                    ("o", lw.o, (d, d)), ("gate", lw.gate, (ff, d)), ("up", lw.up, (ff, d)),
                                    ("down", lw.down, (d, ff))):
                if tuple(qt.shape()) != shape:
                    raise XnqError(1, f"layer {i} {name}: shape {tuple(qt.shape())}, expected {shape}")
        if tuple(weights.lm_head.shape()) != (vocab, d):
            raise XnqError(1, f"lm_head: shape {tuple(weights.lm_head.shape())}")

        def buf(n):
            return torch.zeros((self.b, n), dtype=torch.float32, device=self.device)

        self.x = buf(d)
        self.bufs: List[Dict[str, torch.Tensor]] = []
        for _ in weights.layers:
            q = buf(d)
            self.bufs.append({"q": q, "k": buf(kv), "v": buf(kv), "attn": q if glue is None else buf(d),
                              "o": buf(d), "h": buf(ff), "x_next": None})
        for i, bl in enumerate(self.bufs):
            bl["x"] = self.x if i == 0 else self.bufs[i - 1]["x_next"]
            bl["down"] = buf(d)
            bl["x_next"] = bl["down"] if glue is None else buf(d)
        self.logits = buf(vocab)

        L = _lib.load()
        sizes = []
        for lw in weights.layers:
            hs = (ctypes.c_void_p * 3)(lw.q.storage.handle, lw.k.storage.handle, lw.v.storage.handle)
            sizes.append(L.xnq_matmul_t_group_workspace_size(hs, 3, self.b))
            sizes.append(L.xnq_qtensor_matmul_t_workspace_size(lw.o.storage.handle, self.b))
            sizes.append(L.xnq_mlp_t_workspace_size(lw.gate.storage.handle, lw.up.storage.handle,
                                                    lw.down.storage.handle, self.b))
        sizes.append(L.xnq_qtensor_matmul_t_workspace_size(weights.lm_head.storage.handle, self.b))
        # calls run in stream order, so one workspace serves them all
        self.ws_bytes = max(sizes + [1])
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=self.device)
        self.graph: Optional[CaptureGraph] = None

    # -- the step ------------------------------------------------------------

    def _launch_all(self) -> None:
        L = _lib.load()
        st = _stream(self.device)
        b, d, ff, vocab = self.b, self.w.hidden, self.w.ffn, self.w.vocab
        ws, wsn = _ptr(self.ws), self.ws_bytes
        for i, (lw, bl) in enumerate(zip(self.w.layers, self.bufs)):
            hs = (ctypes.c_void_p * 3)(lw.q.storage.handle, lw.k.storage.handle, lw.v.storage.handle)
            ds = (ctypes.c_void_p * 3)(_ptr(bl["q"]), _ptr(bl["k"]), _ptr(bl["v"]))
            check(L.xnq_matmul_t_group(hs, 3, b, d, _ptr(bl["x"]), ds, ws, wsn, st))
            if self.glue is not None:
                self.glue("attention", i, bl)
            check(L.xnq_qtensor_matmul_t_ws(lw.o.storage.handle, b, d, d, _ptr(bl["attn"]), ws, wsn,
                                            _ptr(bl["o"]), st))
            if self.glue is not None:
                self.glue("post_attention", i, bl)
            check(L.xnq_mlp_t(lw.gate.storage.handle, lw.up.storage.handle, lw.down.storage.handle, b, d, ff,
                              _ptr(bl["o"]), ws, wsn, _ptr(bl["h"]), _ptr(bl["down"]), st))
            if self.glue is not None:
                self.glue("post_mlp", i, bl)
        last = self.bufs[-1]["x_next"] if self.bufs else self.x
        check(L.xnq_qtensor_matmul_t_ws(self.w.lm_head.storage.handle, b, d, vocab, _ptr(last), ws, wsn,
                                        _ptr(self.logits), st))

    def run(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Launch the step's calls directly on `stream` (default: the current stream)."""
        with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream(self.device)):
            self._launch_all()

    def capture(self, stream: Optional[torch.cuda.Stream] = None) -> CaptureGraph:
        """Record the step into a graph (Device::capture_begin / capture_end);
        `replay()` then launches it.  `stream` must not be the null stream."""
        s = stream if stream is not None else torch.cuda.Stream(self.device)
        torch.cuda.synchronize(self.device)
        with capture(s) as c:
            self._launch_all()
        self.graph = c.graph
        self._capture_stream = s
        return self.graph

    def replay(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        if self.graph is None:
            raise XnqError(1, "replay before capture")
        self.graph.launch(stream if stream is not None else self._capture_stream)

    def products(self) -> Sequence[tuple]:
        """(name, weight(s), input, output) of every product of the step, in
        launch order, for checking each one against a reference."""
        out = []
        for i, (lw, bl) in enumerate(zip(self.w.layers, self.bufs)):
            out.append((f"layer{i}.q", lw.q, bl["x"], bl["q"]))
            out.append((f"layer{i}.k", lw.k, bl["x"], bl["k"]))
            out.append((f"layer{i}.v", lw.v, bl["x"], bl["v"]))
            out.append((f"layer{i}.o", lw.o, bl["attn"], bl["o"]))
            out.append((f"layer{i}.gate_up", (lw.gate, lw.up), bl["o"], bl["h"]))
            out.append((f"layer{i}.down", lw.down, bl["h"], bl["down"]))
        last = self.bufs[-1]["x_next"] if self.bufs else self.x
        out.append(("lm_head", self.w.lm_head, last, self.logits))
        return out
