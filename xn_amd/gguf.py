"""GGUF files -> device quantized tensors, and back.

Reads the GGUF container (versions 1-3) the way xn's gguf_file.rs does
(gguf_file.rs:1-483: magic and version, metadata key/values of 13 value
types, tensor infos with dimensions stored fastest-first, tensor data at the
`general.alignment` boundary, default 32) and uploads each quantized tensor to
the device with the library's repack (ggml_file.rs:128-163
qtensor_from_ggml); the file's block bytes are not changed.  The writer
follows gguf_file.rs:493-541 (version 3, 32-byte padding of the tensor-info
section and of every tensor) and takes each tensor's canonical bytes from
QTensor.data(), i.e. raw_data, so read -> write reproduces the input tensors
byte for byte.

Tensor data is read from the file one tensor at a time (seek + read), so a
multi-gigabyte file is never held in host memory at once.
"""
from __future__ import annotations

import enum
import struct
from dataclasses import dataclass
from typing import BinaryIO, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from ._lib import XnqError
from .quantized import GgmlDType, QTensor

DEFAULT_ALIGNMENT = 32
_MAGICS = (0x46554747, 0x47475546)  # "GGUF" read as little- or big-endian u32


class ValueType(enum.IntEnum):
    """GGUF metadata value types (gguf_file.rs ValueType::from_u32)."""

    U8 = 0
    I8 = 1
    U16 = 2
    I16 = 3
    U32 = 4
    I32 = 5
    F32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    U64 = 10
    I64 = 11
    F64 = 12


_SCALAR = {
    ValueType.U8: "<B", ValueType.I8: "<b", ValueType.U16: "<H", ValueType.I16: "<h",
    ValueType.U32: "<I", ValueType.I32: "<i", ValueType.F32: "<f", ValueType.U64: "<Q",
    ValueType.I64: "<q", ValueType.F64: "<d",
}


@dataclass
class Value:
    """One metadata value: its GGUF type and the Python value (a list of
    Value for arrays)."""

    vtype: ValueType
    value: object

    def to_u64(self) -> int:
        """Unsigned integer (or bool) widened to u64, as Value::to_u64."""
        if self.vtype in (ValueType.U8, ValueType.U16, ValueType.U32, ValueType.U64, ValueType.BOOL):
            return int(self.value)
        raise XnqError(1, f"not a u64 or upcastable to u64 {self}")


@dataclass
class TensorInfo:
    ggml_dtype: GgmlDType
    shape: Tuple[int, ...]  # slowest-first, as xn's Shape (the file stores them reversed)
    offset: int             # from the start of the tensor data

    def size_in_bytes(self) -> int:
        elems = int(np.prod(self.shape)) if self.shape else 1
        bs = self.ggml_dtype.block_size()
        if elems % bs:
            raise XnqError(1, f"the number of elements {elems} is not divisible by the block size {bs}")
        return elems // bs * self.ggml_dtype.type_size()


class _Reader:
    def __init__(self, f: BinaryIO):
        self.f = f

    def take(self, fmt: str):
        n = struct.calcsize(fmt)
        b = self.f.read(n)
        if len(b) != n:
            raise XnqError(1, "gguf: unexpected end of file")
        return struct.unpack(fmt, b)[0]

    def string(self, v1: bool) -> str:
        n = self.take("<I" if v1 else "<Q")
        b = self.f.read(n)
        if len(b) != n:
            raise XnqError(1, "gguf: unexpected end of file")
        # GGUF strings should not be null terminated, but some files are (gguf_file.rs:88-91)
        return b.rstrip(b"\0").decode("utf-8", errors="replace")

    def value(self, vt: ValueType, v1: bool) -> Value:
        if vt in _SCALAR:
            return Value(vt, self.take(_SCALAR[vt]))
        if vt == ValueType.BOOL:
            b = self.take("<B")
            if b not in (0, 1):
                raise XnqError(1, f"unexpected bool value {b}")
            return Value(vt, bool(b))
        if vt == ValueType.STRING:
            return Value(vt, self.string(v1))
        if vt == ValueType.ARRAY:
            et = _value_type(self.take("<I"))
            n = self.take("<I" if v1 else "<Q")
            return Value(vt, [self.value(et, v1) for _ in range(n)])
        raise XnqError(1, f"unrecognized value-type {int(vt):#08x}")


def _value_type(v: int) -> ValueType:
    try:
        return ValueType(v)
    except ValueError:
        raise XnqError(1, f"unrecognized value-type {v:#08x}") from None


class Content:
    """The parsed header of a GGUF file (gguf_file.rs Content)."""

    def __init__(self, version: int, metadata: Dict[str, Value], tensor_infos: Dict[str, TensorInfo],
                 tensor_data_offset: int):
        self.version = version
        self.metadata = metadata
        self.tensor_infos = tensor_infos
        self.tensor_data_offset = tensor_data_offset

    @classmethod
    def read(cls, f: BinaryIO) -> "Content":
        r = _Reader(f)
        magic = r.take("<I")
        if magic not in _MAGICS:
            raise XnqError(1, f"unknown magic 0x{magic:08x}")
        version = r.take("<I")
        if version not in (1, 2, 3):
            raise XnqError(1, f"gguf: unsupported magic/version Gguf/{version}")
        v1 = version == 1
        n_tensors = r.take("<I" if v1 else "<Q")
        n_kv = r.take("<I" if v1 else "<Q")
        metadata: Dict[str, Value] = {}
        for _ in range(n_kv):
            key = r.string(v1)
            metadata[key] = r.value(_value_type(r.take("<I")), v1)
        infos: Dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = r.string(v1)
            nd = r.take("<I")
            dims = [r.take("<I" if v1 else "<Q") for _ in range(nd)]
            dt = r.take("<I")
            try:
                gdt = GgmlDType(dt)
            except ValueError:
                raise XnqError(1, f"unknown dtype for tensor {dt}") from None
            offset = r.take("<Q")
            infos[name] = TensorInfo(gdt, tuple(reversed(dims)), offset)
        pos = f.tell()
        align = DEFAULT_ALIGNMENT
        a = metadata.get("general.alignment")
        if a is not None and a.vtype in (ValueType.U8, ValueType.U16, ValueType.U32, ValueType.I8,
                                         ValueType.I16, ValueType.I32) and int(a.value) >= 0:
            align = int(a.value)
        return cls(version, metadata, infos, (pos + align - 1) // align * align)

    def apply_key_map(self, key_map: Callable[[str], Optional[str]]) -> "Content":
        """Rename tensors; a name mapped to None is dropped (gguf_file.rs:455-471)."""
        infos = {}
        for k, v in self.tensor_infos.items():
            nk = key_map(k)
            if nk is not None:
                infos[nk] = v
        return Content(self.version, self.metadata, infos, self.tensor_data_offset)

    def raw_tensor(self, f: BinaryIO, name: str) -> Tuple[TensorInfo, np.ndarray]:
        """The tensor's block bytes exactly as stored in the file."""
        info = self.tensor_infos.get(name)
        if info is None:
            raise XnqError(1, f"cannot find tensor info for {name}")
        n = info.size_in_bytes()
        f.seek(self.tensor_data_offset + info.offset)
        data = np.frombuffer(f.read(n), dtype=np.uint8)
        if data.nbytes != n:
            raise XnqError(1, f"gguf: tensor {name} runs past the end of the file")
        return info, data

    def tensor(self, f: BinaryIO, name: str, device="cuda") -> Union[QTensor, "object"]:
        """Load one tensor onto the device: a QTensor (repacked on the device)
        for Q4_0 / Q8_0 / Q4_K / Q6_K, a torch tensor for F32 / F16 / BF16.
        Other GGML dtypes raise, as xn does for dtypes a device does not
        implement."""
        import torch

        info, data = self.raw_tensor(f, name)
        dt = info.ggml_dtype
        if dt in (GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16):
            tdt = {GgmlDType.F32: torch.float32, GgmlDType.F16: torch.float16,
                   GgmlDType.BF16: torch.bfloat16}[dt]
            t = torch.frombuffer(bytearray(data.tobytes()), dtype=tdt).reshape(info.shape)
            return t.to(device)
        return QTensor.from_gguf_bytes(data, info.shape, dt, device)


def read(path: str) -> Content:
    with open(path, "rb") as f:
        return Content.read(f)


def load_all(path: str, device="cuda", names: Optional[Sequence[str]] = None) -> Dict[str, object]:
    """Every (or the named) tensor of a GGUF file, on the device."""
    with open(path, "rb") as f:
        c = Content.read(f)
        return {n: c.tensor(f, n, device) for n in (names if names is not None else c.tensor_infos)}


class GgufWeights:
    """Named weights of one GGUF file on one device, the GGUF branch of xn's
    VarBuilder (var_builder.rs:213-245 load_gguf / load_gguf_with_key_map,
    :284-330 qtensor / tensor): `qtensor` keeps the blocks quantized on the
    device, `tensor` returns them dequantized (f32, on the device), and the
    names fetched so far are recorded in `used`."""

    def __init__(self, path: str, device="cuda", key_map: Optional[Callable[[str], Optional[str]]] = None):
        self._f = open(path, "rb")
        c = Content.read(self._f)
        self.content = c.apply_key_map(key_map) if key_map is not None else c
        self.device = device
        self.used = set()

    def close(self) -> None:
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor_names(self) -> List[str]:
        return list(self.content.tensor_infos)

    def contains(self, name: str) -> bool:
        return name in self.content.tensor_infos

    def shape(self, name: str) -> Optional[Tuple[int, ...]]:
        info = self.content.tensor_infos.get(name)
        return None if info is None else info.shape

    def qtensor(self, name: str):
        t = self.content.tensor(self._f, name, self.device)
        self.used.add(name)
        return t

    def tensor(self, name: str, shape: Optional[Sequence[int]] = None):
        t = self.qtensor(name)
        out = t.dequantize() if isinstance(t, QTensor) else t.float()
        if shape is not None and tuple(out.shape) != tuple(shape):
            raise XnqError(1, f"shape mismatch for {name}, got {tuple(out.shape)}, expected {tuple(shape)}")
        return out


# ------------------------------------------------------------------ writer
def _write_string(f: BinaryIO, s: str) -> None:
    b = s.encode("utf-8")
    f.write(struct.pack("<Q", len(b)))
    f.write(b)


def _write_value(f: BinaryIO, v: Value) -> None:
    if v.vtype in _SCALAR:
        f.write(struct.pack(_SCALAR[v.vtype], v.value))
    elif v.vtype == ValueType.BOOL:
        f.write(struct.pack("<B", 1 if v.value else 0))
    elif v.vtype == ValueType.STRING:
        _write_string(f, v.value)
    elif v.vtype == ValueType.ARRAY:
        items: List[Value] = list(v.value)
        types = {x.vtype for x in items}
        if len(types) > 1:
            raise XnqError(1, f"multiple value-types in the same array {types}")
        et = types.pop() if types else ValueType.U32
        f.write(struct.pack("<IQ", int(et), len(items)))
        for x in items:
            _write_value(f, x)
    else:
        raise XnqError(1, f"unrecognized value-type {v.vtype}")


def _pad32(n: int) -> int:
    return 31 - (31 + n) % 32


def write(f: BinaryIO, metadata: Sequence[Tuple[str, Value]], tensors: Sequence[Tuple[str, object]]) -> None:
    """Write a version-3 GGUF file.  Each tensor is a QTensor (its canonical
    GGUF bytes via raw_data) or a (GgmlDType, shape, bytes) triple."""
    entries = []
    for name, t in tensors:
        if isinstance(t, QTensor):
            entries.append((name, t.dtype(), tuple(t.shape()), t.data()))
        else:
            dt, shape, data = t
            entries.append((name, GgmlDType(dt), tuple(shape), bytes(data)))
    f.write(struct.pack("<IIQQ", 0x46554747, 3, len(entries), len(metadata)))
    for key, v in metadata:
        _write_string(f, key)
        f.write(struct.pack("<I", int(v.vtype)))
        _write_value(f, v)
    offset = 0
    for name, dt, shape, data in entries:
        _write_string(f, name)
        f.write(struct.pack("<I", len(shape)))
        for d in reversed(shape):
            f.write(struct.pack("<Q", d))
        f.write(struct.pack("<IQ", int(dt), offset))
        offset += len(data) + _pad32(len(data))
    f.write(b"\0" * _pad32(f.tell()))
    for _, _, _, data in entries:
        f.write(data)
        f.write(b"\0" * _pad32(len(data)))
