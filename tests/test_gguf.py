"""GGUF container: reader/writer on the CPU, device upload on the GPU.

The CPU tests pin the reader against files laid out byte by byte in the test
(versions 1, 2 and 3, custom alignment, null-terminated strings), so a reader
that shares a mistake with the writer still fails them.  The GPU tests load
a written file onto the device and check raw_data, dequantization and matmul
against the oracle, and that writing the loaded tensors back reproduces the
file byte for byte.
"""
import io
import struct

import numpy as np
import pytest

from xn_amd import XnqError
from xn_amd.gguf import Content, GgufWeights, TensorInfo, Value, ValueType, write
from xn_amd.quantized import GgmlDType

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14


def _s(b: bytes, v1=False) -> bytes:
    return struct.pack("<I" if v1 else "<Q", len(b)) + b


def _blocks(orc, dt: int, n: int, k: int, seed: int) -> np.ndarray:
    x = np.random.default_rng(seed).normal(0, 1, (n, k)).astype(np.float32)
    return orc.from_float(dt, x)


# ----------------------------------------------------------- CPU: reader
def test_reads_hand_built_v3_file():
    body = struct.pack("<IIQQ", 0x46554747, 3, 2, 3)
    body += _s(b"general.name") + struct.pack("<I", 8) + _s(b"tiny\0\0")  # trailing NULs are stripped
    body += _s(b"llama.block_count") + struct.pack("<II", 4, 7)
    body += _s(b"ids") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<iii", -1, 0, 9)
    body += _s(b"a.weight") + struct.pack("<I", 2) + struct.pack("<QQ", 256, 3) + struct.pack("<IQ", 12, 0)
    body += _s(b"b") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 448)
    hdr = len(body)
    body += b"\0" * (-hdr % 32)
    q4k = bytes(range(144)) * 3
    f32 = struct.pack("<4f", 1.0, -2.0, 0.5, 3.25)
    body += q4k + b"\0" * (448 - len(q4k)) + f32
    f = io.BytesIO(body)
    c = Content.read(f)
    assert c.version == 3
    assert c.tensor_data_offset == hdr + (-hdr % 32)
    assert c.metadata["general.name"].value == "tiny"
    assert c.metadata["llama.block_count"].to_u64() == 7
    assert [v.value for v in c.metadata["ids"].value] == [-1, 0, 9]
    assert c.tensor_infos["a.weight"] == TensorInfo(GgmlDType.Q4K, (3, 256), 0)
    assert c.tensor_infos["b"] == TensorInfo(GgmlDType.F32, (4,), 448)
    info, raw = c.raw_tensor(f, "a.weight")
    assert info.size_in_bytes() == 432 and raw.tobytes() == q4k
    assert c.raw_tensor(f, "b")[1].tobytes() == f32


def test_reads_v1_file_with_u32_lengths_and_custom_alignment():
    body = struct.pack("<IIII", 0x46554747, 1, 1, 2)
    body += _s(b"general.alignment", True) + struct.pack("<II", 4, 64)
    body += _s(b"flag", True) + struct.pack("<IB", 7, 1)
    body += _s(b"t", True) + struct.pack("<I", 2) + struct.pack("<II", 32, 2) + struct.pack("<IQ", 8, 0)
    off = len(body) + (-len(body) % 64)
    blocks = bytes(np.random.default_rng(0).integers(0, 256, 68, dtype=np.uint8))
    body += b"\0" * (off - len(body)) + blocks
    f = io.BytesIO(body)
    c = Content.read(f)
    assert c.version == 1 and c.tensor_data_offset == off and off % 64 == 0
    assert c.metadata["flag"].value is True
    assert c.tensor_infos["t"] == TensorInfo(GgmlDType.Q8_0, (2, 32), 0)
    assert c.raw_tensor(f, "t")[1].tobytes() == blocks


def test_byte_swapped_magic_is_accepted():
    body = struct.pack("<IIQQ", 0x47475546, 2, 0, 0)
    assert Content.read(io.BytesIO(body)).version == 2


@pytest.mark.parametrize("body,msg", [
    (struct.pack("<IIQQ", 0x12345678, 3, 0, 0), "magic"),
    (struct.pack("<IIQQ", 0x46554747, 4, 0, 0), "version"),
    (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s(b"k") + struct.pack("<I", 13), "value-type"),
    (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s(b"k") + struct.pack("<IB", 7, 2), "bool"),
    (struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s(b"t") + struct.pack("<IQIQ", 1, 32, 99, 0), "dtype"),
    (struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s(b"t"), "end of file"),
])
def test_rejects_malformed_headers(body, msg):
    with pytest.raises(XnqError, match=msg):
        Content.read(io.BytesIO(body))


def test_tensor_errors():
    f = io.BytesIO()
    write(f, [], [("w", (GgmlDType.Q8_0, (1, 32), b"\1" * 34))])
    f.seek(0)
    c = Content.read(f)
    with pytest.raises(XnqError, match="cannot find"):
        c.raw_tensor(f, "nope")
    c.tensor_infos["w"] = TensorInfo(GgmlDType.Q8_0, (1, 40), 0)
    with pytest.raises(XnqError, match="divisible"):
        c.raw_tensor(f, "w")
    c.tensor_infos["w"] = TensorInfo(GgmlDType.Q8_0, (4, 32), 0)
    with pytest.raises(XnqError, match="past the end"):
        c.raw_tensor(f, "w")


# ----------------------------------------------------------- CPU: writer
def test_write_read_round_trip(orc):
    meta = [
        ("u8", Value(ValueType.U8, 200)), ("i8", Value(ValueType.I8, -100)),
        ("u16", Value(ValueType.U16, 65535)), ("i16", Value(ValueType.I16, -3)),
        ("u32", Value(ValueType.U32, 1 << 31)), ("i32", Value(ValueType.I32, -(1 << 31))),
        ("f32", Value(ValueType.F32, 0.25)), ("b", Value(ValueType.BOOL, False)),
        ("s", Value(ValueType.STRING, "héllo")), ("u64", Value(ValueType.U64, 1 << 60)),
        ("i64", Value(ValueType.I64, -(1 << 60))), ("f64", Value(ValueType.F64, 1e300)),
        ("arr", Value(ValueType.ARRAY, [Value(ValueType.STRING, "a"), Value(ValueType.STRING, "bc")])),
        ("empty", Value(ValueType.ARRAY, [])),
    ]
    tensors = [
        ("q4k", (GgmlDType.Q4K, (3, 512), _blocks(orc, Q4K, 3, 512, 1).tobytes())),
        ("q6k", (GgmlDType.Q6K, (2, 256), _blocks(orc, Q6K, 2, 256, 2).tobytes())),
        ("q40", (GgmlDType.Q4_0, (5, 64), _blocks(orc, Q4_0, 5, 64, 3).tobytes())),
        ("q80", (GgmlDType.Q8_0, (2, 3, 32), _blocks(orc, Q8_0, 6, 32, 4).tobytes())),
        ("norm", (GgmlDType.F32, (7,), np.arange(7, dtype=np.float32).tobytes())),
    ]
    f = io.BytesIO()
    write(f, meta, tensors)
    f.seek(0)
    c = Content.read(f)
    assert c.version == 3 and c.tensor_data_offset % 32 == 0
    assert {k: v for k, v in c.metadata.items()} == dict(meta)
    for name, (dt, shape, data) in tensors:
        info, raw = c.raw_tensor(f, name)
        assert info.ggml_dtype == dt and info.shape == shape and info.offset % 32 == 0
        assert raw.tobytes() == data
    # Rewriting what was read reproduces the file.
    g = io.BytesIO()
    write(g, list(c.metadata.items()),
          [(n, (i.ggml_dtype, i.shape, c.raw_tensor(f, n)[1].tobytes())) for n, i in c.tensor_infos.items()])
    assert g.getvalue() == f.getvalue()


def test_writer_rejects_mixed_arrays():
    arr = Value(ValueType.ARRAY, [Value(ValueType.U8, 1), Value(ValueType.I8, 1)])
    with pytest.raises(XnqError, match="multiple value-types"):
        write(io.BytesIO(), [("a", arr)], [])


def test_apply_key_map():
    f = io.BytesIO()
    write(f, [], [("blk.0.w", (GgmlDType.F32, (2,), b"\0" * 8)), ("drop", (GgmlDType.F32, (1,), b"\0" * 4))])
    f.seek(0)
    c = Content.read(f).apply_key_map(lambda k: None if k == "drop" else k.replace("blk.", "layers."))
    assert list(c.tensor_infos) == ["layers.0.w"]


# ----------------------------------------------------------- GPU: upload
@pytest.mark.gpu
def test_gguf_file_to_device_and_back(orc, dev, tmp_path):
    import torch

    from xn_amd import QTensor

    specs = [("q4k", Q4K, 40, 512), ("q6k", Q6K, 33, 768), ("q40", Q4_0, 17, 96), ("q80", Q8_0, 9, 320)]
    blocks = {name: _blocks(orc, dt, n, k, 10 + i) for i, (name, dt, n, k) in enumerate(specs)}
    norm = np.linspace(-1, 1, 96, dtype=np.float32)
    path = str(tmp_path / "w.gguf")
    meta = [("general.architecture", Value(ValueType.STRING, "test"))]
    with open(path, "wb") as f:
        write(f, meta, [(name, (GgmlDType(dt), (n, k), blocks[name].tobytes())) for name, dt, n, k in specs]
              + [("norm", (GgmlDType.F32, (96,), norm.tobytes()))])
    rng = np.random.default_rng(5)
    loaded = []
    with GgufWeights(path, dev) as wb:
        assert sorted(wb.tensor_names()) == sorted([s[0] for s in specs] + ["norm"])
        for name, dt, n, k in specs:
            qt = wb.qtensor(name)
            assert isinstance(qt, QTensor) and qt.shape() == (n, k) and qt.dtype() == dt
            assert qt.data() == blocks[name].tobytes()
            deq = wb.tensor(name, (n, k)).cpu().numpy()
            assert np.array_equal(deq.reshape(-1), orc.to_float(dt, blocks[name]).reshape(-1))
            for m in (1, 7, 70):
                x = rng.normal(0, 1, (m, k)).astype(np.float32)
                y = torch.empty((m, n), dtype=torch.float32, device=dev)
                qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), y)
                want = orc.matmul(dt, x, blocks[name], n)
                got = y.cpu().numpy().astype(np.float64)
                rel = np.linalg.norm(got - want) / np.linalg.norm(want)
                assert rel <= 1e-3, f"{name} m={m}: relative L2 {rel:.3e}"
            loaded.append((name, qt))
        t = wb.qtensor("norm")
        assert t.device.type == "cuda" and np.array_equal(t.cpu().numpy(), norm)
        assert wb.used == {s[0] for s in specs} | {"norm"}
    out = io.BytesIO()
    write(out, meta, loaded + [("norm", (GgmlDType.F32, (96,), norm.tobytes()))])
    with open(path, "rb") as f:
        assert out.getvalue() == f.read()
