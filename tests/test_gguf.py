"""GGUF files to the product's weights (kapel_amd/gguf.py), on the CPU: the
cases of kapel-hub/src/gguf.rs:633-790 on files built here byte by byte, and
files written by kapel_amd.gguf.write read back, blocks unchanged."""
import os
import struct

import numpy as np
import pytest

import kapel_amd as ka
from kapel_amd import gguf


def build(metadata, tensors, data):
    """gguf.rs:585-612: metadata [(key, type, value bytes)], tensors [(name,
    dims fastest first, ggml type, offset)], then `data` at the next multiple
    of 32."""
    def string(s):
        raw = s.encode()
        return struct.pack("<Q", len(raw)) + raw
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for key, kind, value in metadata:
        out += string(key) + struct.pack("<I", kind) + value
    for name, dims, ggml_type, offset in tensors:
        out += string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ggml_type, offset)
    out += bytes(-len(out) % 32)
    return bytes(out) + bytes(data)


def valid():
    """Two f32 tensors, [2, 3] and [2] (gguf.rs:616-623)."""
    data = np.arange(8, dtype=np.float32).tobytes()
    return build([("general.alignment", 4, struct.pack("<I", 32))],
                 [("a", [3, 2], 0, 0), ("b", [2], 0, 24)], data)


def error_of(data):
    with pytest.raises(gguf.FormatError) as e:
        gguf.Gguf.from_bytes(data)
    return str(e.value)


def test_a_minimal_file_is_read():
    f = gguf.Gguf.from_bytes(valid())
    assert f.names() == ["a", "b"]
    a = f.array("a")
    assert a.shape == (2, 3) and a.ravel().tolist() == [0, 1, 2, 3, 4, 5]
    assert f.array("b").tolist() == [6.0, 7.0]
    with pytest.raises(gguf.Missing):
        f.array("c")


def test_a_bad_alignment_is_an_error():
    for alignment in (2 ** 64 - 1, 0, 3, 48, gguf.MAX_ALIGNMENT * 2):
        err = error_of(build([("general.alignment", 10, struct.pack("<Q", alignment))],
                             [("a", [1], 0, 0)], bytes(4)))
        assert "general.alignment" in err, alignment
    err = error_of(build([("general.alignment", 8, b"\x01\0\0\0\0\0\0\0x")], [], b""))
    assert "general.alignment" in err
    # The largest alignment accepted, with a much shorter header.
    head = build([("general.alignment", 10, struct.pack("<Q", gguf.MAX_ALIGNMENT))], [("a", [1], 0, 0)], b"")
    padded = head + bytes((1 << 16) - len(head)) + np.float32(1.5).tobytes()
    assert gguf.Gguf.from_bytes(padded).array("a").tolist() == [1.5]
    assert "beyond the file" in error_of(head)


def test_offsets_beyond_the_file_are_errors():
    data = bytes(8)
    for offset in (8, 9, 1 << 40, 2 ** 64 - 1, 2 ** 64 - 32):
        err = error_of(build([], [("a", [2], 0, offset)], data))
        assert "beyond the file" in err or "does not fit" in err, offset
    err = error_of(build([], [("a", [2 ** 32 - 1] * 3, 0, 0)], data))
    assert "does not fit" in err


def test_every_truncation_is_an_error():
    data = valid()
    for n in range(len(data)):
        err = error_of(data[:n])
        assert any(m in err for m in ("truncated", "does not fit", "beyond the file")), n


def test_a_tensor_of_an_unknown_type_fails_alone():
    data = bytes(8)
    f = gguf.Gguf.from_bytes(build([], [("a", [2], 0, 0), ("iq", [32, 4], 16, 8)], data))
    assert f.info("iq").kind is None
    assert f.array("a").size == 2
    with pytest.raises(gguf.FormatError, match="does not read"):
        f.raw("iq")
    assert "starts beyond the file" in error_of(build([], [("iq", [32], 16, 9)], data))


def test_metadata_of_every_type_reads_back(tmp_path):
    E = gguf.Entry
    meta = [("u8", E("u8", 200)), ("i8", E("i8", -3)), ("u16", E("u16", 65000)), ("i16", E("i16", -300)),
            ("u32", E("u32", 4000000000)), ("i32", E("i32", -7)), ("f32", E("f32", 0.5)), ("b", E("bool", True)),
            ("s", E("string", "llama")), ("arr", E("array", [E("string", "a"), E("string", "bc")])),
            ("u64", E("u64", 2 ** 40)), ("i64", E("i64", -2 ** 40)), ("f64", E("f64", 0.1)),
            ("nested", E("array", [E("array", [E("u32", 1), E("u32", 2)])])),
            ("general.alignment", E("u32", 32))]
    path = tmp_path / "m.gguf"
    gguf.write(path, meta, [])
    f = gguf.Gguf.open(path)
    assert f.metadata == {"u8": 200, "i8": -3, "u16": 65000, "i16": -300, "u32": 4000000000, "i32": -7,
                          "f32": 0.5, "b": True, "s": "llama", "arr": ["a", "bc"], "u64": 2 ** 40,
                          "i64": -2 ** 40, "f64": 0.1, "nested": [[1, 2]], "general.alignment": 32}
    with pytest.raises(gguf.FormatError):
        gguf.write(path, [("k", E("u8", 1)), ("k", E("u8", 2))], [])
    with pytest.raises(gguf.FormatError):
        gguf.write(path, [("a", E("array", [E("u8", 1), E("u16", 2)]))], [])
    with pytest.raises(gguf.FormatError):
        gguf.write(path, [("general.alignment", E("u32", 64))], [])


@pytest.mark.parametrize("fmt", [ka.Q4_0, ka.Q4_1, ka.Q5_0, ka.Q5_1, ka.Q8_0, ka.Q2K, ka.Q3K, ka.Q4K,
                                 ka.Q5K, ka.Q6K, ka.IQ4_NL, ka.IQ4_XS, ka.IQ3_S])
def test_quantized_tensors_keep_their_blocks(tmp_path, fmt):
    """A quantized matrix written and read back: the same blocks, byte for
    byte, at a 32-byte aligned offset, its type the ggml one (gguf.rs:65-90)."""
    import torch
    n, k = 6, 512
    rng = np.random.default_rng(fmt)
    blocks = rng.integers(0, 256, size=n * k // ka.block_len(fmt) * ka.block_bytes(fmt), dtype=np.uint8)
    q = ka.QuantizedTensor(torch.from_numpy(blocks), fmt, 0, n, k)
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    path = tmp_path / "q.gguf"
    gguf.write(path, [("general.architecture", gguf.Entry("string", "test"))], [("x", x), ("w", q)])
    f = gguf.Gguf.open(path)
    assert f.info("w").ggml_type == gguf.ggml_type_of_format(fmt)
    back = f.quantized("w")
    assert (back.fmt, back.n, back.k) == (fmt, n, k)
    assert np.array_equal(back.data.numpy(), blocks)
    assert (f.data_start + f.info("w").offset) % 32 == 0
    assert np.array_equal(f.array("x"), x)
    with pytest.raises(ka.InvalidArgument):
        f.quantized("x")


def test_kapel_groups_are_not_gguf(tmp_path):
    import torch
    w = ka.QuantizedTensor(torch.zeros(36, dtype=torch.uint8), ka.INT8, 32, 1, 32)
    with pytest.raises(gguf.FormatError):
        gguf.write(tmp_path / "k.gguf", [], [("w", w)])
    assert not os.path.exists(tmp_path / "k.gguf")
