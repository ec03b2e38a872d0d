"""GGUF files (llama.cpp's format) to the product's weights: the header read,
every tensor's blocks mapped from the file and uploaded unchanged.

Follows kapel-hub/src/gguf.rs: the magic ``GGUF``, version 2 or 3, the counts
of tensors and metadata entries, the typed entries, the tensor descriptions
(name, dimensions fastest first, ggml type, offset), then the data from the
next multiple of ``general.alignment`` (32 by default, a power of two of at
most 64 KiB).  Shapes are given slowest dimension first, as Kapel's.  Every
tensor of a type this module reads must lie in the file; a tensor of another
type fails only when asked for (gguf.rs:204-285).

Quantized tensors keep their blocks: ``quantized`` returns a QuantizedTensor
whose bytes are the file's, copied once to the device, which the product reads
as they are (no repacking).
"""
import mmap
import os
import struct

import numpy as np

from . import (IQ3_S, IQ4_NL, IQ4_XS, Q2K, Q3K, Q4_0, Q4_1, Q4K, Q5_0, Q5_1, Q5K, Q6K, Q8_0,
               InvalidArgument, KapelError, QuantizedTensor, block_bytes, block_len)

DEFAULT_ALIGNMENT = 32
MAX_ALIGNMENT = 1 << 16


class FormatError(KapelError):
    """HubError::Format: not a valid GGUF file, or a tensor it cannot give."""


class Missing(KapelError):
    """HubError::Missing: no tensor of that name."""


# ggml type number -> ("q", format code) for the block formats, or
# ("f", numpy dtype name) for the plain ones (gguf.rs:65-90).
GGML_TYPES = {
    0: ("f", "float32"), 1: ("f", "float16"),
    2: ("q", Q4_0), 3: ("q", Q4_1), 6: ("q", Q5_0), 7: ("q", Q5_1), 8: ("q", Q8_0),
    10: ("q", Q2K), 11: ("q", Q3K), 12: ("q", Q4K), 13: ("q", Q5K), 14: ("q", Q6K),
    20: ("q", IQ4_NL), 21: ("q", IQ3_S), 23: ("q", IQ4_XS),
    24: ("f", "int8"), 26: ("f", "int32"), 28: ("f", "float64"), 30: ("f", "bfloat16"),
}
_FLOAT_BYTES = {"float32": 4, "float16": 2, "int8": 1, "int32": 4, "float64": 8, "bfloat16": 2}


def ggml_type_of_format(fmt):
    """The ggml type number of a block format (gguf.rs:454-457)."""
    for t, (kind, code) in GGML_TYPES.items():
        if kind == "q" and code == fmt:
            return t
    return None


class TensorInfo:
    """A tensor's description: shape (slowest first), ggml type, what this
    module reads it as (None: a type it does not read), offset in the data."""

    def __init__(self, shape, ggml_type, offset):
        self.shape = tuple(shape)
        self.ggml_type = ggml_type
        self.kind = GGML_TYPES.get(ggml_type)
        self.offset = offset

    def __repr__(self):
        return f"TensorInfo(shape={self.shape}, ggml_type={self.ggml_type})"


class _Reader:
    def __init__(self, data, name):
        self.data, self.at, self.name = data, 0, name

    def take(self, n):
        end = self.at + n
        if n < 0 or end > len(self.data):
            raise FormatError(f"{self.name}: truncated header at byte {self.at}")
        b = self.data[self.at:end]
        self.at = end
        return b

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def size(self):
        n = self.u64()
        if n > len(self.data):
            raise FormatError(f"{self.name}: a length of {n} does not fit in the file")
        return n

    def string(self):
        raw = bytes(self.take(self.size()))
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError:
            raise FormatError(f"{self.name}: a string is not UTF-8") from None

    def value(self, kind, depth=0):
        """gguf.rs:143-187: the value of a metadata entry of GGUF type `kind`."""
        fixed = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q",
                 11: "<q", 12: "<d"}
        if kind in fixed:
            fmt = fixed[kind]
            v = struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
            return float(v) if kind in (6, 12) else int(v)
        if kind == 7:
            return self.take(1)[0] != 0
        if kind == 8:
            return self.string()
        if kind == 9:
            if depth > 8:
                raise FormatError(f"{self.name}: arrays nested too deep")
            inner = self.u32()
            count = self.size()
            return [self.value(inner, depth + 1) for _ in range(count)]
        raise FormatError(f"{self.name}: unknown metadata type {kind}")


class Gguf:
    """A GGUF file, mapped in memory (Gguf::open) or held in bytes
    (Gguf::from_bytes)."""

    def __init__(self, data, name="<memory>", keep=None):
        self._data = data
        self._keep = keep
        self.name = name
        r = _Reader(data, name)
        if bytes(r.take(4)) != b"GGUF":
            raise FormatError(f"{name}: not a GGUF file (bad magic)")
        version = r.u32()
        if version not in (2, 3):
            raise FormatError(f"{name}: GGUF version {version} is not supported")
        tensor_count, kv_count = r.size(), r.size()
        self.metadata = {}
        self.metadata_types = {}  # key -> GGUF type number
        for _ in range(kv_count):
            key = r.string()
            kind = r.u32()
            self.metadata[key] = r.value(kind)
            self.metadata_types[key] = kind
        self._tensors = {}
        for _ in range(tensor_count):
            tname = r.string()
            dims = r.u32()
            if dims > 8:
                raise FormatError(f"{name}: tensor {tname!r} has {dims} dimensions")
            shape = [r.size() for _ in range(dims)][::-1]
            ggml_type = r.u32()
            offset = r.size()
            self._tensors[tname] = TensorInfo(shape, ggml_type, offset)
        alignment = self.metadata.get("general.alignment", DEFAULT_ALIGNMENT)
        unsigned = self.metadata_types.get("general.alignment", 4) in (0, 2, 4, 10)
        if (not unsigned or alignment <= 0 or alignment & (alignment - 1) or alignment > MAX_ALIGNMENT):
            raise FormatError(f"{name}: general.alignment is {alignment!r}: a power of two of at most "
                              f"{MAX_ALIGNMENT} is expected")
        self.data_start = -(-r.at // alignment) * alignment
        for tname, info in self._tensors.items():
            if info.kind is not None:
                self._range(tname)
            else:
                self._start(tname, info)

    @classmethod
    def open(cls, path):
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size == 0:
                raise FormatError(f"{path}: truncated header at byte 0")
            m = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        return cls(memoryview(m), str(path), keep=m)

    @classmethod
    def from_bytes(cls, data):
        return cls(memoryview(bytes(data)))

    def names(self):
        return sorted(self._tensors)

    def info(self, name):
        return self._tensors.get(name)

    def _start(self, name, info):
        start = self.data_start + info.offset
        if start > len(self._data):
            raise FormatError(f"{self.name}: tensor {name!r} starts beyond the file")
        return start

    def _range(self, name):
        info = self._tensors.get(name)
        if info is None:
            raise Missing(f"no tensor {name!r}")
        if info.kind is None:
            raise FormatError(f"{self.name}: tensor {name!r} has ggml type {info.ggml_type}, "
                              "which this library does not read")
        count = 1
        for d in info.shape:
            count *= d
        kind, code = info.kind
        if kind == "q":
            length = block_len(code, 0)
            if count % length:
                raise FormatError(f"{self.name}: tensor {name!r}: {count} elements in blocks of {length}")
            nbytes = count // length * block_bytes(code, 0)
        else:
            nbytes = count * _FLOAT_BYTES[code]
        start = self._start(name, info)
        if start + nbytes > len(self._data):
            raise FormatError(f"{self.name}: tensor {name!r} reaches beyond the file")
        return info, start, nbytes

    def raw(self, name):
        """The tensor's bytes in the file (no copy): numpy uint8."""
        _, start, nbytes = self._range(name)
        return np.frombuffer(self._data, dtype=np.uint8, count=nbytes, offset=start)

    def array(self, name):
        """A plain tensor as a numpy array of its shape (bf16 as uint16 bits)."""
        info, _, _ = self._range(name)
        kind, code = info.kind
        if kind != "f":
            raise InvalidArgument(f"tensor {name!r} is quantized: use quantized()")
        dt = np.uint16 if code == "bfloat16" else np.dtype(code)
        return self.raw(name).view(dt).reshape(info.shape)

    def quantized(self, name, device=None):
        """A quantized matrix [n, k] as a QuantizedTensor, its blocks copied
        unchanged (to `device` when given)."""
        import torch
        info, _, _ = self._range(name)
        kind, code = info.kind
        if kind != "q":
            raise InvalidArgument(f"tensor {name!r} is not quantized")
        if len(info.shape) != 2:
            raise InvalidArgument(f"tensor {name!r} has shape {info.shape}: [n, k] expected")
        n, k = info.shape
        data = torch.from_numpy(self.raw(name).copy())
        t = QuantizedTensor(data, code, 0, n, k)
        return t.to(device) if device is not None else t


# --------------------------------------------------------------- writing
class Entry:
    """A metadata value with its GGUF type (gguf.rs:365-452): kind is one of
    u8 i8 u16 i16 u32 i32 f32 bool string array u64 i64 f64."""
    KINDS = {"u8": (0, "<B"), "i8": (1, "<b"), "u16": (2, "<H"), "i16": (3, "<h"), "u32": (4, "<I"),
             "i32": (5, "<i"), "f32": (6, "<f"), "bool": (7, None), "string": (8, None),
             "array": (9, None), "u64": (10, "<Q"), "i64": (11, "<q"), "f64": (12, "<d")}

    def __init__(self, kind, value):
        if kind not in self.KINDS:
            raise InvalidArgument(f"unknown metadata kind {kind}")
        self.kind, self.value = kind, value

    def code(self):
        return self.KINDS[self.kind][0]

    def encode(self):
        code, fmt = self.KINDS[self.kind]
        if fmt:
            return struct.pack(fmt, self.value)
        if self.kind == "bool":
            return bytes([1 if self.value else 0])
        if self.kind == "string":
            raw = self.value.encode("utf-8")
            return struct.pack("<Q", len(raw)) + raw
        values = self.value
        inner = values[0].code() if values else 8
        if any(v.code() != inner for v in values):
            raise FormatError("an array mixes types")
        return struct.pack("<IQ", inner, len(values)) + b"".join(v.encode() for v in values)


def write(path, metadata, tensors):
    """A GGUF file (version 3): `metadata` [(key, Entry)] in order, then
    `tensors` [(name, QuantizedTensor or numpy array)], each aligned on 32
    bytes (gguf.rs:498-580)."""
    def string(s):
        raw = s.encode("utf-8")
        return struct.pack("<Q", len(raw)) + raw

    header = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    seen = set()
    for key, value in metadata:
        if key in seen:
            raise FormatError(f"key {key!r} given twice")
        seen.add(key)
        if key == "general.alignment" and not (value.kind == "u32" and value.value == DEFAULT_ALIGNMENT):
            raise FormatError("only the default alignment (32) is written")
        header += string(key) + struct.pack("<I", value.code()) + value.encode()
    blobs, offset = [], 0
    for name, t in tensors:
        if isinstance(t, QuantizedTensor):
            kind = ggml_type_of_format(t.fmt)
            if kind is None or t.group:
                raise FormatError(f"tensor {name!r}: GGUF cannot hold format {t.fmt}/{t.group}")
            shape = (t.n, t.k)
            blob = np.ascontiguousarray(t.data.cpu().numpy()).tobytes()
        else:
            arr = np.ascontiguousarray(t)
            kind = next((g for g, (kk, c) in GGML_TYPES.items() if kk == "f" and c == arr.dtype.name), None)
            if kind is None:
                raise FormatError(f"tensor {name!r}: GGUF cannot hold {arr.dtype}")
            shape = arr.shape
            blob = arr.tobytes()
        header += string(name) + struct.pack("<I", len(shape))
        header += b"".join(struct.pack("<Q", d) for d in reversed(shape))
        header += struct.pack("<IQ", kind, offset)
        blobs.append(blob)
        offset = -(-(offset + len(blob)) // DEFAULT_ALIGNMENT) * DEFAULT_ALIGNMENT
    header += bytes(-len(header) % DEFAULT_ALIGNMENT)
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(header)
        for blob in blobs:
            f.write(blob)
            f.write(bytes(-len(blob) % DEFAULT_ALIGNMENT))
    os.replace(tmp, path)


__all__ = ["Gguf", "Entry", "write", "FormatError", "Missing", "TensorInfo", "GGML_TYPES",
           "ggml_type_of_format"]
