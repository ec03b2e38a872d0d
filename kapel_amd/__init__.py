"""kapel_amd: Kapel's product by quantized weights on MI355X (gfx950).

The host side of the HIP library ``libkapel_hip.so`` (C ABI in
``include/kapel_hip.h``), shaped as the reference's interface for the path:

- ``QuantizedMatmul`` (kapel-ops/src/matmul.rs:89-156): ``infer`` refuses the
  same inputs with the same errors; ``Hip().forward(QuantizedMatmul(), [x, w...])``
  runs it on the device, as ``Run<QuantizedMatmul>::forward`` does;
- ``Hip`` (the backend, as kapel-cuda's ``Cuda`` / kapel-cpu's ``Cpu``):
  ``Hip(ordinal)``, ``with_byte_activations`` (kapel-cpu/src/backend.rs:71-81),
  ``upload`` / ``download`` (kapel-ops/src/lib.rs:146-161);
- ``quantize`` / ``dequantize``: the load-time quantizers and the codec.

PyTorch only provides device memory and streams.  There is no fallback: if the
library is not built or no GPU is present, the calls raise.
"""
import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkapel_hip.so")

# Quantized formats (include/kapel_hip.h; kapel-cuda-abi/src/lib.rs:167-194).
INT8, INT4, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4K, Q5K, Q6K = range(10)
IQ4_NL, IQ4_XS, IQ3_S = 10, 11, 12
Q2K, Q3K = 13, 14
FORMAT_NAMES = {INT8: "int8", INT4: "int4", Q8_0: "q8_0", Q4_0: "q4_0", Q4_1: "q4_1",
                Q5_0: "q5_0", Q5_1: "q5_1", Q4K: "q4_k", Q5K: "q5_k", Q6K: "q6_k",
                Q2K: "q2_k", Q3K: "q3_k", IQ4_NL: "iq4_nl", IQ4_XS: "iq4_xs", IQ3_S: "iq3_s"}
# Float types (kapel-cuda-abi/src/lib.rs:152-163).
F32, BF16, F16 = 0, 1, 2
BYTE_ACTIVATIONS = 1
BYTE_ACTIVATIONS_ALL_ROWS = 4
REUSE_ACTIVATIONS = 2

KH_OK, KH_ERR_ARITY, KH_ERR_DTYPE, KH_ERR_SHAPE, KH_ERR_MISALIGNED = 0, 1, 2, 3, 4
KH_ERR_OVERFLOW, KH_ERR_WORKSPACE, KH_ERR_HIP, KH_ERR_NULL = 5, 6, 7, 8


# ------------------------------------------------------------- errors
# The variants of kapel_core::Error (kapel-core/src/error.rs) the op returns.
class KapelError(Exception):
    pass


class Arity(KapelError):
    pass


class UnsupportedDType(KapelError):
    pass


class InvalidArgument(KapelError):
    pass


class BlockMisaligned(KapelError):
    pass


class Overflow(KapelError):
    pass


class DeviceError(KapelError):
    pass


_STATUS_ERRORS = {KH_ERR_ARITY: Arity, KH_ERR_DTYPE: UnsupportedDType,
                  KH_ERR_SHAPE: InvalidArgument, KH_ERR_MISALIGNED: BlockMisaligned,
                  KH_ERR_OVERFLOW: Overflow, KH_ERR_WORKSPACE: DeviceError,
                  KH_ERR_HIP: DeviceError, KH_ERR_NULL: InvalidArgument}


# ------------------------------------------------------------- the library
class _Weight(ctypes.Structure):
    _fields_ = [("format", ctypes.c_uint32), ("group", ctypes.c_uint32),
                ("data", ctypes.c_void_p), ("bytes", ctypes.c_uint64),
                ("n", ctypes.c_uint64)]


_lib = None

# Every entry point include/kapel_hip.h declares.
SYMBOLS = ("kh_version", "kh_error_string", "kh_block_len", "kh_block_bytes",
           "kh_qmatmul_workspace", "kh_qmatmul", "kh_quantize_x", "kh_block_dots",
           "kh_dequantize", "kh_dequantize_rows", "kh_quantize_host",
           "kh_expert_matmul_workspace", "kh_expert_matmul", "kh_qmatmul_static")


def lib():
    """The loaded libkapel_hip.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m kapel_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    u32, u64, i64, P = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p
    W = ctypes.POINTER(_Weight)
    L.kh_version.restype = ctypes.c_char_p
    L.kh_error_string.argtypes = [ctypes.c_int]
    L.kh_error_string.restype = ctypes.c_char_p
    L.kh_block_len.argtypes = [u32, u32]
    L.kh_block_len.restype = u32
    L.kh_block_bytes.argtypes = [u32, u32]
    L.kh_block_bytes.restype = u32
    L.kh_qmatmul_workspace.argtypes = [W, u32, u64, u64, u32]
    L.kh_qmatmul_workspace.restype = u64
    L.kh_qmatmul.argtypes = [W, u32, u64, u32, P, u64, u32, P, u32, P, u64, P]
    L.kh_qmatmul_static.argtypes = [W, u32, u64, u32, P, u64, u32, P, u32, P]
    L.kh_quantize_x.argtypes = [u32, P, u64, u64, P, P, P, P]
    L.kh_block_dots.argtypes = [W, u64, P, u64, P, P, u64, P]
    L.kh_dequantize.argtypes = [W, u64, u64, u64, u32, P, P]
    L.kh_dequantize_rows.argtypes = [W, u64, P, u64, u32, P, P]
    L.kh_quantize_host.argtypes = [u32, u32, P, u64, P, ctypes.c_int]
    L.kh_quantize_host.restype = i64
    L.kh_expert_matmul_workspace.argtypes = [W, u32, u64, u64, u32, u32, u32, u32]
    L.kh_expert_matmul_workspace.restype = u64
    L.kh_expert_matmul.argtypes = [W, u32, u64, u32, P, u64, u32, u32, P, u32, P, u32, P, u64, P]
    _lib = L
    return L


def _raise(status, what=""):
    if status != KH_OK:
        message = lib().kh_error_string(status).decode()
        raise _STATUS_ERRORS.get(status, KapelError)(f"{message}{': ' + what if what else ''}")


def block_len(fmt, group=0):
    """kapel-core/src/dtype.rs:140-162."""
    return lib().kh_block_len(fmt, group)


def block_bytes(fmt, group=0):
    """kapel-core/src/dtype.rs:165-187."""
    return lib().kh_block_bytes(fmt, group)


def row_bytes(fmt, group, k):
    length = block_len(fmt, group)
    if length == 0:
        raise UnsupportedDType(f"format {fmt}")
    if k % length:
        raise BlockMisaligned(f"{k} elements in blocks of {length}")
    return k // length * block_bytes(fmt, group)


def quantize(fmt, group, values, threads=None):
    """Host quantization at load time (kapel-core/src/dtype.rs:751-782;
    the K formats and Q5_0/Q5_1 by this library's encoders)."""
    values = np.ascontiguousarray(values, dtype=np.float32).ravel()
    length = block_len(fmt, group)
    if length == 0:
        raise UnsupportedDType(f"format {fmt}")
    if values.size % length:
        raise BlockMisaligned(f"{values.size} elements in blocks of {length}")
    out = np.empty(values.size // length * block_bytes(fmt, group), dtype=np.uint8)
    t = threads if threads is not None else min(32, os.cpu_count() or 1)
    n = lib().kh_quantize_host(fmt, group, values.ctypes.data, values.size, out.ctypes.data, t)
    if n < 0:
        _raise(-n)
    return out


# ------------------------------------------------------------- tensors
def _torch():
    import torch
    return torch


_FLOAT_KINDS = {}


def float_kind(dtype):
    torch = _torch()
    if not _FLOAT_KINDS:
        _FLOAT_KINDS.update({torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16})
    if dtype not in _FLOAT_KINDS:
        raise UnsupportedDType(f"activations of type {dtype}")
    return _FLOAT_KINDS[dtype]


@dataclass
class QuantizedTensor:
    """A quantized matrix [n, k]: its blocks as bytes (a torch uint8 tensor,
    on the host or the device), rows of whole blocks along k."""
    data: object
    fmt: int
    group: int
    n: int
    k: int

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def nbytes(self):
        return int(self.data.numel())

    def to(self, device):
        return QuantizedTensor(self.data.to(device), self.fmt, self.group, self.n, self.k)

    def weight(self):
        return _Weight(self.fmt, self.group, self.data.data_ptr(), self.nbytes, self.n)


def quantized(values, fmt, group=0, device=None):
    """Quantizes a float matrix [n, k] (numpy) into a QuantizedTensor."""
    torch = _torch()
    values = np.ascontiguousarray(values, dtype=np.float32)
    n, k = values.shape
    data = torch.from_numpy(quantize(fmt, group, values))
    t = QuantizedTensor(data, fmt, group, n, k)
    return t.to(device) if device is not None else t


class QuantizedMatmul:
    """y[..., n] = sum_k x[..., k] w[n, k], several weights stacked
    (kapel-ops/src/matmul.rs:89-156)."""

    NAME = "quantized_matmul"

    def infer(self, inputs):
        """Shape and type of the output, or the reference's error
        (kapel-ops/src/matmul.rs:105-150)."""
        if len(inputs) < 2:
            raise Arity(f"{self.NAME}: expected 2 or more inputs, got {len(inputs)}")
        x = inputs[0]
        devices = {str(t.data.device) if isinstance(t, QuantizedTensor) else str(t.device)
                   for t in inputs}
        if len(devices) > 1:
            raise InvalidArgument(f"{self.NAME}: inputs on several devices {sorted(devices)}")
        float_kind(x.dtype)
        k = x.shape[-1] if x.dim() > 0 else None
        n = 0
        for w in inputs[1:]:
            if not isinstance(w, QuantizedTensor):
                raise UnsupportedDType(f"{self.NAME}: weights of type {getattr(w, 'dtype', w)}")
            if k is None or w.k != k:
                raise InvalidArgument(
                    f"expected x [..., K] and w [N, K], got {tuple(x.shape)} and {w.shape}")
            length = block_len(w.fmt, w.group)
            if length == 0:
                raise UnsupportedDType(f"{self.NAME}: format {w.fmt}")
            if w.k % length:
                raise BlockMisaligned(f"{w.k} elements in blocks of {length}")
            if w.nbytes != w.n * row_bytes(w.fmt, w.group, w.k):
                raise InvalidArgument(f"{self.NAME}: {w.nbytes} bytes for {w.shape}")
            n += w.n
        return tuple(x.shape[:-1]) + (n,), x.dtype


class IndexOutOfRange(KapelError):
    pass


class ExpertMatmul:
    """The product of each token by its experts (kapel-ops/src/experts.rs:
    130-229): x [T, K] or [T, k, K], the experts' weights stacked
    [E N, K] (one QuantizedTensor), idx [T, k] integers; y [T, k, N] in x's
    type, y[t, j, n] = sum_i x[t, (j,) i] w[idx[t, j] N + n, i]."""

    NAME = "expert_matmul"

    def __init__(self, experts):
        self.experts = int(experts)

    def infer(self, inputs):
        """Shape and type of the output, or the reference's error
        (kapel-ops/src/experts.rs:166-225)."""
        if len(inputs) != 3:
            raise Arity(f"{self.NAME}: expected 3 inputs, got {len(inputs)}")
        x, w, idx = inputs
        devices = {str(t.data.device) if isinstance(t, QuantizedTensor) else str(t.device)
                   for t in inputs}
        if len(devices) > 1:
            raise InvalidArgument(f"{self.NAME}: inputs on several devices {sorted(devices)}")
        float_kind(x.dtype)
        if idx.dtype.is_floating_point or idx.dim() != 2:
            raise InvalidArgument(f"{self.NAME}: the experts must be integers [T, k]")
        if not isinstance(w, QuantizedTensor):
            raise UnsupportedDType(f"{self.NAME}: weights of type {getattr(w, 'dtype', w)}")
        t, k = idx.shape
        width = w.k
        if tuple(x.shape) not in ((t, width), (t, k, width)):
            raise InvalidArgument(f"inputs {tuple(x.shape)} for experts {tuple(idx.shape)} and "
                                  f"weights {w.shape}: [T, K] or [T, k, K]")
        if self.experts == 0 or w.n % self.experts:
            raise InvalidArgument(f"{w.n} rows of weights for {self.experts} experts")
        length = block_len(w.fmt, w.group)
        if length == 0:
            raise UnsupportedDType(f"{self.NAME}: format {w.fmt}")
        if width % length:
            raise BlockMisaligned(f"{width} elements in blocks of {length}")
        return (t, k, w.n // self.experts), x.dtype

    def check(self, idx):
        """experts.rs:151-163: the first index out of range is an error."""
        bad = [int(i) for i in idx if int(i) >= self.experts or int(i) < 0]
        if bad:
            raise IndexOutOfRange(f"{self.NAME}: index {bad[0]} of {self.experts}")


class Hip:
    """The HIP backend of the path: one per device ordinal, one stream (the
    current torch stream of that device), a workspace kept between calls."""

    def __init__(self, ordinal=0):
        torch = _torch()
        if not torch.cuda.is_available():
            raise DeviceError("no HIP device")
        self.device = torch.device("cuda", ordinal)
        self.byte_activations = False
        self.byte_rows_all = False
        self._workspace = None
        lib()

    def with_byte_activations(self, on=True, all_rows=False):
        """kapel-cpu/src/backend.rs:71-81: activations quantized to bytes by
        blocks of 32 in the products by quantized weights, for x of up to 16
        rows as kapel-cpu/src/matmul.rs:292-306 (more rows: f32).  all_rows:
        bytes at every row count (KH_BYTE_ACTIVATIONS_ALL_ROWS, the int8 MFMA
        product of batched decode and prefill; not a mode of the reference)."""
        self.byte_activations = bool(on)
        self.byte_rows_all = bool(on) and bool(all_rows)
        return self

    def _flags(self):
        if self.byte_rows_all:
            return BYTE_ACTIVATIONS_ALL_ROWS
        return BYTE_ACTIVATIONS if self.byte_activations else 0

    def upload(self, t):
        if isinstance(t, QuantizedTensor):
            return t.to(self.device)
        return t.to(self.device)

    def download(self, t):
        return t.cpu()

    def workspace(self, size):
        torch = _torch()
        if self._workspace is None or self._workspace.numel() < size:
            # Zero-filled once: the library leaves it reusable after every call.
            self._workspace = torch.zeros(max(size, 1 << 20), dtype=torch.uint8, device=self.device)
        return self._workspace

    def stream(self):
        return _torch().cuda.current_stream(self.device).cuda_stream

    def forward(self, op, inputs, out=None, reuse_activations=False, check_indices=True):
        """Run<QuantizedMatmul>::forward (or Run<ExpertMatmul>): the product
        on the device."""
        if isinstance(op, ExpertMatmul):
            return self._experts(op, inputs, out, check_indices)
        if not isinstance(op, QuantizedMatmul):
            raise UnsupportedDType(f"op {op}")
        torch = _torch()
        shape, dtype = op.infer(inputs)
        x = inputs[0].contiguous()
        weights = inputs[1:]
        for w in weights:
            if w.data.device != self.device and w.n * w.k > 0:
                raise InvalidArgument(f"weights on {w.data.device}, backend on {self.device}")
        k = weights[0].k
        rows = 1
        for s in shape[:-1]:
            rows *= s
        if out is None:
            out = torch.empty(shape, dtype=dtype, device=self.device)
        array = (_Weight * len(weights))(*[w.weight() for w in weights])
        flags = self._flags()
        size = lib().kh_qmatmul_workspace(array, len(weights), k, rows, flags)
        if reuse_activations:
            flags |= REUSE_ACTIVATIONS
        ws = self.workspace(size)
        status = lib().kh_qmatmul(array, len(weights), k, float_kind(x.dtype),
                                  x.data_ptr() if x.numel() else None, rows, float_kind(dtype),
                                  out.data_ptr() if out.numel() else None, flags, ws.data_ptr(),
                                  ws.numel(), self.stream())
        _raise(status)
        return out

    def _experts(self, op, inputs, out, check_indices):
        """kapel-cuda/src/experts.rs:127-250: the indices read (and checked)
        as the reference's backends do; without the check (check_indices
        False) an index out of range gives NaN for its route, the device
        never faults."""
        torch = _torch()
        shape, dtype = op.infer(inputs)
        x, w, idx = inputs
        if check_indices:
            op.check(idx.reshape(-1).tolist())
        x = x.contiguous()
        if w.data.device != self.device and w.n * w.k > 0:
            raise InvalidArgument(f"weights on {w.data.device}, backend on {self.device}")
        tokens, topk = idx.shape
        per_route = 1 if x.dim() == 3 else 0
        idx32 = idx.to(self.device, torch.int32).contiguous()
        if out is None:
            out = torch.empty(shape, dtype=dtype, device=self.device)
        weight = w.weight()
        flags = BYTE_ACTIVATIONS if self.byte_activations else 0
        size = lib().kh_expert_matmul_workspace(ctypes.byref(weight), op.experts, w.k, tokens, topk,
                                                per_route, float_kind(x.dtype), flags)
        ws = self.workspace(size)
        _raise(lib().kh_expert_matmul(ctypes.byref(weight), op.experts, w.k, float_kind(x.dtype),
                                      x.data_ptr() if x.numel() else None, tokens, topk, per_route,
                                      idx32.data_ptr() if idx32.numel() else None, float_kind(dtype),
                                      out.data_ptr() if out.numel() else None, flags, ws.data_ptr(),
                                      ws.numel(), self.stream()))
        return out

    # -- the pieces, exposed for the parity checks ---------------------------
    def quantize_x(self, x):
        """bytes.rs:144-158 on the device: (q i8, scale f32, sums32 f32)."""
        torch = _torch()
        x = x.contiguous()
        rows, k = x.shape
        q = torch.empty((rows, k), dtype=torch.int8, device=self.device)
        s = torch.empty((rows, k // 32), dtype=torch.float32, device=self.device)
        sums = torch.empty((rows, k // 32), dtype=torch.float32, device=self.device)
        _raise(lib().kh_quantize_x(float_kind(x.dtype), x.data_ptr(), rows, k, q.data_ptr(),
                                   s.data_ptr(), sums.data_ptr(), self.stream()))
        return q, s, sums

    def block_dots(self, w, q):
        """The i32 block dots [rows, n, k/16] of the byte product."""
        torch = _torch()
        rows, k = q.shape
        weight = w.weight()
        size = lib().kh_qmatmul_workspace(ctypes.byref(weight), 1, k, rows, BYTE_ACTIVATIONS)
        ws = self.workspace(size)
        dots = torch.zeros((rows, w.n, k // 16), dtype=torch.int32, device=self.device)
        _raise(lib().kh_block_dots(ctypes.byref(weight), k, q.contiguous().data_ptr(), rows,
                                   dots.data_ptr(), ws.data_ptr(), ws.numel(), self.stream()))
        return dots

    def dequantize(self, w, first=0, count=None, dtype=None):
        """kernels/src/lib.rs:3745: rows first .. first + count, as floats."""
        torch = _torch()
        count = w.n - first if count is None else count
        dtype = dtype or torch.float32
        out = torch.empty((count, w.k), dtype=dtype, device=self.device)
        weight = w.weight()
        _raise(lib().kh_dequantize(ctypes.byref(weight), w.k, first, count, float_kind(dtype),
                                   out.data_ptr(), self.stream()))
        return out

    def dequantize_rows(self, w, indices, dtype=None):
        """kernels/src/lib.rs:3773: gathered rows of a quantized table."""
        torch = _torch()
        dtype = dtype or torch.float32
        indices = indices.to(self.device, torch.int32).contiguous()
        out = torch.empty((indices.numel(), w.k), dtype=dtype, device=self.device)
        weight = w.weight()
        _raise(lib().kh_dequantize_rows(ctypes.byref(weight), w.k, indices.data_ptr(),
                                        indices.numel(), float_kind(dtype), out.data_ptr(),
                                        self.stream()))
        return out
