"""ctypes face of the oracle (TEST INFRASTRUCTURE ONLY).

The C restatement in ``kapel_oracle.c`` of the reference's CPU path is the
checker of the HIP library.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` import this module; the product never
does.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkapel_oracle.so")

# Format codes of kapel-cuda-abi/src/lib.rs:167-194, plus Q2_K and Q3_K.
INT8, INT4, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4K, Q5K, Q6K = range(10)
IQ4_NL, IQ4_XS, IQ3_S = 10, 11, 12
Q2K, Q3K = 13, 14

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: run `make -C {HERE}`")
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, u32 = ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
        P = ctypes.c_void_p
        L.ko_block_len.argtypes = [i32, i32]
        L.ko_block_bytes.argtypes = [i32, i32]
        L.ko_f16_decode.argtypes = [u32]
        L.ko_f16_decode.restype = ctypes.c_double
        L.ko_f16_encode.argtypes = [ctypes.c_double]
        L.ko_f16_encode.restype = u32
        L.ko_half_f32.argtypes = [u32]
        L.ko_half_f32.restype = ctypes.c_float
        L.ko_dequantize.argtypes = [i32, i32, P, i64, P]
        L.ko_quantize.argtypes = [i32, i32, P, i64, P]
        L.ko_quantize.restype = i64
        L.ko_decode_f32.argtypes = [i32, i32, P, P]
        L.ko_product_f32.argtypes = [i32, P, P, P, P, i64, P, i64, P, i32]
        L.ko_product_bytes.argtypes = [i32, P, P, P, P, i64, P, P, i64, P, P, i32]
        L.ko_product_f64.argtypes = [i32, P, P, P, P, i64, P, i64, P]
        L.ko_quantize_x.argtypes = [P, i64, i64, P, P, P]
        L.ko_bytes_layout.argtypes = [i32, i32, P, P, P, P]
        L.ko_iq_table.argtypes = [i32, i32]
        L.ko_iq_table.restype = i64
        L.ko_wide_available.argtypes = []
        L.ko_wide_product_f32.argtypes = [i32, P, P, P, P, i64, P, i64, P, i32]
        L.ko_vnni_product_bytes.argtypes = [i32, P, P, P, P, i64, P, P, P, i64, P, i32]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def block_len(fmt, group=0):
    return lib().ko_block_len(fmt, group)


def block_bytes(fmt, group=0):
    return lib().ko_block_bytes(fmt, group)


def row_bytes(fmt, group, k):
    return k // block_len(fmt, group) * block_bytes(fmt, group)


def f16_decode(bits):
    return lib().ko_f16_decode(int(bits))


def f16_encode(x):
    return lib().ko_f16_encode(float(x))


def half_f32(bits):
    return lib().ko_half_f32(int(bits))


def dequantize(fmt, group, data):
    """The exact f64 value of every element (kapel-core/src/dtype.rs:342)."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    size, length = block_bytes(fmt, group), block_len(fmt, group)
    assert data.size % size == 0
    blocks = data.size // size
    out = np.empty(blocks * length, dtype=np.float64)
    rc = lib().ko_dequantize(fmt, group, _p(data), blocks, _p(out))
    assert rc == 0, rc
    return out


def quantize(fmt, group, values):
    """The reference quantizers (dtype.rs:751-782): int8, int4, Q8_0, Q4_0, Q4_1."""
    values = np.ascontiguousarray(values, dtype=np.float32).ravel()
    length = block_len(fmt, group)
    out = np.empty(values.size // length * block_bytes(fmt, group), dtype=np.uint8)
    n = lib().ko_quantize(fmt, group, _p(values), values.size, _p(out))
    assert n == out.size, n
    return out


def iq_table(which, index):
    """0: IQ4_NL's 16 values; 1: IQ3_S's grid of 512 (-1 past the end)."""
    return lib().ko_iq_table(which, index)


def decode_f32(fmt, group, block):
    block = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.empty(block_len(fmt, group), dtype=np.float32)
    assert lib().ko_decode_f32(fmt, group, _p(block), _p(out)) == 0
    return out


def _weights(weights):
    count = len(weights)
    fmts = np.array([w[0] for w in weights], dtype=np.int32)
    groups = np.array([w[1] for w in weights], dtype=np.int32)
    datas = [np.ascontiguousarray(w[2], dtype=np.uint8) for w in weights]
    ptrs = np.array([d.ctypes.data for d in datas], dtype=np.uint64)
    ns = np.array([w[3] for w in weights], dtype=np.int64)
    return count, fmts, groups, datas, ptrs, ns


def product_f32(weights, k, x, threads=1):
    """kapel-cpu's in-place product (quantized.rs:117-175), f32 activations.

    ``weights``: list of (fmt, group, bytes, n).  ``x``: [rows, k] f32."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k) if k else np.zeros((x.shape[0], 0), np.float32)
    count, fmts, groups, datas, ptrs, ns = _weights(weights)
    out = np.zeros((x.shape[0], int(ns.sum())), dtype=np.float32)
    rc = lib().ko_product_f32(count, _p(fmts), _p(groups), _p(ptrs), _p(ns), k, _p(x), x.shape[0],
                              _p(out), threads)
    assert rc == 0, rc
    return out


def product_f64(weights, k, x):
    """kapel-ref's product (kapel-ref/src/matmul.rs:96-117) in f64."""
    x = np.ascontiguousarray(x, dtype=np.float64).reshape(-1, k) if k else np.zeros((x.shape[0], 0))
    count, fmts, groups, datas, ptrs, ns = _weights(weights)
    out = np.zeros((x.shape[0], int(ns.sum())), dtype=np.float64)
    rc = lib().ko_product_f64(count, _p(fmts), _p(groups), _p(ptrs), _p(ns), k, _p(x), x.shape[0],
                              _p(out))
    assert rc == 0, rc
    return out


def wide_available():
    """(AVX-512, AVX-512 VNNI) on this host, as kapel-cpu detects them
    (kapel-cpu/src/isa.rs:20-35, bytes.rs:89)."""
    bits = lib().ko_wide_available()
    return bool(bits & 1), bool(bits & 2)


WIDE_FORMATS = (Q8_0, Q4_0, Q4K, Q6K)  # the formats of the restated AVX-512 kernels


def product_wide(weights, k, x, threads=1):
    """kapel-cpu's product with its AVX-512 kernels (quantized.rs:699-1021,
    `wide::fused`), f32 activations; None where this host or a format does
    not take them."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    count, fmts, groups, datas, ptrs, ns = _weights(weights)
    out = np.zeros((x.shape[0], int(ns.sum())), dtype=np.float32)
    rc = lib().ko_wide_product_f32(count, _p(fmts), _p(groups), _p(ptrs), _p(ns), k, _p(x),
                                   x.shape[0], _p(out), threads)
    if rc == -2:
        return None
    assert rc == 0, rc
    return out


def product_vnni(weights, k, x=None, threads=1, prepared=None):
    """kapel-cpu's byte-activation product with its AVX-512 VNNI kernels
    (bytes.rs:395-652); ``prepared`` = quantize_x(x) to skip that step.  None
    where this host or a format does not take them."""
    q, s, sums = prepared if prepared is not None else quantize_x(np.asarray(x, np.float32).reshape(-1, k))
    count, fmts, groups, datas, ptrs, ns = _weights(weights)
    out = np.zeros((q.shape[0], int(ns.sum())), dtype=np.float32)
    rc = lib().ko_vnni_product_bytes(count, _p(fmts), _p(groups), _p(ptrs), _p(ns), k, _p(q), _p(s),
                                     _p(sums), q.shape[0], _p(out), threads)
    if rc == -2:
        return None
    assert rc == 0, rc
    return out


def quantize_x(x):
    """Activations to bytes (bytes.rs:144-158): (q i8 [rows,k], scale f32
    [rows,k/32], sums32 f32 [rows,k/32] = scale * sum(q))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    q = np.empty((rows, k), dtype=np.int8)
    s = np.empty((rows, k // 32), dtype=np.float32)
    sums = np.empty((rows, k // 32), dtype=np.float32)
    lib().ko_quantize_x(_p(x), rows, k, _p(q), _p(s), _p(sums))
    return q, s, sums


def bytes_supported(fmt, group=0):
    a = np.zeros(4, dtype=np.int32)
    return bool(lib().ko_bytes_layout(fmt, group, _p(a[0:]), _p(a[1:]), _p(a[2:]), _p(a[3:])))


def product_bytes(weights, k, x, threads=1, with_dots=False):
    """kapel-cpu's byte-activation product (bytes.rs:168-242, portable :356-394).

    Returns out [rows, width] f32 and, with ``with_dots``, the i32 block dots
    [rows, width, k/16] (a dot over 32 elements at its even slot)."""
    q, s, _ = quantize_x(np.asarray(x, dtype=np.float32).reshape(-1, k))
    count, fmts, groups, datas, ptrs, ns = _weights(weights)
    rows, width = q.shape[0], int(ns.sum())
    out = np.zeros((rows, width), dtype=np.float32)
    dots = np.zeros((rows, width, k // 16), dtype=np.int32) if with_dots else None
    rc = lib().ko_product_bytes(count, _p(fmts), _p(groups), _p(ptrs), _p(ns), k, _p(q), _p(s),
                                rows, _p(out), _p(dots) if with_dots else None, threads)
    assert rc == 0, rc
    return (out, dots) if with_dots else out


def expert_product(fmt, group, data, experts, k, x, idx, byte_activations=False, threads=1):
    """kapel-cpu's experts' product (kapel-cpu/src/experts.rs:62-110): the
    routes of each expert gathered in route order, multiplied by its rows in
    one product (the f32 product, or the byte one where the format has it),
    each result row put back at its route.  ``x`` [T, K] or [T, topk, K],
    ``idx`` [T, topk] (every index below ``experts``); returns [T, topk, N].
    """
    idx = np.asarray(idx).reshape(np.shape(idx)[0], -1)
    tokens, topk = idx.shape
    x = np.asarray(x, dtype=np.float32)
    per_route = x.ndim == 3
    rows_of = x.reshape(-1, k)
    data = np.ascontiguousarray(data, dtype=np.uint8)
    n = data.size // row_bytes(fmt, group, k) // experts if k else 0
    size = n * row_bytes(fmt, group, k)
    out = np.zeros((tokens * topk, n), dtype=np.float32)
    flat = idx.reshape(-1)
    use_bytes = byte_activations and bytes_supported(fmt, group)
    for e in range(experts):
        routes = [r for r in range(tokens * topk) if flat[r] == e]
        if not routes or n == 0:
            continue
        rows = rows_of[[r if per_route else r // topk for r in routes]]
        w = [(fmt, group, data[e * size:(e + 1) * size], n)]
        y = product_bytes(w, k, rows, threads) if use_bytes else product_f32(w, k, rows, threads)
        out[routes] = y
    return out.reshape(tokens, topk, n)
