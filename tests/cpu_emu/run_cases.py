"""Runs the product's kernels, built for the host (libkapel_hip_emu.so), on
the cases of the GPU parity tests, under AddressSanitizer, and checks them
against the oracle.  Started by tests/test_emulated.py with the ASan runtime
preloaded; prints one line per case and exits non-zero on a mismatch.

    python tests/cpu_emu/run_cases.py [quick|all]
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.dirname(HERE)]

import oracle as ko  # noqa: E402
from refrng import Rng, lcg_bytes  # noqa: E402

INT8, INT4, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4K, Q5K, Q6K = range(10)
IQ4_NL, IQ4_XS, IQ3_S = 10, 11, 12
Q2K, Q3K = 13, 14
F32, BF16, F16 = 0, 1, 2


class W(ctypes.Structure):
    _fields_ = [("format", ctypes.c_uint32), ("group", ctypes.c_uint32),
                ("data", ctypes.c_void_p), ("bytes", ctypes.c_uint64), ("n", ctypes.c_uint64)]


L = ctypes.CDLL(os.path.join(HERE, "libkapel_hip_emu.so"))
u32, u64, P = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p
L.kh_qmatmul_workspace.argtypes = [ctypes.POINTER(W), u32, u64, u64, u32]
L.kh_qmatmul_workspace.restype = u64
L.kh_qmatmul.argtypes = [ctypes.POINTER(W), u32, u64, u32, P, u64, u32, P, u32, P, u64, P]
L.kh_block_dots.argtypes = [ctypes.POINTER(W), u64, P, u64, P, P, u64, P]
L.kh_quantize_x.argtypes = [u32, P, u64, u64, P, P, P, P]
L.kh_dequantize.argtypes = [ctypes.POINTER(W), u64, u64, u64, u32, P, P]
L.kh_expert_matmul.argtypes = [ctypes.POINTER(W), u32, u64, u32, P, u64, u32, u32, P, u32, P, u32, P, u64, P]

HALVES = {Q8_0: [0], Q4_0: [0], Q5_0: [0], Q4_1: [0, 2], Q5_1: [0, 2], Q4K: [0, 2], Q5K: [0, 2],
          Q2K: [80, 82], Q3K: [108], Q6K: [208], IQ4_NL: [0], IQ4_XS: [0], IQ3_S: [0]}
FAILED = []


def blocks(fmt, group, count, seed):
    nxt = lcg_bytes(seed)
    size = ko.block_bytes(fmt, group)
    raw = np.frombuffer(bytes(nxt() for _ in range(count * size)), dtype=np.uint8).copy()
    raw = raw.reshape(count, size)
    rng = np.random.default_rng(seed)
    for at in HALVES.get(fmt, []):
        h = np.array([ko.f16_encode(v) for v in rng.uniform(0.005, 0.02, count)], dtype=np.uint16)
        raw[:, at:at + 2] = h.view(np.uint8).reshape(count, 2)
    if fmt in (INT8, INT4):
        raw[:, :4] = np.frombuffer(rng.uniform(0.005, 0.02, count).astype(np.float32).tobytes(),
                                   dtype=np.uint8).reshape(count, 4)
    # The device reads a matrix by whole dwords: the last one may extend two
    # bytes past an odd-halfword end, inside the same dword (never a fault on
    # the device); the host allocation keeps those bytes addressable.
    padded = np.zeros(count * size + 4, np.uint8)
    padded[:count * size] = raw.ravel()
    return padded[:count * size]


def xs(rows, k, seed):
    rng = Rng(seed)
    return np.array([[rng.uniform(-1, 1) for _ in range(k)] for _ in range(rows)], np.float32)


def aligned(nbytes):
    """A zeroed byte buffer at a 256-byte aligned address."""
    raw = np.zeros(nbytes + 256, np.uint8)
    off = (-raw.ctypes.data) % 256
    return raw[off:off + nbytes]


# One workspace for every case, as a caller keeps one: each call must leave it
# ready for the next, whatever the shapes.
WORKSPACE = aligned(64 << 20)


def workspace(size):
    assert size <= WORKSPACE.size
    return WORKSPACE


def product(parts, k, x, flags=0):
    arr = (W * len(parts))(*[W(f, g, d.ctypes.data, d.size, n) for f, g, d, n in parts])
    rows = x.shape[0]
    width = sum(p[3] for p in parts)
    size = L.kh_qmatmul_workspace(arr, len(parts), k, rows, flags)
    ws = workspace(size)
    out = np.full((rows, width), np.nan, np.float32)
    st = L.kh_qmatmul(arr, len(parts), k, F32, x.ctypes.data, rows, F32, out.ctypes.data, flags,
                      ws.ctypes.data, ws.size, None)
    assert st == 0, st
    return out


def report(name, ok):
    print(("ok   " if ok else "FAIL ") + name, flush=True)
    if not ok:
        FAILED.append(name)


def check_f32(name, got, e64):
    ok = bool(np.all(np.abs(got.astype(np.float64) - e64) <= 1e-4 * (1 + np.abs(e64))))
    report(name, ok)


def case_product(fmt, group, n, k, rows, seed=5):
    d = blocks(fmt, group, n * k // ko.block_len(fmt, group), seed + fmt)
    x = xs(rows, k, 100 + rows)
    got = product([(fmt, group, d, n)], k, x)
    check_f32(f"product fmt {fmt}/{group} n {n} k {k} rows {rows}", got,
              ko.product_f64([(fmt, group, d, n)], k, x))


def case_float_kinds(fmt, group, n, k, rows, kind, seed=7, kernel=None):
    """The many-row product with bf16, f16 or f32 activations (f32 out),
    against the f64 product of the activations as given; `kernel` forces the
    float or the int8 many-row kernel (KH_MANY_KERNEL)."""
    d = blocks(fmt, group, n * k // ko.block_len(fmt, group), seed + fmt)
    x = xs(rows, k, 200 + rows)
    if kind == BF16:
        xb = (x.view(np.uint32) >> 16).astype(np.uint16)
        x = (xb.astype(np.uint32) << 16).view(np.float32)
    elif kind == F16:
        xb = x.astype(np.float16).view(np.uint16)
        x = xb.view(np.float16).astype(np.float32)
    else:
        xb = x
    arr = (W * 1)(W(fmt, group, d.ctypes.data, d.size, n))
    ws = workspace(L.kh_qmatmul_workspace(arr, 1, k, rows, 0))
    out = np.full((rows, n), np.nan, np.float32)
    if kernel:
        os.environ["KH_MANY_KERNEL"] = kernel
    try:
        st = L.kh_qmatmul(arr, 1, k, kind, xb.ctypes.data, rows, F32, out.ctypes.data, 0,
                          ws.ctypes.data, ws.size, None)
    finally:
        os.environ.pop("KH_MANY_KERNEL", None)
    assert st == 0, st
    check_f32(f"many rows fmt {fmt}/{group} n {n} k {k} rows {rows} kind {kind} {kernel or ''}", out,
              ko.product_f64([(fmt, group, d, n)], k, x))


def case_bytes(fmt, group, n, k, rows, dots=True):
    d = blocks(fmt, group, n * k // ko.block_len(fmt, group), 3)
    i = np.arange(rows * k)
    x = ((((i * 7919) % 201).astype(np.float32) / np.float32(100.0) - np.float32(1.0))
         * (1 + (i // 32) % 7).astype(np.float32)).reshape(rows, k)
    out_cpu, dots_cpu = ko.product_bytes([(fmt, group, d, n)], k, x, with_dots=True)
    q, s, _ = ko.quantize_x(x)
    w = W(fmt, group, d.ctypes.data, d.size, n)
    flags = 1 if rows <= 16 else 4  # bytes above 16 rows: KH_BYTE_ACTIVATIONS_ALL_ROWS
    size = L.kh_qmatmul_workspace(ctypes.byref(w), 1, k, rows, flags)
    ws = workspace(size)
    if dots:
        dots = np.zeros((rows, n, k // 16), np.int32)
        assert L.kh_block_dots(ctypes.byref(w), k, q.ctypes.data, rows, dots.ctypes.data,
                               ws.ctypes.data, ws.size, None) == 0
        report(f"dots fmt {fmt}/{group} rows {rows}", bool(np.array_equal(dots, dots_cpu)))
    got = product([(fmt, group, d, n)], k, x, flags=flags).astype(np.float64)
    dense = ko.dequantize(fmt, group, d).reshape(n, k)
    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    e = xq @ dense.T
    size = np.abs(xq) @ np.abs(dense).T
    report(f"bytes fmt {fmt}/{group} rows {rows}", bool(np.all(np.abs(got - e) <= 1e-5 * size + 1e-6)))


def case_stalled_wait():
    """The small-M kernel's bounded wait for its activations, forced to
    give up (KH_SPIN_LIMIT negative): every output NaN, none wrong; then the
    normal wait again gives the product."""
    d = blocks(Q4K, 0, 20 * 1024 // 256, 9)
    x = xs(3, 1024, 4)
    os.environ["KH_SPIN_LIMIT"] = "-1"
    try:
        got = product([(Q4K, 0, d, 20)], 1024, x)
    finally:
        del os.environ["KH_SPIN_LIMIT"]
    report("stalled wait: NaN outputs", bool(np.isnan(got).all()))
    check_f32("after a stalled wait", product([(Q4K, 0, d, 20)], 1024, x),
              ko.product_f64([(Q4K, 0, d, 20)], 1024, x))


def case_kinds():
    """bf16 / f16 activations and outputs, and the empty shapes."""
    n, k = 20, 512
    d = blocks(Q4K, 0, n * k // 256, 9)
    x = xs(2, k, 3)
    w = (W * 1)(W(Q4K, 0, d.ctypes.data, d.size, n))
    for kind in (BF16, F16):
        if kind == BF16:
            xb = (x.view(np.uint32) >> 16).astype(np.uint16)
            xf = (xb.astype(np.uint32) << 16).view(np.float32)
        else:
            xb = x.astype(np.float16).view(np.uint16)
            xf = xb.view(np.float16).astype(np.float32)
        size = L.kh_qmatmul_workspace(w, 1, k, 2, 0)
        ws = workspace(size)
        out = np.zeros((2, n), np.uint16)
        assert L.kh_qmatmul(w, 1, k, kind, xb.ctypes.data, 2, kind, out.ctypes.data, 0,
                            ws.ctypes.data, ws.size, None) == 0
        got = ((out.astype(np.uint32) << 16).view(np.float32) if kind == BF16
               else out.view(np.float16).astype(np.float32))
        e = ko.product_f64([(Q4K, 0, d, n)], k, xf)
        tol = 5e-2 if kind == BF16 else 1e-2
        report(f"kind {kind}", bool(np.all(np.abs(got - e) <= tol * max(1, np.abs(e).max()))))
    # K = 0: zeros.
    w0 = (W * 1)(W(Q8_0, 0, None, 0, 5))
    out = np.full((3, 5), 7.0, np.float32)
    assert L.kh_qmatmul(w0, 1, 0, F32, None, 3, F32, out.ctypes.data, 0, None, 0, None) == 0
    report("k = 0", bool(np.all(out == 0)))


def case_experts(fmt, group, n, k, experts, tokens, topk, per_route, flags=0):
    """The experts' product against the oracle's (kapel-cpu/src/experts.rs:62-110);
    an index past the experts gives NaN for its route."""
    d = blocks(fmt, group, experts * n * k // ko.block_len(fmt, group), 9 + fmt)
    rng = np.random.default_rng(tokens)
    idx = rng.integers(0, experts, size=(tokens, topk)).astype(np.uint32)
    shape = (tokens, topk, k) if per_route else (tokens, k)
    x = np.ascontiguousarray(rng.uniform(-1, 1, size=shape).astype(np.float32))
    w = W(fmt, group, d.ctypes.data, d.size, experts * n)
    bad = idx.copy()
    bad[0, 0] = experts
    out = np.zeros((tokens, topk, n), np.float32)
    st = L.kh_expert_matmul(ctypes.byref(w), experts, k, F32, x.ctypes.data, tokens, topk, int(per_route),
                            bad.ctypes.data, F32, out.ctypes.data, flags, WORKSPACE.ctypes.data,
                            WORKSPACE.size, None)
    assert st == 0, st
    want = ko.expert_product(fmt, group, d, experts, k, x, idx, byte_activations=bool(flags))
    name = f"experts fmt {fmt}/{group} n {n} k {k} {tokens}x{topk} of {experts} per_route {per_route} flags {flags}"
    ok = bool(np.all(np.isnan(out[0, 0])))
    tol = 1e-4 * (1 + np.abs(want)) if not flags else 2e-4 * (1 + np.abs(want))
    rest = np.ones((tokens, topk), bool)
    rest[0, 0] = False
    ok = ok and bool(np.all(np.abs(out[rest] - want[rest]) <= tol[rest]))
    report(name, ok)


def case_quantize_x():
    x = xs(3, 256, 4)
    x[0, :32] = 0
    q = np.zeros((3, 256), np.int8)
    s = np.zeros((3, 8), np.float32)
    sums = np.zeros((3, 8), np.float32)
    assert L.kh_quantize_x(F32, x.ctypes.data, 3, 256, q.ctypes.data, s.ctypes.data,
                           sums.ctypes.data, None) == 0
    oq, os_, osums = ko.quantize_x(x)
    report("quantize_x", bool(np.array_equal(q, oq) and np.array_equal(s, os_)
                              and np.array_equal(sums, osums)))


def case_dequantize(fmt, group):
    n, k = 3, 520 if group == 40 else 512
    d = blocks(fmt, group, n * k // ko.block_len(fmt, group), 21)
    w = W(fmt, group, d.ctypes.data, d.size, n)
    out = np.zeros((n, k), np.float32)
    assert L.kh_dequantize(ctypes.byref(w), k, 0, n, F32, out.ctypes.data, None) == 0
    size, length = ko.block_bytes(fmt, group), ko.block_len(fmt, group)
    want = np.concatenate([ko.decode_f32(fmt, group, d[i * size:(i + 1) * size])
                           for i in range(n * k // length)]).reshape(n, k)
    report(f"dequantize fmt {fmt}/{group}", bool(np.array_equal(out.view(np.uint32), want.view(np.uint32))))


FORMATS = [(INT8, 32), (INT8, 64), (INT8, 40), (INT8, 128), (INT4, 32), (INT4, 64), (INT4, 128),
           (INT4, 40), (Q8_0, 0), (Q4_0, 0), (Q4_1, 0), (Q5_0, 0), (Q5_1, 0), (Q2K, 0), (Q3K, 0),
           (Q4K, 0), (Q5K, 0), (Q6K, 0), (IQ4_NL, 0), (IQ4_XS, 0), (IQ3_S, 0)]
BYTE_FORMATS = [(Q8_0, 0), (Q4_0, 0), (Q4K, 0), (Q5K, 0), (Q6K, 0), (INT8, 32), (INT8, 128),
                (INT4, 32), (INT4, 64)]


def main(which):
    case_product(INT8, 32, 7, 1280, 1)  # the first case of the GPU tests
    for rows in (1, 3, 17):             # then more rows, then another shape
        case_product(INT8, 32, 7, 1280, rows)
    case_product(INT8, 64, 7, 1280, 1)
    case_quantize_x()
    case_kinds()
    case_stalled_wait()
    for fmt, group in FORMATS:
        case_product(fmt, group, 7, 1280, 1)
        case_dequantize(fmt, group)
    case_product(Q8_0, 0, 5, 96, 2)        # K % 64 == 32: a step of one block
    case_product(Q4K, 0, 100, 2048, 2)      # several tiles and workgroups
    case_product(Q6K, 0, 33, 1024, 3)
    case_product(Q4K, 0, 40, 4096, 1)       # decode: K split over 4 workgroups
    case_product(Q6K, 0, 48, 8192, 1)       # decode: K split over 8 workgroups
    # The streamed decode kernel (launches of eight or more rounds of the
    # emulator's two CUs): one wave a tile, each walking several tiles
    # through a ring of whole units smaller than its stream.
    case_product(Q6K, 0, 600, 1024, 1)
    case_product(Q4K, 0, 520, 256, 1)       # one unit of K: a ring of four units
    case_product(Q8_0, 0, 600, 1024, 1)     # units of 128
    case_product(IQ3_S, 0, 300, 512, 1)     # the grid in LDS
    case_bytes(Q4K, 0, 600, 1024, 3)
    case_product(Q4K, 0, 100, 2048, 8)      # K in two chunks of the small-M product
    case_product(Q4_0, 0, 40, 4096, 5)      # four chunks, two waves per tile
    case_product(Q3K, 0, 20, 2048, 7)
    for fmt, group in BYTE_FORMATS:
        case_bytes(fmt, group, 13, 1024, 1 if which == "quick" else 6)
    case_bytes(Q6K, 0, 40, 4096, 16)        # byte activations, 16 rows, four chunks
    case_bytes(Q4K, 0, 20, 512, 40)         # byte activations, 40 rows: three row chunks
    case_product(Q4_0, 0, 24, 256, 19)      # f32 activations, 19 rows: the many-row product
    # The many-row product: partial column groups and row tiles, K splits,
    # units past K, stacked weights of one format.
    case_product(Q4K, 0, 300, 1024, 40)     # three planes, two row tiles, two K splits
    case_bytes(Q8_0, 0, 270, 1024, 70, dots=False)  # bytes, 64-row tiles, units past K: no
    case_bytes(Q6K, 0, 40, 512, 33, dots=False)     # groups of 16
    case_product(Q2K, 0, 30, 512, 20)       # groups of 16 with minimums
    case_product(Q4_0, 0, 20, 96, 33)       # a unit past K (96 = 3 blocks)
    case_product(Q5_1, 0, 20, 160, 9)       # minimums of the 32-element blocks
    case_bytes(INT4, 32, 20, 160, 24, dots=False)
    # The experts' product: MFMA formats, the generic kernel (int8/40),
    # inputs per route, byte activations.
    case_experts(Q8_0, 0, 7, 256, 4, 5, 3, False)
    case_experts(IQ3_S, 0, 7, 256, 4, 5, 3, True)
    case_experts(Q4K, 0, 40, 512, 6, 3, 2, False, flags=1)
    case_experts(INT8, 40, 7, 160, 4, 5, 3, True)
    # The non-linear formats: decode kernels (1, 3 rows), many rows, a unit
    # past K for IQ4_NL.
    case_product(IQ3_S, 0, 40, 512, 3)
    case_product(IQ4_XS, 0, 40, 512, 3)
    case_product(IQ4_NL, 0, 20, 160, 3)
    case_product(IQ3_S, 0, 300, 1024, 40)
    case_product(IQ4_XS, 0, 130, 512, 20)
    case_product(IQ4_NL, 0, 20, 96, 9)
    # The float many-row kernel: bf16 / f16 / f32 activations (1, 2, 3
    # planes), two row tiles, two column groups and a K split, groups of 16,
    # a unit past K with minimums, Kapel's int4 groups; the int8 kernel it
    # replaces, forced.
    case_float_kinds(Q8_0, 0, 300, 1024, 140, BF16)
    case_float_kinds(Q6K, 0, 70, 512, 20, F16, kernel="float")
    case_float_kinds(Q4_1, 0, 40, 160, 30, F32, kernel="float")
    case_float_kinds(INT4, 64, 40, 320, 25, BF16, kernel="float")
    case_float_kinds(IQ3_S, 0, 40, 512, 100, BF16)
    case_float_kinds(Q8_0, 0, 50, 32, 20, BF16)      # one block of K
    case_float_kinds(Q4_0, 0, 70, 96, 70, BF16)      # K % 64 != 0: planes prepared, a unit past K
    k = 256
    parts = [(Q8_0, 0, blocks(Q8_0, 0, n * k // 32, 70 + i), n) for i, n in enumerate((150, 40))]
    xf = xs(20, k, 9)
    xb = (xf.view(np.uint32) >> 16).astype(np.uint16)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    arr = (W * 2)(*[W(f, g, d.ctypes.data, d.size, n) for f, g, d, n in parts])
    ws = workspace(L.kh_qmatmul_workspace(arr, 2, k, 20, 0))
    out = np.full((20, 190), np.nan, np.float32)
    assert L.kh_qmatmul(arr, 2, k, BF16, xb.ctypes.data, 20, F32, out.ctypes.data, 0, ws.ctypes.data,
                        ws.size, None) == 0
    check_f32("stacked many rows, bf16 (float kernel)", out, ko.product_f64(parts, k, xf))
    case_float_kinds(Q4K, 0, 300, 1024, 40, F32, kernel="int8")
    case_float_kinds(Q8_0, 0, 20, 256, 5, F32, kernel="float")
    k = 512
    parts = [(Q4K, 0, blocks(Q4K, 0, n * k // 256, 60 + i), n) for i, n in enumerate((260, 7))]
    x = xs(21, k, 5)
    check_f32("stacked many-row", product(parts, k, x), ko.product_f64(parts, k, x))
    if which == "all":
        for fmt, group in FORMATS:
            for rows in (3, 17):
                case_product(fmt, group, 7, 1280, rows)
        for fmt, group in BYTE_FORMATS:
            case_bytes(fmt, group, 13, 1024, 64)
        # Stacked, several formats.
        k = 512
        parts = [(f, 0, blocks(f, 0, n * k // ko.block_len(f), 40 + i), n)
                 for i, (f, n) in enumerate(((Q4K, 5), (Q6K, 3), (Q8_0, 2)))]
        x = xs(3, k, 3)
        check_f32("stacked", product(parts, k, x), ko.product_f64(parts, k, x))
    print("failed:", len(FAILED), flush=True)
    sys.exit(1 if FAILED else 0)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "quick")
