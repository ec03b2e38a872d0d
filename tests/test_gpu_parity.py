"""Parity of the HIP path with the oracle (the restated CPU algorithm), on the
device, through the C ABI.

Bars (stated per test):
- integer work bit-exact: activation bytes and scales (bytes.rs:144-158),
  i32 block dots (bytes.rs:356-394), decoded weights (the f32 decoders of
  quantized.rs:403-682);
- f32 products within 1e-4 (1 + |e|) of the f64 product of the dequantized
  weights (quantized.rs:1176-1179) and within the conformity tolerance
  1e-4 max(1, max|y|) (conformity.rs:66, :1835-1840);
- byte-activation products within 1e-5 sum|x_q w| + 1e-6 of the exact
  product of the quantized activations (bytes.rs:753-770);
- every result bitwise the same on a second run.
"""
import json
import os

import numpy as np
import pytest
import torch

import kapel_amd as ka
import oracle as ko
from kapel_amd import synth
from refrng import Rng, lcg_bytes

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def hip():
    return ka.Hip(0)


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda:0") if dtype is None else t.to("cuda:0", dtype)


HALVES = {ka.Q8_0: [0], ka.Q4_0: [0], ka.Q5_0: [0], ka.Q4_1: [0, 2], ka.Q5_1: [0, 2],
          ka.Q4K: [0, 2], ka.Q5K: [0, 2], ka.Q2K: [80, 82], ka.Q3K: [108], ka.Q6K: [208],
          ka.IQ4_NL: [0], ka.IQ4_XS: [0], ka.IQ3_S: [0]}


def random_blocks(fmt, group, count, seed):
    """Random bytes with valid f16 scales (conformity.rs:601-635 / the
    LCG of quantized.rs:1027-1062)."""
    nxt = lcg_bytes(seed)
    size = ko.block_bytes(fmt, group)
    raw = np.frombuffer(bytes(nxt() for _ in range(count * size)), dtype=np.uint8).copy()
    raw = raw.reshape(count, size)
    rng = np.random.default_rng(seed)
    for at in HALVES.get(fmt, []):
        h = np.array([ko.f16_encode(v) for v in rng.uniform(0.005, 0.02, count)], dtype=np.uint16)
        raw[:, at:at + 2] = h.view(np.uint8).reshape(count, 2)
    if fmt in (ka.INT8, ka.INT4):
        raw[:, :4] = np.frombuffer(rng.uniform(0.005, 0.02, count).astype(np.float32).tobytes(),
                                   dtype=np.uint8).reshape(count, 4)
    return raw.ravel()


def weight(fmt, group, n, k, seed, hip):
    data = random_blocks(fmt, group, n * k // ko.block_len(fmt, group), seed)
    return data, ka.QuantizedTensor(dev(data), fmt, group, n, k)


def x_uniform(rows, k, seed):
    rng = Rng(seed)
    return np.array([[rng.uniform(-1, 1) for _ in range(k)] for _ in range(rows)], np.float32)


FORMATS = [(ka.INT8, 32), (ka.INT8, 64), (ka.INT8, 40), (ka.INT8, 128), (ka.INT4, 32),
           (ka.INT4, 64), (ka.INT4, 128), (ka.INT4, 40), (ka.Q8_0, 0), (ka.Q4_0, 0), (ka.Q4_1, 0),
           (ka.Q5_0, 0), (ka.Q5_1, 0), (ka.Q2K, 0), (ka.Q3K, 0), (ka.Q4K, 0), (ka.Q5K, 0),
           (ka.Q6K, 0), (ka.IQ4_NL, 0), (ka.IQ4_XS, 0), (ka.IQ3_S, 0)]


def check_f32(got, e64, what):
    got = got.astype(np.float64)
    bad = np.abs(got - e64) > 1e-4 * (1 + np.abs(e64))
    assert not bad.any(), f"{what}: {np.argwhere(bad)[:3]} got {got[bad][:3]} want {e64[bad][:3]}"
    scale = max(1.0, np.abs(e64).max()) if e64.size else 1.0
    assert np.all(np.abs(got - e64) <= 1e-4 * scale), what


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_products_of_every_format(hip, fmt, group):
    """conformity.rs:877-935: [1 | 3 | 17, 1280] . fmt [7, 1280]^T, and the
    oracle's f32 product (quantized.rs:117-175) alongside."""
    k, n = 1280, 7
    data, w = weight(fmt, group, n, k, 5 + fmt, hip)
    for rows in (1, 3, 17):
        x = x_uniform(rows, k, 100 + rows)
        e64 = ko.product_f64([(fmt, group, data, n)], k, x)
        cpu = ko.product_f32([(fmt, group, data, n)], k, x)
        out = hip.forward(ka.QuantizedMatmul(), [dev(x), w])
        got = out.cpu().numpy()
        check_f32(got, e64, f"fmt {fmt}/{group} rows {rows}")
        # The GPU and the CPU algorithm agree as closely as each does with f64.
        assert np.all(np.abs(got - cpu) <= 2e-4 * (1 + np.abs(e64)))
        again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.fixture
def streamed():
    """The streamed decode kernel for every M = 1 launch it can take
    (KH_DECODE_KERNEL is read at each call), then the automatic choice."""
    os.environ["KH_DECODE_KERNEL"] = "streamed"
    yield
    os.environ.pop("KH_DECODE_KERNEL", None)


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_streamed_decode_of_every_format(hip, streamed, fmt, group):
    """The streamed decode kernel (per-wave rings) against f64 and against
    the staged kernel: K of 19 blocks of 256 (odd blocks: rows that start 2
    bytes past a dword for Q6_K and the other odd-sized blocks), K long
    enough that a wave's ring wraps (16384), and a stack of three matrices
    whose rows are not a whole number of tiles."""
    cases = [(37, 4864), (24, 16384)]
    for n, k in cases:
        if k % ko.block_len(fmt, group):
            continue
        data, w = weight(fmt, group, n, k, 70 + fmt + n, hip)
        x = x_uniform(1, k, n)
        e64 = ko.product_f64([(fmt, group, data, n)], k, x)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        check_f32(got, e64, f"streamed fmt {fmt}/{group} n {n} k {k}")
        again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        os.environ["KH_DECODE_KERNEL"] = "staged"
        staged = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        os.environ["KH_DECODE_KERNEL"] = "streamed"
        assert np.all(np.abs(got - staged) <= 2e-4 * (1 + np.abs(e64)))
    k = 2048
    if k % ko.block_len(fmt, group) == 0:
        parts, ws = [], []
        for i, n in enumerate((21, 5, 40)):
            data, w = weight(fmt, group, n, k, 90 + i, hip)
            parts.append((fmt, group, data, n))
            ws.append(w)
        x = x_uniform(1, k, 3)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x)] + ws).cpu().numpy()
        check_f32(got, ko.product_f64(parts, k, x), f"streamed stack fmt {fmt}/{group}")


def fast_blocks(fmt, n, k, seed):
    """Random codes with f16 scales in [0.005, 0.02) from numpy's generator:
    the bytes of a large matrix in a fraction of a second."""
    size, count = ko.block_bytes(fmt, 0), n * k // ko.block_len(fmt, 0)
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (count, size), dtype=np.uint8)
    for at in HALVES[fmt]:
        h = rng.uniform(0.005, 0.02, count).astype(np.float16).view(np.uint16)
        raw[:, at:at + 2] = h.view(np.uint8).reshape(count, 2)
    return raw.ravel()


def test_streamed_decode_walking_many_tiles(hip):
    """Launches of eight and more rounds of the CUs take the streamed kernel
    with one wave a tile, each wave walking several tiles through a ring of
    whole units (a ring of one tile's units for Q6_K at K = 1024, of four
    units over two-unit tiles for Q4_K at K = 512, units of 128 with the last
    one past K for Q8_0 at K = 1312), the last tile ragged: every row against
    f64, a bitwise rerun, and the staged kernel within the bar."""
    for fmt, n, k in ((ka.Q4K, 65541, 512), (ka.Q6K, 40003, 1024), (ka.Q8_0, 33007, 1312)):
        data = fast_blocks(fmt, n, k, 300 + fmt)
        w = ka.QuantizedTensor(dev(data), fmt, 0, n, k)
        x = x_uniform(1, k, 7 + fmt)
        e64 = ko.product_f64([(fmt, 0, data, n)], k, x)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        check_f32(got, e64, f"walking fmt {fmt} n {n} k {k}")
        again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        os.environ["KH_DECODE_KERNEL"] = "staged"
        try:
            staged = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        finally:
            os.environ.pop("KH_DECODE_KERNEL", None)
        assert np.all(np.abs(got - staged) <= 2e-4 * (1 + np.abs(e64)))
    # Byte activations, three rows: the product of the quantized rows.
    n, k = 40003, 512
    data = fast_blocks(ka.Q4K, n, k, 333)
    w = ka.QuantizedTensor(dev(data), ka.Q4K, 0, n, k)
    x = byte_x(3, k)
    q, s_, _ = ko.quantize_x(x)
    xq = np.repeat(s_.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    dense = ko.dequantize(ka.Q4K, 0, data).reshape(n, k)
    e, size = xq @ dense.T, np.abs(xq) @ np.abs(dense).T
    got = hip.with_byte_activations(True).forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
    hip.with_byte_activations(False)
    assert np.all(np.abs(got - e) <= 1e-5 * size + 1e-6)


def test_streamed_decode_with_byte_activations(hip, streamed):
    """The streamed kernel with byte activations (up to four rows) is the
    product of the quantized activations (bytes.rs:753-770)."""
    k = 4096
    for fmt, n in ((ka.Q4K, 40), (ka.Q6K, 33), (ka.Q8_0, 20)):
        data, w = weight(fmt, 0, n, k, 11 + fmt, hip)
        for rows in (1, 3, 4):
            x = byte_x(rows, k)
            q, s_, _ = ko.quantize_x(x)
            xq = np.repeat(s_.astype(np.float64), 32, axis=1) * q.astype(np.float64)
            dense = ko.dequantize(fmt, 0, data).reshape(n, k)
            e, size = xq @ dense.T, np.abs(xq) @ np.abs(dense).T
            got = hip.with_byte_activations(True).forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
            hip.with_byte_activations(False)
            assert np.all(np.abs(got - e) <= 1e-5 * size + 1e-6), (fmt, rows)


def test_stacked_weights_of_several_formats(hip):
    """conformity.rs:936-947: [q4_k 5; q6_k 3; q8_0 2] x 512, one output."""
    k = 512
    parts, ws = [], []
    for i, (fmt, n) in enumerate(((ka.Q4K, 5), (ka.Q6K, 3), (ka.Q8_0, 2))):
        data, w = weight(fmt, 0, n, k, 40 + i, hip)
        parts.append((fmt, 0, data, n))
        ws.append(w)
    for rows in (1, 3, 17):
        x = x_uniform(rows, k, rows)
        e64 = ko.product_f64(parts, k, x)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x)] + ws).cpu().numpy()
        assert got.shape == (rows, 10)
        check_f32(got, e64, f"stacked rows {rows}")


def test_empty_shapes(hip):
    """conformity.rs:1414-1430: no rows, N = 0, K = 0 (zeros)."""
    for fmt in (ka.INT8, ka.Q8_0):
        group = 32 if fmt == ka.INT8 else 0
        _, w = weight(fmt, group, 5, 64, 1, hip)
        out = hip.forward(ka.QuantizedMatmul(), [torch.zeros((0, 64), device="cuda:0"), w])
        assert out.shape == (0, 5)
        empty = ka.QuantizedTensor(torch.zeros(0, dtype=torch.uint8, device="cuda:0"), fmt, group, 0, 64)
        out = hip.forward(ka.QuantizedMatmul(), [torch.ones((3, 64), device="cuda:0"), empty])
        assert out.shape == (3, 0)
        k0 = ka.QuantizedTensor(torch.zeros(0, dtype=torch.uint8, device="cuda:0"), fmt, group, 5, 0)
        out = hip.forward(ka.QuantizedMatmul(), [torch.ones((3, 0), device="cuda:0"), k0])
        assert out.shape == (3, 5) and bool((out == 0).all())


def test_activation_types(hip):
    """bf16 and f16 activations give outputs of their type (the op's
    signature), within the conformity tolerance of that type."""
    k, n = 1024, 48
    data, w = weight(ka.Q4K, 0, n, k, 9, hip)
    x = x_uniform(2, k, 3)
    for dtype, tol in ((torch.bfloat16, 5e-2), (torch.float16, 1e-2)):
        xt = dev(x).to(dtype)
        e64 = ko.product_f64([(ka.Q4K, 0, data, n)], k, xt.float().cpu().numpy())
        got = hip.forward(ka.QuantizedMatmul(), [xt, w])
        assert got.dtype == dtype
        assert np.all(np.abs(got.float().cpu().numpy() - e64) <= tol * max(1, np.abs(e64).max()))


BYTE_FORMATS = [(ka.Q8_0, 0), (ka.Q4_0, 0), (ka.Q4K, 0), (ka.Q5K, 0), (ka.Q6K, 0), (ka.INT8, 32),
                (ka.INT8, 128), (ka.INT4, 32), (ka.INT4, 64)]


def byte_x(rows, k):
    i = np.arange(rows * k)
    base = ((i * 7919) % 201).astype(np.float32) / np.float32(100.0) - np.float32(1.0)
    return (base * (1 + (i // 32) % 7).astype(np.float32)).reshape(rows, k)


def test_activation_bytes_are_bit_exact(hip):
    """bytes.rs:144-158 on the device: q, scale and sums equal the oracle's
    bit for bit, ties and zero blocks included."""
    x = byte_x(6, 1024)
    x[0, :32] = 0.0
    x[1, :4] = [127.0, 0.5, 1.5, -2.5]
    x[2, 64:96] = np.float32(1e-30)
    q, s, sums = hip.quantize_x(dev(x))
    oq, os_, osums = ko.quantize_x(x)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(sums.cpu().numpy().view(np.uint32), osums.view(np.uint32))


@pytest.mark.parametrize("fmt,group", BYTE_FORMATS)
def test_byte_products_and_block_dots(hip, fmt, group):
    """bytes.rs:720-774 plus the bit-exact i32 block dots."""
    n, k = 13, 1024
    data, w = weight(fmt, group, n, k, 3, hip)
    for rows in (1, 6, 64):
        x = byte_x(rows, k)
        out_cpu, dots_cpu = ko.product_bytes([(fmt, group, data, n)], k, x, with_dots=True)
        q, s, _ = ko.quantize_x(x)
        dots = hip.block_dots(w, dev(q)).cpu().numpy()
        assert np.array_equal(dots, dots_cpu), f"fmt {fmt} rows {rows}"
        got = hip.with_byte_activations(True, all_rows=rows > 16).forward(ka.QuantizedMatmul(), [dev(x), w])
        hip.with_byte_activations(False)
        got = got.cpu().numpy().astype(np.float64)
        dense = ko.dequantize(fmt, group, data).reshape(n, k)
        xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
        e = xq @ dense.T
        size = np.abs(xq) @ np.abs(dense).T
        assert np.all(np.abs(got - e) <= 1e-5 * size + 1e-6), f"fmt {fmt} rows {rows}"
        assert np.all(np.abs(got - out_cpu) <= 2e-5 * size + 2e-6)


def test_byte_mode_stops_at_sixteen_rows(hip):
    """kapel-cpu/src/matmul.rs:14,292-306: byte activations only for x of at
    most 16 rows (IN_PLACE_ROWS); above, the product is the f32 one, bit for
    bit, unless bytes are asked for at every row count
    (KH_BYTE_ACTIVATIONS_ALL_ROWS, then within the byte bound)."""
    k, n = 1024, 40
    data, w = weight(ka.Q4K, 0, n, k, 77, hip)
    for rows in (16, 17, 64):
        x = x_uniform(rows, k, 500 + rows)
        f32 = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        byte = hip.with_byte_activations(True).forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        every = hip.with_byte_activations(True, all_rows=True).forward(ka.QuantizedMatmul(), [dev(x), w])
        hip.with_byte_activations(False)
        e, size = exact_bytes(ka.Q4K, 0, data, n, k, x)
        assert np.all(np.abs(every.cpu().numpy().astype(np.float64) - e) <= 1e-5 * size + 1e-6), rows
        if rows <= 16:
            assert np.all(np.abs(byte.astype(np.float64) - e) <= 1e-5 * size + 1e-6), rows
            assert not np.array_equal(byte, f32)
        else:
            assert np.array_equal(byte.view(np.uint32), f32.view(np.uint32)), rows


def test_reused_activations(hip):
    """KH_REUSE_ACTIVATIONS: one x by weights given in several calls, the
    activations prepared by the first call only (the many-row product's
    prepared planes): bitwise equal to the calls without reuse, f32 and
    bytes."""
    k = 1280
    hip.workspace(64 << 20)  # one workspace for all the calls
    parts = [weight(ka.Q4K, 0, 300, k, 90, hip), weight(ka.Q4K, 0, 200, k, 91, hip)]
    x = dev(x_uniform(40, k, 7))
    for byte in (False, True):
        hip.with_byte_activations(byte, all_rows=byte)
        try:
            plain = [hip.forward(ka.QuantizedMatmul(), [x, w]).cpu().numpy() for _, w in parts]
            first = hip.forward(ka.QuantizedMatmul(), [x, parts[0][1]]).cpu().numpy()
            second = hip.forward(ka.QuantizedMatmul(), [x, parts[1][1]], reuse_activations=True).cpu().numpy()
        finally:
            hip.with_byte_activations(False)
        assert np.array_equal(first.view(np.uint32), plain[0].view(np.uint32))
        assert np.array_equal(second.view(np.uint32), plain[1].view(np.uint32)), byte
    # The float many-row kernel's bf16 planes, reused: bf16 activations,
    # Q8_0 at 64 rows (its dot mode) and Q4_K at 128 (split weights).
    for fmt, rows in ((ka.Q8_0, 64), (ka.Q4K, 128)):
        parts = [weight(fmt, 0, 300, k, 92, hip), weight(fmt, 0, 200, k, 93, hip)]
        xb = dev(x_uniform(rows, k, 8), torch.bfloat16)
        plain = [hip.forward(ka.QuantizedMatmul(), [xb, w]).cpu() for _, w in parts]
        first = hip.forward(ka.QuantizedMatmul(), [xb, parts[0][1]]).cpu()
        second = hip.forward(ka.QuantizedMatmul(), [xb, parts[1][1]], reuse_activations=True).cpu()
        assert torch.equal(first.view(torch.int16), plain[0].view(torch.int16))
        assert torch.equal(second.view(torch.int16), plain[1].view(torch.int16)), fmt


def test_byte_mode_falls_back_for_other_formats(hip):
    """matmul.rs:293: one weight without a byte reader (Q2_K) puts the whole
    product in f32 activations."""
    k = 512
    d1, w1 = weight(ka.Q4K, 0, 4, k, 1, hip)
    d2, w2 = weight(ka.Q2K, 0, 4, k, 2, hip)
    x = x_uniform(2, k, 9)
    e64 = ko.product_f64([(ka.Q4K, 0, d1, 4), (ka.Q2K, 0, d2, 4)], k, x)
    got = hip.with_byte_activations(True).forward(ka.QuantizedMatmul(), [dev(x), w1, w2])
    hip.with_byte_activations(False)
    check_f32(got.cpu().numpy(), e64, "fallback")


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_dequantize_matches_the_cpu_decoders(hip, fmt, group):
    """kernels/src/lib.rs:3745 equivalent: the f32 values of the CPU's
    portable decoders (quantized.rs:403-682), bit for bit, and gathered rows."""
    n, k = 5, 512 if ko.block_len(fmt, group) != 40 else 520
    data, w = weight(fmt, group, n, k, 21, hip)
    got = hip.dequantize(w).cpu().numpy()
    size, length = ko.block_bytes(fmt, group), ko.block_len(fmt, group)
    want = np.concatenate([ko.decode_f32(fmt, group, data[i * size:(i + 1) * size])
                           for i in range(n * k // length)]).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    rows = hip.dequantize_rows(w, torch.tensor([4, 0, 2, 2])).cpu().numpy()
    assert np.array_equal(rows, want[[4, 0, 2, 2]])


def test_golden_blocks_on_the_device(hip):
    """The golden blocks of kapel-ref/src/golden.rs (tests/golden), decoded
    on the device, within 1e-6 relative of their GGML-order values."""
    with open(os.path.join(HERE, "golden", "golden_blocks.json")) as f:
        cases = json.load(f)
    for case in cases:
        data = np.frombuffer(bytes.fromhex(case["bytes"]), dtype=np.uint8)
        length = ko.block_len(case["format"], 0)
        w = ka.QuantizedTensor(dev(data), case["format"], 0, 1, length)
        got = hip.dequantize(w).cpu().numpy()[0].astype(np.float64)
        want = np.array(case["values"])
        assert np.all(np.abs(got - want) <= 1e-6 * np.maximum(np.abs(want), 1e-3)), case["name"]


# ------------------------------------------------------------ full sizes

LLAMA_3B = [("q", 3072, 3072, ka.Q4K), ("k", 1024, 3072, ka.Q4K), ("v", 1024, 3072, ka.Q4K),
            ("o", 3072, 3072, ka.Q4K), ("gate", 8192, 3072, ka.Q4K), ("up", 8192, 3072, ka.Q4K),
            ("down", 3072, 8192, ka.Q6K)]


def synth_weight(fmt, group, n, k, seed):
    values = synth.normal(seed, n * k, 0.02).reshape(n, k)
    data = ka.quantize(fmt, group, values)
    return data, ka.QuantizedTensor(dev(data), fmt, group, n, k)


@pytest.mark.parametrize("byte", [False, True])
def test_llama_3b_layer_at_full_size(hip, byte):
    """Configs 2 and 3: each stacked call of the layer (qkv, o, gate+up, down)
    at full size, M = 1 and M = 64 (bytes).  A sample of 96 output rows of
    each matrix is checked against the oracle; every output is finite and a
    second run is bitwise equal."""
    rows = 64 if byte else 1
    hip.with_byte_activations(byte, all_rows=byte)
    try:
        mats = {name: synth_weight(fmt, 0, n, k, 1000 + i) + (fmt, n, k)
                for i, (name, n, k, fmt) in enumerate(LLAMA_3B)}
        for call in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            k = mats[call[0]][4]
            x = synth.normal(7, rows * k, 1.0).reshape(rows, k)
            ws = [mats[c][1] for c in call]
            got = hip.forward(ka.QuantizedMatmul(), [dev(x)] + ws).cpu().numpy()
            again = hip.forward(ka.QuantizedMatmul(), [dev(x)] + ws).cpu().numpy()
            assert np.isfinite(got).all()
            assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
            col = 0
            for c in call:
                data, _, fmt, n, kk = mats[c]
                sample = np.linspace(0, n - 1, 96).astype(int)
                rb = ko.row_bytes(fmt, 0, kk)
                sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in sample])
                # Rows from every 32-row tile of the launch: 0-3, 31, 32,
                # 47, 60-63 at M = 64.
                pick = np.unique(np.r_[0:4, 31, 32, 47, rows - 4:rows]) if byte else np.r_[0:1]
                xr = x[pick]
                if byte:
                    want = ko.product_bytes([(fmt, 0, sub, len(sample))], kk, xr)
                    q, s, _ = ko.quantize_x(xr)
                    dense = ko.dequantize(fmt, 0, sub).reshape(len(sample), kk)
                    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
                    size = np.abs(xq) @ np.abs(dense).T
                    assert np.all(np.abs(got[pick][:, col + sample] - want) <= 2e-5 * size + 2e-6), c
                else:
                    e64 = ko.product_f64([(fmt, 0, sub, len(sample))], kk, xr)
                    check_f32(got[pick][:, col + sample], e64, c)
                col += n
    finally:
        hip.with_byte_activations(False)


def test_config_1_exactly(hip):
    """Config 1: Q4_0 8192 x 2048 from N(0, 0.02) values of seed 0, x from
    N(0, 1) of seed 1; all 8192 outputs against the f64 product within
    1e-4 max(1, max|y|) (kapel-ref/src/conformity.rs:1835-1840) and 1e-4 (1 +
    |e|), and a second run bitwise equal."""
    n, k = 8192, 2048
    data = ka.quantize(ka.Q4_0, 0, synth.normal(0, n * k, 0.02))
    w = ka.QuantizedTensor(dev(data), ka.Q4_0, 0, n, k)
    x = synth.normal(1, k, 1.0).reshape(1, k)
    got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
    again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
    e64 = ko.product_f64([(ka.Q4_0, 0, data, n)], k, x)
    check_f32(got, e64, "config 1")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_config_5_output_table_at_full_size(hip):
    """Config 5's Q6_K output table, 151936 x 4096 (510 MB), at M = 1 and 8:
    every output finite, 272 rows (the first, the last tile's 16 and an even
    spread) against the f64 product, a second run bitwise equal.  The values
    are 4 Mi N(0, 0.02) draws repeated over the table (as the bench)."""
    n, k = 151936, 4096
    values = np.resize(synth.normal(77, 1 << 22, 0.02), n * k)
    data = ka.quantize(ka.Q6K, 0, values)
    del values
    w = ka.QuantizedTensor(dev(data), ka.Q6K, 0, n, k)
    rb = ko.row_bytes(ka.Q6K, 0, k)
    sample = np.unique(np.r_[np.linspace(0, n - 17, 256).astype(int), n - 16:n])
    sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in sample])
    for rows in (1, 8):
        x = synth.normal(6 + rows, rows * k, 1.0).reshape(rows, k)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        assert got.shape == (rows, n) and np.isfinite(got).all()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        e64 = ko.product_f64([(ka.Q6K, 0, sub, len(sample))], k, x)
        check_f32(got[:, sample], e64, f"table rows {rows}")


def test_qwen3_8b_prefill_in_f32_at_full_size(hip):
    """Config 4 in the reference's own mode above 16 rows (f32 products of
    the bf16 activations, kapel-cpu/src/matmul.rs:303-306): the Q8_0 gate/up
    and down calls at M = 512, a sample of 48 weight rows on 8 activation rows
    against the f64 product within the bf16 output's rounding."""
    rows = 512
    calls = [((("gate", 12288), ("up", 12288)), 4096), ((("down", 4096),), 12288)]
    for i, (call, k) in enumerate(calls):
        mats = [synth_weight(ka.Q8_0, 0, n, k, 3100 + 10 * i + j) + (n,) for j, (_, n) in enumerate(call)]
        xb = dev(synth.normal(21 + i, rows * k, 1.0).reshape(rows, k), torch.bfloat16)
        got = hip.forward(ka.QuantizedMatmul(), [xb] + [m[1] for m in mats]).float().cpu().numpy()
        assert np.isfinite(got).all()
        x = xb.float().cpu().numpy()
        pick = np.r_[0:4, rows - 4:rows]
        col = 0
        for data, _, n in mats:
            sample = np.linspace(0, n - 1, 48).astype(int)
            rb = ko.row_bytes(ka.Q8_0, 0, k)
            sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in sample])
            e64 = ko.product_f64([(ka.Q8_0, 0, sub, len(sample))], k, x[pick])
            have = got[pick][:, col + sample].astype(np.float64)
            assert np.all(np.abs(have - e64) <= 2 ** -8 * np.abs(e64) + 1e-4 * (1 + np.abs(e64))), call
            col += n


def test_low_bit_mix_and_output_table_sample(hip):
    """Config 5 shapes at M in {1, 8}: the Q2_K, Q3_K and Q5_K FFN matrices
    (up 12288 x 4096 and down 4096 x 12288 each), int4/32 attention (q and o
    4096 x 4096, k and v 1024 x 4096), Q6_K output-table rows (a slice of
    4096 rows of the table; the whole table has its own test)."""
    cases = [(ka.Q2K, 0, 12288, 4096), (ka.Q2K, 0, 4096, 12288), (ka.Q3K, 0, 12288, 4096),
             (ka.Q3K, 0, 4096, 12288), (ka.Q5K, 0, 12288, 4096), (ka.Q5K, 0, 4096, 12288),
             (ka.INT4, 32, 4096, 4096), (ka.INT4, 32, 1024, 4096), (ka.Q6K, 0, 4096, 4096)]
    for i, (fmt, group, n, k) in enumerate(cases):
        data, w = synth_weight(fmt, group, n, k, 2000 + i)
        for rows in (1, 8):
            x = synth.normal(50 + rows, rows * k, 1.0).reshape(rows, k)
            got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
            sample = np.linspace(0, n - 1, 64).astype(int)
            rb = ko.row_bytes(fmt, group, k)
            sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in sample])
            e64 = ko.product_f64([(fmt, group, sub, len(sample))], k, x)
            check_f32(got[:, sample], e64, f"fmt {fmt} rows {rows}")


# ------------------------------------------------------------ many rows

def exact_bytes(fmt, group, data, n, k, x):
    """The exact product of the quantized activations (bytes.rs:144-158) and
    the dequantized weights, and the size bound sum |x_q w|."""
    q, s, _ = ko.quantize_x(x)
    dense = ko.dequantize(fmt, group, data).reshape(n, k)
    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    return xq @ dense.T, np.abs(xq) @ np.abs(dense).T


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_many_rows_of_every_format(hip, fmt, group):
    """The many-row product (M > 16): 40 and 130 activation rows by 300
    weight rows (a partial column group, partial row tiles, splits of K),
    f32 activations against the f64 product, bytes against the exact product
    of the quantized activations; bitwise equal on a second run."""
    k, n = 1280, 300
    data, w = weight(fmt, group, n, k, 70 + fmt, hip)
    byte = (fmt, group) in BYTE_FORMATS
    for rows in (40, 130):
        x = x_uniform(rows, k, 300 + rows)
        got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy().astype(np.float64)
        e64 = ko.product_f64([(fmt, group, data, n)], k, x)
        # Within 1e-4 (1 + |e|), plus 1e-7 sum |x w| for the outputs near
        # zero: the rounding of an f32 sum of K terms scales with the terms
        # (the CPU algorithm's error on these cases reaches 3e-8 of it).
        size = np.abs(x.astype(np.float64)) @ np.abs(ko.dequantize(fmt, group, data).reshape(n, k)).T
        bad = np.abs(got - e64) > 1e-4 * (1 + np.abs(e64)) + 1e-7 * size
        assert not bad.any(), f"fmt {fmt}/{group} rows {rows}: {np.argwhere(bad)[:3]}"
        got = got.astype(np.float32)
        again = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        if byte:
            hip.with_byte_activations(True, all_rows=True)
            try:
                got = hip.forward(ka.QuantizedMatmul(), [dev(x), w]).cpu().numpy().astype(np.float64)
            finally:
                hip.with_byte_activations(False)
            e, size = exact_bytes(fmt, group, data, n, k, x)
            assert np.all(np.abs(got - e) <= 1e-5 * size + 1e-6), f"bytes fmt {fmt}/{group} rows {rows}"


@pytest.fixture
def float_kernel():
    """The float many-row kernel forced at every row count (KH_MANY_KERNEL is
    read at each call), then the automatic choice."""
    os.environ["KH_MANY_KERNEL"] = "float"
    yield
    os.environ.pop("KH_MANY_KERNEL", None)


MM_FORMATS = [f for f in FORMATS if f[0] not in (ka.INT8, ka.INT4) or f[1] in (32, 64, 128)]


def product_f32_out(hip, xt, ws):
    """kh_qmatmul with f32 outputs whatever the activations' type (the C ABI
    takes the two types apart; the Python op gives x's type)."""
    rows, k = xt.shape
    arr = (ka._Weight * len(ws))(*[w.weight() for w in ws])
    width = sum(w.n for w in ws)
    space = hip.workspace(ka.lib().kh_qmatmul_workspace(arr, len(ws), k, rows, 0))
    out = torch.full((rows, width), float("nan"), device="cuda:0")
    st = ka.lib().kh_qmatmul(arr, len(ws), k, ka.float_kind(xt.dtype), xt.data_ptr(), rows, 0,
                             out.data_ptr(), 0, space.data_ptr(), space.numel(), hip.stream())
    assert st == 0, st
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt,group", MM_FORMATS)
def test_float_many_row_kernel_of_every_format(hip, float_kernel, fmt, group):
    """The many-row product on the bf16 matrix cores (weights in three bf16
    parts, activations in one, two or three exact bf16 planes): bf16, f16 and
    f32 activations, 130 rows (a full and a partial row tile) by 300 weight
    rows (partial column group) with K split, against the f64 product of the
    activations as given within 1e-4 (1 + |e|) + 1e-7 sum|x w|, as the f32
    many-row test; bitwise equal on a second run."""
    k, n, rows = 1280, 300, 130
    data, w = weight(fmt, group, n, k, 90 + fmt, hip)
    dense = ko.dequantize(fmt, group, data).reshape(n, k)
    x32 = x_uniform(rows, k, 500 + fmt)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        xt = dev(x32, dtype)
        x = xt.float().cpu().numpy().astype(np.float64)
        got = product_f32_out(hip, xt, [w]).astype(np.float64)
        e64 = x @ dense.T
        size = np.abs(x) @ np.abs(dense).T
        bad = np.abs(got - e64) > 1e-4 * (1 + np.abs(e64)) + 1e-7 * size
        assert not bad.any(), f"fmt {fmt}/{group} {dtype}: {np.argwhere(bad)[:3]}"
        again = product_f32_out(hip, xt, [w])
        assert np.array_equal(got.astype(np.float32).view(np.uint32), again.view(np.uint32))


def test_float_many_row_kernel_is_the_default_for_bf16_rows(hip):
    """From 96 rows of bf16 activations the automatic choice is the float
    kernel: its result equals the forced float kernel's bit for bit, and the
    int8-plane kernel's within the f32 bar."""
    k, n, rows = 512, 260, 96
    data, w = weight(ka.Q4K, 0, n, k, 77, hip)
    xt = dev(x_uniform(rows, k, 77), torch.bfloat16)
    auto = product_f32_out(hip, xt, [w])
    res = {}
    for kern in ("float", "int8"):
        os.environ["KH_MANY_KERNEL"] = kern
        try:
            res[kern] = product_f32_out(hip, xt, [w])
        finally:
            os.environ.pop("KH_MANY_KERNEL", None)
    assert np.array_equal(auto.view(np.uint32), res["float"].view(np.uint32))
    e = res["int8"].astype(np.float64)
    assert np.all(np.abs(auto - e) <= 1e-4 * (1 + np.abs(e)))


QWEN3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
            ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]


def test_qwen3_8b_prefill_at_full_size(hip):
    """Config 4: the Q8_0 layer of Qwen3-8B at M = 512 with bf16 activations
    and byte activations, each stacked call at full size.  A sample of 64
    weight rows of each matrix is checked on the first and last 8 activation
    rows against the CPU algorithm (bytes.rs:200-241); every output is
    finite and a second run is bitwise equal."""
    rows = 512
    hip.with_byte_activations(True, all_rows=True)
    try:
        mats = {name: synth_weight(ka.Q8_0, 0, n, k, 3000 + i) + (n, k)
                for i, (name, n, k) in enumerate(QWEN3_8B)}
        for call in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            k = mats[call[0]][3]
            xb = dev(synth.normal(11, rows * k, 1.0).reshape(rows, k), torch.bfloat16)
            ws = [mats[c][1] for c in call]
            got = hip.forward(ka.QuantizedMatmul(), [xb] + ws)
            again = hip.forward(ka.QuantizedMatmul(), [xb] + ws)
            got = got.float().cpu().numpy()
            assert np.isfinite(got).all()
            assert np.array_equal(got, again.float().cpu().numpy())
            x = xb.float().cpu().numpy()
            pick = np.r_[0:8, rows - 8:rows]
            col = 0
            for c in call:
                data, _, n, kk = mats[c]
                sample = np.linspace(0, n - 1, 64).astype(int)
                rb = ko.row_bytes(ka.Q8_0, 0, kk)
                sub = np.concatenate([data[r * rb:(r + 1) * rb] for r in sample])
                want = ko.product_bytes([(ka.Q8_0, 0, sub, len(sample))], kk, x[pick])
                e, size = exact_bytes(ka.Q8_0, 0, sub, len(sample), kk, x[pick])
                have = got[pick][:, col + sample].astype(np.float64)
                # bf16 output: within its rounding of the CPU's f32 result.
                assert np.all(np.abs(have - want) <= 2 ** -8 * np.abs(want) + 2e-5 * size + 2e-6), c
                col += n
    finally:
        hip.with_byte_activations(False)


# ------------------------------------------------------------- experts

EXPERT_FORMATS = [(ka.Q8_0, 0), (ka.IQ4_XS, 0), (ka.IQ3_S, 0), (ka.IQ4_NL, 0), (ka.Q4K, 0),
                  (ka.Q6K, 0), (ka.INT8, 40)]


def expert_f64(fmt, group, data, experts, n, k, x, idx):
    """kapel-ref/src/experts.rs:64-90: the f64 definition."""
    size = n * ko.row_bytes(fmt, group, k)
    dense = {e: ko.dequantize(fmt, group, data[e * size:(e + 1) * size]).reshape(n, k)
             for e in set(int(v) for v in np.ravel(idx))}
    tokens, topk = idx.shape
    rows = x.reshape(tokens, -1, k).astype(np.float64)
    out = np.zeros((tokens, topk, n))
    for t in range(tokens):
        for j in range(topk):
            out[t, j] = rows[t, j if rows.shape[1] > 1 else 0] @ dense[int(idx[t, j])].T
    return out


@pytest.mark.parametrize("fmt,group", EXPERT_FORMATS)
def test_expert_products(hip, fmt, group):
    """conformity.rs:975-990: [5, K] and [5, 3, K] by 3 of 4 experts of
    [7, K]; within 1e-4 (1 + |e|) of the f64 definition, alongside the
    CPU's experts' product (kapel-cpu/src/experts.rs:62-110); bitwise the
    same on a second run."""
    k = 320 if group == 40 else 256
    n, experts, tokens, topk = 7, 4, 5, 3
    data, w = weight(fmt, group, experts * n, k, 40 + fmt, hip)
    rng = np.random.default_rng(12)
    idx = rng.integers(0, experts, size=(tokens, topk))
    op = ka.ExpertMatmul(experts)
    for per_route in (False, True):
        shape = (tokens, topk, k) if per_route else (tokens, k)
        x = rng.uniform(-1, 1, size=shape).astype(np.float32)
        got = hip.forward(op, [dev(x), w, dev(idx)]).cpu().numpy()
        assert got.shape == (tokens, topk, n)
        e64 = expert_f64(fmt, group, data, experts, n, k, x, idx)
        check_f32(got.reshape(-1, n), e64.reshape(-1, n), f"experts fmt {fmt} per_route {per_route}")
        cpu = ko.expert_product(fmt, group, data, experts, k, x, idx)
        assert np.all(np.abs(got - cpu) <= 2e-4 * (1 + np.abs(e64)))
        again = hip.forward(op, [dev(x), w, dev(idx)]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_expert_products_in_bf16_and_bytes(hip):
    """bf16 activations (output bf16), and byte activations for the formats
    that have them (kapel-cuda/src/experts.rs:166-172 takes bytes for Q8_0):
    within the bound of bytes.rs:753-770."""
    k, n, experts, tokens, topk = 512, 24, 6, 4, 2
    rng = np.random.default_rng(3)
    idx = rng.integers(0, experts, size=(tokens, topk))
    op = ka.ExpertMatmul(experts)
    for fmt in (ka.Q8_0, ka.Q4K):
        data, w = weight(fmt, 0, experts * n, k, 60 + fmt, hip)
        x = rng.uniform(-1, 1, size=(tokens, k)).astype(np.float32)
        xb = torch.from_numpy(x).to(torch.bfloat16)
        got = hip.forward(op, [xb.to("cuda:0"), w, dev(idx)])
        assert got.dtype == torch.bfloat16
        e = expert_f64(fmt, 0, data, experts, n, k, xb.float().numpy(), idx)
        got = got.float().cpu().numpy()
        assert np.all(np.abs(got - e) <= 1e-2 * (1 + np.abs(e))), f"bf16 fmt {fmt}"
        hip.with_byte_activations(True)
        try:
            got = hip.forward(op, [dev(x), w, dev(idx)]).cpu().numpy().astype(np.float64)
        finally:
            hip.with_byte_activations(False)
        q, s, _ = ko.quantize_x(x)
        xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
        dense = ko.dequantize(fmt, 0, data).reshape(experts, n, k)
        for t in range(tokens):
            for j in range(topk):
                d = dense[idx[t, j]]
                bound = 1e-5 * (np.abs(xq[t]) @ np.abs(d).T) + 1e-6
                assert np.all(np.abs(got[t, j] - xq[t] @ d.T) <= bound), f"bytes fmt {fmt} {t} {j}"


def test_expert_indices_out_of_range(hip):
    """An index of `experts` or more: the op's check refuses it
    (experts.rs:151-163); unchecked, its route's outputs are NaN and the
    others are unchanged (kernels/src/lib.rs:3499-3504)."""
    k, n, experts = 256, 16, 4
    data, w = weight(ka.Q4K, 0, experts * n, k, 8, hip)
    x = np.random.default_rng(1).uniform(-1, 1, size=(2, k)).astype(np.float32)
    op = ka.ExpertMatmul(experts)
    idx = np.array([[1, 4], [3, 0]])
    with pytest.raises(ka.IndexOutOfRange):
        hip.forward(op, [dev(x), w, dev(idx)])
    got = hip.forward(op, [dev(x), w, dev(idx)], check_indices=False).cpu().numpy()
    assert np.all(np.isnan(got[0, 1]))
    good = np.array([[1, 0], [3, 0]])
    want = ko.expert_product(ka.Q4K, 0, data, experts, k, x, good)
    for t, j in ((0, 0), (1, 0), (1, 1)):
        assert np.all(np.abs(got[t, j] - want[t, j]) <= 2e-4 * (1 + np.abs(want[t, j])))


def test_moe_ffn_at_full_size(hip):
    """A mixture-of-experts FFN at the size of Qwen3-30B-A3B's (128 experts,
    8 a token, 768 x 2048 gate/up and 2048 x 768 down, Q4_K): decode (1
    token) and 16 tokens; every route against the CPU's product of its expert
    for a sample of tokens."""
    experts, topk, hidden, inner = 128, 8, 2048, 768
    for name, n, k in (("up", inner, hidden), ("down", hidden, inner)):
        data, w = weight(ka.Q4K, 0, experts * n, k, 90 + k, hip)
        for tokens in (1, 16):
            rng = np.random.default_rng(tokens + k)
            idx = np.stack([rng.choice(experts, topk, replace=False) for _ in range(tokens)])
            x = rng.uniform(-1, 1, size=(tokens, k)).astype(np.float32)
            got = hip.forward(ka.ExpertMatmul(experts), [dev(x), w, dev(idx)]).cpu().numpy()
            assert np.isfinite(got).all()
            sample = [0, tokens - 1]
            want = ko.expert_product(ka.Q4K, 0, data, experts, k, x[sample], idx[sample])
            e64 = expert_f64(ka.Q4K, 0, data, experts, n, k, x[sample], idx[sample])
            assert np.all(np.abs(got[sample] - e64) <= 1e-4 * (1 + np.abs(e64))), f"{name} {tokens}"
            assert np.all(np.abs(got[sample] - want) <= 2e-4 * (1 + np.abs(e64)))


def test_gguf_weights_to_the_product(hip, tmp_path):
    """GGUF on disk to the device (kapel-hub/src/gguf.rs): Q4_K and Q6_K
    matrices written to a file, mapped, uploaded with their blocks unchanged
    and multiplied stacked; against the oracle on the file's bytes."""
    from kapel_amd import gguf
    k = 1024
    d1 = random_blocks(ka.Q4K, 0, 40 * k // 256, 81)
    d2 = random_blocks(ka.Q6K, 0, 24 * k // 256, 82)
    path = tmp_path / "layer.gguf"
    gguf.write(path, [("general.architecture", gguf.Entry("string", "llama"))],
               [("blk.0.ffn_up.weight", ka.QuantizedTensor(torch.from_numpy(d1), ka.Q4K, 0, 40, k)),
                ("blk.0.ffn_down.weight", ka.QuantizedTensor(torch.from_numpy(d2), ka.Q6K, 0, 24, k))])
    f = gguf.Gguf.open(path)
    w1 = f.quantized("blk.0.ffn_up.weight", device="cuda:0")
    w2 = f.quantized("blk.0.ffn_down.weight", device="cuda:0")
    x = x_uniform(3, k, 17)
    got = hip.forward(ka.QuantizedMatmul(), [dev(x), w1, w2]).cpu().numpy()
    e64 = ko.product_f64([(ka.Q4K, 0, f.raw("blk.0.ffn_up.weight"), 40),
                          (ka.Q6K, 0, f.raw("blk.0.ffn_down.weight"), 24)], k, x)
    check_f32(got, e64, "gguf")


def test_unaligned_and_extreme_activations(hip):
    """Activations that are not 16-byte aligned (copied to the workspace
    first), rows of zeros, blocks mixing magnitudes 1e-30 to 1e+30, and
    subnormal values, at M = 1, 3 and 40 (the decode, small-M and many-row
    kernels): within 1e-4 (1 + |e|) of the f64 product."""
    k, n = 1024, 40
    data, w = weight(ka.Q4K, 0, n, k, 33, hip)
    rng = np.random.default_rng(6)
    for rows in (1, 3, 40):
        x = rng.uniform(-1, 1, size=(rows, k)).astype(np.float32)
        if rows > 1:
            x[1] = 0.0
        x[0, 64:96] *= np.float32(1e-30)
        x[0, 96] = np.float32(1e30) if rows > 1 else np.float32(3.0)
        x[-1, 128:160] = np.float32(1e-40)
        base = torch.zeros(rows * k + 1, dtype=torch.float32, device="cuda:0")
        xt = base[1:].view(rows, k)
        xt.copy_(dev(x))
        assert xt.data_ptr() % 16 != 0
        e64 = ko.product_f64([(ka.Q4K, 0, data, n)], k, x)
        got = hip.forward(ka.QuantizedMatmul(), [xt, w]).cpu().numpy().astype(np.float64)
        assert np.all(np.abs(got - e64) <= 1e-4 * (1 + np.abs(e64))), rows
        if rows > 1:
            assert np.all(got[1] == 0.0)


def test_unaligned_activations_of_the_float_many_row_kernel(hip):
    """bf16, f16 and f32 activations 2 or 4 bytes off a 16-byte boundary at 96
    rows (the float many-row kernel's choice for Q8_0), within 1e-4 (1 + |e|)
    of the f64 product of the activations as given (f32 outputs)."""
    k, n, rows = 512, 140, 96
    data, w = weight(ka.Q8_0, 0, n, k, 34, hip)
    dense = ko.dequantize(ka.Q8_0, 0, data).reshape(n, k)
    x32 = np.random.default_rng(8).uniform(-1, 1, size=(rows, k)).astype(np.float32)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        base = torch.zeros(rows * k + 1, dtype=dtype, device="cuda:0")
        xt = base[1:].view(rows, k)
        xt.copy_(dev(x32, dtype))
        assert xt.data_ptr() % 16 != 0
        x = xt.float().cpu().numpy().astype(np.float64)
        got = product_f32_out(hip, xt, [w]).astype(np.float64)
        e64 = x @ dense.T
        assert np.all(np.abs(got - e64) <= 1e-4 * (1 + np.abs(e64))), dtype


def test_outputs_written_in_full_and_workspace_reused(hip):
    """kapel-cuda/src/lib.rs:70-74 (outputs poisoned before each op: a part
    left unwritten gives NaN): every kernel path writes its whole output.
    Launches of different shapes, kinds and formats share one workspace and
    run interleaved, twice, on the default and on another stream: every
    result is bitwise the same (the workspace's counters return to their
    starting state after each launch; nothing depends on the stream)."""
    k = 1280
    mats = {}
    for i, (fmt, group) in enumerate([(ka.Q4K, 0), (ka.Q6K, 0), (ka.Q8_0, 0), (ka.Q4_0, 0), (ka.INT4, 32)]):
        mats[fmt] = [weight(fmt, group, n, k, 300 + 10 * i + j, hip) for j, n in enumerate((48, 16))]
    cases = [(fmt, rows, byte) for fmt in mats for rows in (1, 3, 17, 64) for byte in (False, True)]
    xs = {rows: dev(x_uniform(rows, k, 400 + rows)) for rows in (1, 3, 17, 64)}

    def run(fmt, rows, byte):
        hip.with_byte_activations(byte, all_rows=byte)
        ws = [w for _, w in mats[fmt]]
        out = torch.full((rows, sum(w.n for w in ws)), float("nan"), device="cuda:0")
        hip.forward(ka.QuantizedMatmul(), [xs[rows]] + ws, out=out)
        return out

    try:
        first = {}
        for case in cases:
            out = run(*case).cpu().numpy()
            assert not np.isnan(out).any(), f"unwritten outputs: format {case[0]}, rows {case[1]}, bytes {case[2]}"
            first[case] = out
            if case[1] == 3 and not case[2]:
                data = [(case[0], w.group, d, w.n) for d, w in mats[case[0]]]
                check_f32(out, ko.product_f64(data, k, xs[3].cpu().numpy()), f"format {case[0]} stacked")
        side = torch.cuda.Stream()
        for use_side in (False, True):
            with torch.cuda.stream(side if use_side else torch.cuda.current_stream()):
                again = {case: run(*case) for case in reversed(cases)}
            torch.cuda.synchronize()
            for case in cases:
                got = again[case].cpu().numpy()
                assert np.array_equal(got.view(np.uint32), first[case].view(np.uint32)), \
                    f"format {case[0]}, rows {case[1]}, bytes {case[2]}, side stream {use_side}"
    finally:
        hip.with_byte_activations(False)
