"""Pins the oracle (the C restatement of kapel's CPU path) before it is trusted.

Each check is one that a plausible mistake in the restatement (a wrong index,
shift, sign or rounding) fails:

- f16: all 65,536 patterns against numpy's IEEE half (kapel-core/src/float.rs
  tests :188-257 and kapel-cpu/src/quantized.rs:1085-1094);
- dequantize: the golden blocks of kapel-ref/src/golden.rs, decoded here by
  transcriptions of GGML's ``dequantize_row_*`` loops (which walk the output in
  order, unlike the per-element formulas of the oracle), and the hand cases of
  kapel-core/src/dtype.rs:920-945;
- quantize: the bounds of dtype.rs:948-1027;
- f32 decoders and products: quantized.rs:1097-1191;
- byte activations: bytes.rs:720-774, plus brute-force i32 block dots.
"""
import numpy as np
import pytest

import oracle as ko
from refrng import Rng, lcg_bytes

HALF, QUARTER, MINUS_ONE_AND_HALF, TWO = 0x3800, 0x3400, 0xBE00, 0x4000


# ----------------------------------------------------------------- f16 ---

def test_every_f16_pattern_decodes_exactly():
    bits = np.arange(1 << 16, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float64)
    expected32 = bits.view(np.float16).astype(np.float32)
    for b in range(1 << 16):
        e = expected[b]
        g = ko.f16_decode(b)
        h = ko.half_f32(b)
        if np.isnan(e):
            assert np.isnan(g) and np.isnan(h)
            continue
        assert g == e, hex(b)
        assert np.float32(h).view(np.uint32) == expected32[b].view(np.uint32), hex(b)
        # Every value round-trips (float.rs:191-203).
        assert ko.f16_encode(g) == b, hex(b)


def test_f16_encoding_rounds_to_nearest_even():
    # float.rs:218-230
    assert ko.f16_decode(ko.f16_encode(1.0 + 2.0 ** -11)) == 1.0
    assert ko.f16_decode(ko.f16_encode(1.0 + 3.0 * 2.0 ** -11)) == 1.0 + 2.0 ** -9
    assert ko.f16_decode(ko.f16_encode(1.0 + 2.0 ** -11 + 2.0 ** -30)) == 1.0 + 2.0 ** -10
    # float.rs:250-256: tiny values.
    smallest = ko.f16_decode(1)
    assert smallest == 2.0 ** -24
    assert ko.f16_encode(smallest * 0.5) == 0
    assert ko.f16_encode(smallest * 0.51) == 1
    assert ko.f16_encode(1e-300) == 0
    # float.rs:233-241: overflow.
    assert np.isinf(ko.f16_decode(ko.f16_encode(70000.0)))
    assert ko.f16_decode(0x7BFF) == 65504.0
    assert ko.f16_encode(-0.0) == 0x8000
    # Random doubles against numpy's correctly rounded conversion.
    rng = np.random.default_rng(5)
    values = rng.standard_normal(20000) * np.exp(rng.uniform(-25, 12, 20000))
    with np.errstate(over="ignore"):
        for v in values:
            assert ko.f16_encode(v) == int(np.float16(v).view(np.uint16)), v


# ------------------------------------------------------- golden blocks ---

def golden_block(length, seed, halves):
    """kapel-ref/src/golden.rs:22-29."""
    rng = Rng(seed)
    data = bytearray(rng.next_u64() & 0xFF for _ in range(length))
    for at, bits in halves:
        data[at] = bits & 0xFF
        data[at + 1] = bits >> 8
    return np.frombuffer(bytes(data), dtype=np.uint8)


def same(got, expected):
    assert len(got) == len(expected)
    for i, (g, e) in enumerate(zip(got, expected)):
        assert g == e, f"element {i}: {g} != {e}"


def test_golden_q4_1():
    # golden.rs:44-66
    d, m = 0.5, -1.5
    data = golden_block(20, 1, [(0, HALF), (2, MINUS_ONE_AND_HALF)])
    qs = data[4:]
    y = [0.0] * 32
    for j in range(16):
        y[j] = float(qs[j] & 0x0F) * d + m
        y[j + 16] = float(qs[j] >> 4) * d + m
    same(ko.dequantize(ko.Q4_1, 0, data), y)
    by_hand = np.array([0x00, 0x38, 0x00, 0xBE, 0xF0, 0x21] + [0] * 14, dtype=np.uint8)
    got = ko.dequantize(ko.Q4_1, 0, by_hand)
    assert (got[0], got[1], got[16], got[17], got[2]) == (-1.5, -1.0, 6.0, -0.5, -1.5)


def ggml_q5(data, d, m):
    """golden.rs:71-97, GGML's dequantize_row_q5_0 / _q5_1."""
    rest = data[4:] if m is not None else data[2:]
    qh = int(rest[0]) | int(rest[1]) << 8 | int(rest[2]) << 16 | int(rest[3]) << 24
    qs = rest[4:]
    y = [0.0] * 32
    for j in range(16):
        xh_0 = ((qh >> j) << 4) & 0x10
        xh_1 = (qh >> (j + 12)) & 0x10
        x0 = float((int(qs[j]) & 0x0F) | xh_0)
        x1 = float((int(qs[j]) >> 4) | xh_1)
        if m is not None:
            y[j], y[j + 16] = x0 * d + m, x1 * d + m
        else:
            y[j], y[j + 16] = (x0 - 16.0) * d, (x1 - 16.0) * d
    return y


def test_golden_q5_0_and_q5_1():
    # golden.rs:99-122
    data = golden_block(22, 2, [(0, HALF)])
    same(ko.dequantize(ko.Q5_0, 0, data), ggml_q5(data, 0.5, None))
    data = golden_block(24, 3, [(0, QUARTER), (2, MINUS_ONE_AND_HALF)])
    same(ko.dequantize(ko.Q5_1, 0, data), ggml_q5(data, 0.25, -1.5))
    by_hand = np.array([0x00, 0x38] + list((1 << 17).to_bytes(4, "little")) + [0] * 16,
                       dtype=np.uint8)
    got = ko.dequantize(ko.Q5_0, 0, by_hand)
    assert (got[17], got[1], got[16]) == (0.0, -8.0, -8.0)


def ggml_q2k(data, d, dmin):
    """golden.rs:128-147."""
    scales, qs = data[:16], data[16:80]
    y, i = [], 0
    for n in range(2):
        q = qs[32 * n:]
        for j in range(4):
            shift = 2 * j
            for half in (0, 16):
                sc = int(scales[i]); i += 1
                dl, ml = d * (sc & 0x0F), dmin * (sc >> 4)
                for l in range(16):
                    y.append(dl * float((int(q[l + half]) >> shift) & 3) - ml)
    return y


def test_golden_q2k():
    data = golden_block(84, 4, [(80, HALF), (82, QUARTER)])
    same(ko.dequantize(ko.Q2K, 0, data), ggml_q2k(data, 0.5, 0.25))


def ggml_q3k_scales(packed):
    """golden.rs:157-169: GGML's unpacking on 32-bit words."""
    word = lambda i: int.from_bytes(bytes(packed[i:i + 4]), "little")
    kmask1, kmask2 = 0x03030303, 0x0F0F0F0F
    aux = [word(0), word(4), word(8), 0]
    tmp = aux[2]
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4)
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4)
    aux[0] = (aux[0] & kmask2) | ((tmp & kmask1) << 4)
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4)
    raw = b"".join(w.to_bytes(4, "little") for w in aux)
    return [b - 256 if b > 127 else b for b in raw]


def ggml_q3k(data, d):
    """golden.rs:151-186."""
    hmask, qs, packed = data[:32], data[32:96], data[96:108]
    scales = ggml_q3k_scales(packed)
    y, i, m = [], 0, 1
    for n in range(2):
        q = qs[32 * n:]
        for j in range(4):
            shift = 2 * j
            for half in (0, 16):
                dl = d * float(scales[i] - 32); i += 1
                for l in range(16):
                    low = (int(q[l + half]) >> shift) & 3
                    sub = 0 if int(hmask[l + half]) & m else 4
                    y.append(dl * float(low - sub))
            m <<= 1
    return y


def test_golden_q3k():
    data = golden_block(110, 5, [(108, TWO)])
    same(ko.dequantize(ko.Q3K, 0, data), ggml_q3k(data, 2.0))


def scale_min_k4(j, q):
    """golden.rs:190-200, GGML's get_scale_min_k4."""
    if j < 4:
        return float(q[j] & 63), float(q[j + 4] & 63)
    return (float((int(q[j + 4]) & 0x0F) | ((int(q[j - 4]) >> 6) << 4)),
            float((int(q[j + 4]) >> 4) | ((int(q[j]) >> 6) << 4)))


def ggml_q4k(data, d, dmin):
    """golden.rs:202-223."""
    scales, qs = data[4:16], data[16:]
    y = []
    for c in range(4):
        chunk = qs[32 * c:32 * c + 32]
        sc1, m1 = scale_min_k4(2 * c, scales)
        sc2, m2 = scale_min_k4(2 * c + 1, scales)
        y += [d * sc1 * float(int(q) & 0x0F) - dmin * m1 for q in chunk]
        y += [d * sc2 * float(int(q) >> 4) - dmin * m2 for q in chunk]
    return y


def test_golden_q4k():
    data = golden_block(144, 6, [(0, QUARTER), (2, HALF)])
    same(ko.dequantize(ko.Q4K, 0, data), ggml_q4k(data, 0.25, 0.5))


def ggml_q5k(data, d, dmin):
    """golden.rs:225-249."""
    scales, qh, qs = data[4:16], data[16:48], data[48:]
    y, u1, u2 = [], 1, 2
    for c in range(4):
        ql = qs[32 * c:]
        sc1, m1 = scale_min_k4(2 * c, scales)
        sc2, m2 = scale_min_k4(2 * c + 1, scales)
        for l in range(32):
            high = 16.0 if int(qh[l]) & u1 else 0.0
            y.append(d * sc1 * (float(int(ql[l]) & 0x0F) + high) - dmin * m1)
        for l in range(32):
            high = 16.0 if int(qh[l]) & u2 else 0.0
            y.append(d * sc2 * (float(int(ql[l]) >> 4) + high) - dmin * m2)
        u1 <<= 2
        u2 <<= 2
    return y


def test_golden_q5k():
    data = golden_block(176, 7, [(0, HALF), (2, QUARTER)])
    same(ko.dequantize(ko.Q5K, 0, data), ggml_q5k(data, 0.5, 0.25))


def ggml_q6k(data, d):
    """golden.rs:251-280."""
    ql_all, qh_all, sc_all = data[:128], data[128:192], data[192:208]
    y = [0.0] * 256
    for n in range(2):
        ql, qh, sc = ql_all[64 * n:], qh_all[32 * n:], sc_all[8 * n:]
        base = 128 * n
        s = lambda i: float(int(sc[i]) - 256 if sc[i] > 127 else int(sc[i]))
        code = lambda low, high: (low | (high & 3) << 4) - 32
        for l in range(32):
            is_ = l // 16
            q1 = code(int(ql[l]) & 0x0F, int(qh[l]))
            q2 = code(int(ql[l + 32]) & 0x0F, int(qh[l]) >> 2)
            q3 = code(int(ql[l]) >> 4, int(qh[l]) >> 4)
            q4 = code(int(ql[l + 32]) >> 4, int(qh[l]) >> 6)
            y[base + l] = d * s(is_) * float(q1)
            y[base + l + 32] = d * s(is_ + 2) * float(q2)
            y[base + l + 64] = d * s(is_ + 4) * float(q3)
            y[base + l + 96] = d * s(is_ + 6) * float(q4)
    return y


def test_golden_q6k():
    data = golden_block(210, 8, [(208, HALF)])
    same(ko.dequantize(ko.Q6K, 0, data), ggml_q6k(data, 0.5))
    by_hand = np.zeros(210, dtype=np.uint8)
    by_hand[192:208] = 1
    by_hand[192] = 0xFE  # -2
    by_hand[208:] = [0x00, 0x38]
    got = ko.dequantize(ko.Q6K, 0, by_hand)
    assert (got[0], got[15], got[16], got[255]) == (32.0, 32.0, -16.0, -16.0)


# ------------------------------------------- the non-linear IQ formats ---
# Their tables are format constants (ggml's kvalues_iq4nl and iq3s_grid);
# tests/golden/iq_tables.json holds them as kapel-core/src/iq.rs:7-78 gives
# them.  The transcriptions below follow GGML's dequantize_row_iq4_nl,
# _iq4_xs and _iq3_s loops (a group of 32 at a time, pairs of groups for
# IQ3_S), not the oracle's per-element formulas.

def iq_tables():
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "iq_tables.json")) as f:
        t = json.load(f)
    return t["iq4nl_values"], t["iq3s_grid"]


def test_iq_tables_are_the_formats_tables():
    values, grid = iq_tables()
    # What the formats fix: 16 increasing values of a signed byte; 512
    # distinct groups of four odd magnitudes 1..15 (3 bits each).
    assert len(values) == 16 and all(a < b for a, b in zip(values, values[1:]))
    assert values[0] == -127 and values[-1] == 113
    assert len(grid) == 512 and len(set(grid)) == 512
    for g in grid:
        for j in range(4):
            m = (g >> (8 * j)) & 0xFF
            assert m % 2 == 1 and 1 <= m <= 15
    # The oracle holds the same tables.
    assert [ko.iq_table(0, i) for i in range(16)] == values
    assert [ko.iq_table(1, i) for i in range(512)] == grid
    assert ko.iq_table(0, 16) == -1 and ko.iq_table(1, 512) == -1


def ggml_iq4_nl(data, d):
    values, _ = iq_tables()
    qs = data[2:18]
    y = [0.0] * 32
    for j in range(16):
        y[j] = d * values[qs[j] & 0xF]
        y[j + 16] = d * values[qs[j] >> 4]
    return y


def ggml_iq4_xs(data, d):
    values, _ = iq_tables()
    scales_h = int(data[2]) | int(data[3]) << 8
    scales_l, qs = data[4:8], data[8:136]
    y = []
    for ib in range(8):
        ls = ((int(scales_l[ib // 2]) >> 4 * (ib % 2)) & 0xF) | ((scales_h >> 2 * ib) & 3) << 4
        dl = d * (ls - 32)
        q = qs[16 * ib:16 * ib + 16]
        y += [dl * values[q[j] & 0xF] for j in range(16)]
        y += [dl * values[q[j] >> 4] for j in range(16)]
    return y


def ggml_iq3_s(data, d):
    _, grid = iq_tables()
    qs, qh, signs, scales = data[2:66], data[66:74], data[74:106], data[106:110]
    y = []
    q, s, h = 0, 0, 0
    for ib32 in range(0, 8, 2):
        for half in range(2):
            db = d * (1 + 2 * ((int(scales[ib32 // 2]) >> 4 * half) & 0xF))
            for l in range(4):
                g1 = grid[int(qs[q + 2 * l]) | ((int(qh[h + half]) << (8 - 2 * l)) & 256)]
                g2 = grid[int(qs[q + 2 * l + 1]) | ((int(qh[h + half]) << (7 - 2 * l)) & 256)]
                sg = int(signs[s + l])
                for j in range(4):
                    y.append(db * ((g1 >> 8 * j) & 0xFF) * (-1.0 if sg & (1 << j) else 1.0))
                for j in range(4):
                    y.append(db * ((g2 >> 8 * j) & 0xFF) * (-1.0 if sg & (1 << (j + 4)) else 1.0))
            q += 8
            s += 4
        h += 2
    return y


def test_golden_iq4_nl():
    data = golden_block(18, 9, [(0, HALF)])
    same(ko.dequantize(ko.IQ4_NL, 0, data), ggml_iq4_nl(data, 0.5))
    by_hand = np.array([0x00, 0x3C, 0xF0] + [0x87] * 15, dtype=np.uint8)
    got = ko.dequantize(ko.IQ4_NL, 0, by_hand)
    assert (got[0], got[16], got[1], got[17]) == (-127.0, 113.0, -10.0, 1.0)


def test_golden_iq4_xs():
    data = golden_block(136, 10, [(0, QUARTER)])
    same(ko.dequantize(ko.IQ4_XS, 0, data), ggml_iq4_xs(data, 0.25))
    by_hand = np.zeros(136, dtype=np.uint8)
    by_hand[0:2] = [0x00, 0x3C]          # d = 1
    by_hand[2:4] = [0x02, 0xC0]          # group 0: high bits 2; group 7: 3
    by_hand[4:8] = [0x01, 0, 0, 0xF0]    # group 0: low 1 -> s = 33; group 7: 15 | 48 = 63
    by_hand[8] = 0x0F                    # element 0: code 15, element 16: code 0
    got = ko.dequantize(ko.IQ4_XS, 0, by_hand)
    assert (got[0], got[16], got[1]) == (113.0, -127.0, -127.0)
    assert got[224] == 31.0 * -127.0 and got[32] == -32.0 * -127.0


def test_golden_iq3_s():
    data = golden_block(110, 11, [(0, HALF)])
    same(ko.dequantize(ko.IQ3_S, 0, data), ggml_iq3_s(data, 0.5))
    _, grid = iq_tables()
    by_hand = np.zeros(110, dtype=np.uint8)
    by_hand[0:2] = [0x00, 0x3C]          # d = 1
    by_hand[66] = 0x01                   # group 0, first index: + 256
    by_hand[74] = 0x01                   # element 0 negative
    by_hand[106] = 0x20                  # group 1: s = 2, scale 5
    got = ko.dequantize(ko.IQ3_S, 0, by_hand)
    first = [(grid[256] >> 8 * j) & 0xFF for j in range(4)]
    assert list(got[:4]) == [-first[0], first[1], first[2], first[3]]
    assert list(got[4:8]) == [1.0] * 4 and list(got[32:36]) == [5.0] * 4


# ----------------------------------------------------- dtype.rs tests ---

def test_kapel_formats_dequantize():
    # dtype.rs:920-934
    block = np.frombuffer(np.float32(0.5).tobytes() + bytes([0x0F, 0x80]), dtype=np.uint8)
    same(ko.dequantize(ko.INT4, 4, block), [3.5, -4.0, -4.0, 0.0])
    block = np.frombuffer(np.float32(2.0).tobytes() + bytes([0xFF, 0x02]), dtype=np.uint8)
    same(ko.dequantize(ko.INT8, 2, block), [-2.0, 4.0])


def test_q4_0_puts_low_nibbles_first():
    # dtype.rs:936-946
    block = np.array([0x00, 0x3C] + [(j % 16) | (15 - j % 16) << 4 for j in range(16)],
                     dtype=np.uint8)
    v = ko.dequantize(ko.Q4_0, 0, block)
    assert (v[0], v[15], v[16], v[31]) == (-8.0, 7.0, 7.0, -8.0)


def test_geometry():
    # dtype.rs:898-917 and the block sizes of :140-187
    assert ko.block_len(ko.INT4, 64) * 2 == 128 and ko.block_bytes(ko.INT4, 64) == 36
    assert 512 // ko.block_len(ko.Q4K) * ko.block_bytes(ko.Q4K) == 288
    sizes = {ko.Q8_0: 34, ko.Q4_0: 18, ko.Q4_1: 20, ko.Q5_0: 22, ko.Q5_1: 24, ko.Q2K: 84,
             ko.Q3K: 110, ko.Q4K: 144, ko.Q5K: 176, ko.Q6K: 210, ko.IQ4_NL: 18,
             ko.IQ4_XS: 136, ko.IQ3_S: 110}
    for fmt, size in sizes.items():
        assert ko.block_bytes(fmt) == size


QUANTIZED = [(ko.INT8, 32), (ko.INT4, 64), (ko.Q8_0, 0), (ko.Q4_0, 0), (ko.Q4_1, 0)]


def test_quantization_rounds_to_the_nearest_code():
    # dtype.rs:948-1027
    values = np.array([(i - 31.5) / 10.0 for i in range(64)], dtype=np.float32)
    for fmt, group in QUANTIZED:
        data = ko.quantize(fmt, group, values)
        assert data.size == 64 // ko.block_len(fmt, group) * ko.block_bytes(fmt, group)
        back = ko.dequantize(fmt, group, data)
        length = ko.block_len(fmt, group)
        top = {ko.Q4_0: 8.0, ko.Q4_1: 7.5}.get(fmt, 127.0)
        for b in range(64 // length):
            block = values[b * length:(b + 1) * length].astype(np.float64)
            got = back[b * length:(b + 1) * length]
            if fmt == ko.INT4:
                step = np.abs(block).max() / 7.0
                plain = sum((x - step * np.clip(np.round(x / step), -7, 7)) ** 2 for x in block)
                chosen = float(((block - got) ** 2).sum())
                assert chosen <= plain * (1 + 1e-9)
                continue
            if fmt == ko.Q4_1:
                step = (block.max() - block.min()) / 2.0 / top
            else:
                step = np.abs(block).max() / top
            slack = 0.07 if fmt in (ko.Q8_0, ko.Q4_0, ko.Q4_1) else 0.001
            assert np.all(np.abs(block - got) <= (0.5 + slack) * step)
    zeros = ko.quantize(ko.INT4, 32, np.zeros(32, np.float32))
    assert np.all(ko.dequantize(ko.INT4, 32, zeros) == 0.0)


def test_quantizer_hand_cases():
    # Q4_0 of 0..31 / 4: the largest magnitude 7.75 → d = −0.96875 (exact in
    # f16), code = floor(x / d + 8.5) clamped: x = 0 → 8, x = 7.75 → 0.
    x = np.arange(32, dtype=np.float32) / 4
    data = ko.quantize(ko.Q4_0, 0, x)
    assert ko.f16_decode(int(data[0]) | int(data[1]) << 8) == -0.96875
    codes = [int(data[2 + j]) & 0xF for j in range(16)] + [int(data[2 + j]) >> 4 for j in range(16)]
    assert codes[0] == 8 and codes[31] == 0
    # Each code is the nearest level: |x − d (c − 8)| ≤ d / 2.
    assert all(abs(x[i] - (-0.96875) * (codes[i] - 8)) <= 0.96875 / 2 + 1e-6 for i in range(32))
    # Q8_0 of a block whose largest magnitude is 127: d = 1, codes = round(x).
    x = np.linspace(-127, 127, 32).astype(np.float32)
    data = ko.quantize(ko.Q8_0, 0, x)
    assert ko.f16_decode(int(data[0]) | int(data[1]) << 8) == 1.0
    assert list(data[2:].view(np.int8)) == [int(np.copysign(np.floor(abs(v) + 0.5), v)) for v in x]
    # int8 rounds half away from zero: 0.5·(1/127·127) → 1, −2.5 → −3.
    x = np.zeros(32, np.float32); x[0] = 127.0; x[1] = 2.5; x[2] = -2.5; x[3] = 0.5
    data = ko.quantize(ko.INT8, 32, x)
    assert list(data[4:8].view(np.int8)) == [127, 3, -3, 1]


# ------------------------------------------- quantized.rs decoders/products

FORMATS = [(ko.INT8, 32), (ko.INT8, 40), (ko.INT4, 64), (ko.INT4, 40), (ko.Q8_0, 0),
           (ko.Q4_0, 0), (ko.Q4_1, 0), (ko.Q5_0, 0), (ko.Q5_1, 0), (ko.Q2K, 0), (ko.Q3K, 0),
           (ko.Q4K, 0), (ko.Q5K, 0), (ko.Q6K, 0), (ko.IQ4_NL, 0), (ko.IQ4_XS, 0),
           (ko.IQ3_S, 0)]

HALVES = {ko.Q8_0: [0], ko.Q4_0: [0], ko.Q5_0: [0], ko.Q4_1: [0, 2], ko.Q5_1: [0, 2],
          ko.Q4K: [0, 2], ko.Q5K: [0, 2], ko.Q2K: [80, 82], ko.Q3K: [108], ko.Q6K: [208],
          ko.IQ4_NL: [0], ko.IQ4_XS: [0], ko.IQ3_S: [0]}


def lcg_blocks(fmt, group, count, seed):
    """quantized.rs:1027-1062: random blocks with f16 scales at their places."""
    nxt = lcg_bytes(seed)
    size = ko.block_bytes(fmt, group)
    out = bytearray()
    for _ in range(count):
        block = bytearray(nxt() for _ in range(size))
        for at in HALVES.get(fmt, []):
            value = 0.001 + nxt() / 255.0 * 0.02
            h = ko.f16_encode(value)
            block[at], block[at + 1] = h & 0xFF, h >> 8
        if fmt in (ko.INT8, ko.INT4):
            block[:4] = np.float32(0.0125).tobytes()
        out += block
    return np.frombuffer(bytes(out), dtype=np.uint8)


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_blocks_decode_as_the_reference(fmt, group):
    # quantized.rs:1097-1122
    data = lcg_blocks(fmt, group, 3, 7)
    expected = ko.dequantize(fmt, group, data)
    size, length = ko.block_bytes(fmt, group), ko.block_len(fmt, group)
    for b in range(3):
        got = ko.decode_f32(fmt, group, data[b * size:(b + 1) * size]).astype(np.float64)
        e = expected[b * length:(b + 1) * length]
        assert np.all(np.abs(got - e) <= 1e-6 * np.maximum(np.abs(e), 1e-3))


@pytest.mark.parametrize("fmt,group", FORMATS)
def test_products_match_the_dequantized_weights_on_any_threads(fmt, group):
    # quantized.rs:1150-1191
    n, k, rows = 37, 1280, 11
    i = np.arange(rows * k)
    x = (((i * 7919) % 201).astype(np.float32) / np.float32(100.0) - np.float32(1.0))
    x = x.reshape(rows, k)
    w = lcg_blocks(fmt, group, n * k // ko.block_len(fmt, group), 11)
    dense = ko.dequantize(fmt, group, w).reshape(n, k)
    e = x.astype(np.float64) @ dense.T
    first = None
    for threads in (1, 3):
        out = ko.product_f32([(fmt, group, w, n)], k, x, threads)
        assert np.all(np.abs(out - e) <= 1e-4 * (1 + np.abs(e)))
        if first is None:
            first = out
        else:
            assert np.array_equal(first.view(np.uint32), out.view(np.uint32))


def test_stacked_weights_and_empty_shapes():
    # conformity.rs:936-947 (stacked q4_k/q6_k/q8_0) and :1414-1430 (empty).
    rng = Rng(3)
    k = 512
    stack = []
    for fmt, n in ((ko.Q4K, 5), (ko.Q6K, 3), (ko.Q8_0, 2)):
        stack.append((fmt, 0, lcg_blocks(fmt, 0, n * k // ko.block_len(fmt), 5 + n), n))
    for rows in (1, 3, 17):
        x = np.array([[rng.uniform(-1, 1) for _ in range(k)] for _ in range(rows)], np.float32)
        e = ko.product_f64(stack, k, x)
        got = ko.product_f32(stack, k, x, 2)
        assert np.all(np.abs(got - e) <= 1e-4 * max(1.0, np.abs(e).max()))
    # K = 0: zeros; no rows or no weight rows: empty.
    w0 = np.zeros(0, np.uint8)
    assert np.all(ko.product_f32([(ko.Q8_0, 0, w0, 5)], 0, np.zeros((3, 0), np.float32)) == 0)
    assert ko.product_f32([(ko.Q8_0, 0, w0, 0)], 64, np.zeros((3, 64), np.float32)).shape == (3, 0)


# ------------------------------------------------------ byte activations

BYTE_FORMATS = [(ko.Q8_0, 0), (ko.Q4_0, 0), (ko.Q4K, 0), (ko.Q5K, 0), (ko.Q6K, 0),
                (ko.INT8, 32), (ko.INT8, 128), (ko.INT4, 32), (ko.INT4, 64)]


def byte_blocks(fmt, group, count, seed):
    """bytes.rs:680-707."""
    nxt = lcg_bytes(seed)
    size = ko.block_bytes(fmt, group)
    halves = {ko.Q8_0: [0], ko.Q4_0: [0], ko.Q4K: [0, 2], ko.Q5K: [0, 2], ko.Q6K: [208]}.get(fmt, [])
    out = bytearray()
    for _ in range(count):
        block = bytearray(nxt() for _ in range(size))
        for at in halves:
            h = ko.f16_encode(0.001 + nxt() / 255.0 * 0.02)
            block[at], block[at + 1] = h & 0xFF, h >> 8
        if not halves:
            block[:4] = np.float32(0.0125).tobytes()
        out += block
    return np.frombuffer(bytes(out), dtype=np.uint8)


def byte_x(rows, k):
    i = np.arange(rows * k)
    base = ((i * 7919) % 201).astype(np.float32) / np.float32(100.0) - np.float32(1.0)
    return (base * (1 + (i // 32) % 7).astype(np.float32)).reshape(rows, k)


def test_activation_bytes_closed_form():
    # bytes.rs:144-158: s = max|x| / 127, q = round-half-even(x · 127/max).
    x = byte_x(3, 256)
    x[0, :32] = 0.0          # a block of zeros: scale 0, codes 0
    x[1, 32:64] = np.linspace(-1, 1, 32, dtype=np.float32)
    x[2, 0] = 127.0 / 2 * 0 + 2.5  # ties: 2.5·(127/2.5) = 127 exactly
    q, s, sums = ko.quantize_x(x)
    for r in range(3):
        for b in range(8):
            v = x[r, 32 * b:32 * b + 32]
            m = np.float32(np.abs(v).max())
            assert s[r, b] == np.float32(m / np.float32(127.0))
            inv = np.float32(127.0) / m if m > 0 else np.float32(0.0)
            want = np.clip(np.rint(v * inv), -127, 127).astype(np.int8)  # rint: half to even
            assert np.array_equal(q[r, 32 * b:32 * b + 32], want)
            assert sums[r, b] == np.float32(s[r, b] * np.float32(int(want.astype(np.int32).sum())))
    assert np.all(q[0, :32] == 0) and s[0, 0] == 0.0
    # A tie at exactly .5 goes to even: 0.5 → 0, 1.5 → 2, −2.5 → −2.
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [127.0, 0.5, 1.5, -2.5]
    q, s, _ = ko.quantize_x(x)
    assert list(q[0, :4]) == [127, 0, 2, -2]


def byte_codes(fmt, group, block):
    """The integer codes of one block, by GGML's loop orders (golden.rs
    transcriptions): the values that bytes.rs:282-353 decodes."""
    b = [int(v) for v in block]
    if fmt == ko.Q8_0:
        return [v - 256 if v > 127 else v for v in b[2:34]]
    if fmt == ko.Q4_0:
        return [v & 15 for v in b[2:18]] + [v >> 4 for v in b[2:18]]
    if fmt in (ko.Q4K, ko.Q5K):
        qh, qs = (b[16:48], b[48:176]) if fmt == ko.Q5K else (None, b[16:144])
        out, u1, u2 = [], 1, 2
        for c in range(4):
            ql = qs[32 * c:]
            out += [(ql[l] & 15) + (16 if qh and qh[l] & u1 else 0) for l in range(32)]
            out += [(ql[l] >> 4) + (16 if qh and qh[l] & u2 else 0) for l in range(32)]
            u1 <<= 2
            u2 <<= 2
        return out
    if fmt == ko.Q6K:
        out = [0] * 256
        for n in range(2):
            ql, qh = b[64 * n:], b[128 + 32 * n:]
            for l in range(32):
                out[128 * n + l] = ((ql[l] & 15) | (qh[l] & 3) << 4) - 32
                out[128 * n + l + 32] = ((ql[l + 32] & 15) | ((qh[l] >> 2) & 3) << 4) - 32
                out[128 * n + l + 64] = ((ql[l] >> 4) | ((qh[l] >> 4) & 3) << 4) - 32
                out[128 * n + l + 96] = ((ql[l + 32] >> 4) | ((qh[l] >> 6) & 3) << 4) - 32
        return out
    if fmt == ko.INT8:
        return [v - 256 if v > 127 else v for v in b[4:4 + group]]
    if fmt == ko.INT4:
        out = []
        for v in b[4:4 + group // 2]:
            out += [v & 15, v >> 4]
        return out
    raise ValueError(fmt)


@pytest.mark.parametrize("fmt,group", BYTE_FORMATS)
def test_products_are_those_of_the_activations_in_bytes(fmt, group):
    # bytes.rs:720-774, plus the exact i32 block dots.
    n, k, rows = 13, 1024, 6
    x = byte_x(rows, k)
    w = byte_blocks(fmt, group, n * k // ko.block_len(fmt, group), 3)
    dense = ko.dequantize(fmt, group, w).reshape(n, k)
    out, dots = ko.product_bytes([(fmt, group, w, n)], k, x, threads=3, with_dots=True)
    q, s, _ = ko.quantize_x(x)
    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    e = xq @ dense.T
    size = np.abs(xq) @ np.abs(dense).T
    assert np.all(np.abs(out - e) <= 1e-5 * size + 1e-6)
    # Brute-force dots on codes unpacked independently of the oracle.
    length, bsize = ko.block_len(fmt, group), ko.block_bytes(fmt, group)
    width = 16 if fmt == ko.Q6K else 32
    codes = np.array([byte_codes(fmt, group, w[i * bsize:(i + 1) * bsize])
                      for i in range(n * k // length)], dtype=np.int64).reshape(n, k)
    for r in range(rows):
        for j in range(n):
            prod = codes[j] * q[r].astype(np.int64)
            want = prod.reshape(-1, width).sum(axis=1)
            got = dots[r, j].reshape(-1, width // 16)[:, 0]
            assert np.array_equal(got, want), (r, j)
    # Results do not depend on the thread count.
    again = ko.product_bytes([(fmt, group, w, n)], k, x, threads=1)
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32))


def test_golden_fixture_matches_the_oracle():
    """tests/golden/golden_blocks.json (written by make_golden.py from the
    GGML transcriptions above) decodes exactly under the oracle."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "golden_blocks.json")) as f:
        cases = json.load(f)
    assert len(cases) == 11
    for case in cases:
        data = np.frombuffer(bytes.fromhex(case["bytes"]), dtype=np.uint8)
        same(ko.dequantize(case["format"], 0, data), case["values"])


# ------------------------------------------------------------- experts ---

@pytest.mark.parametrize("fmt", [ko.Q8_0, ko.IQ4_XS, ko.IQ3_S, ko.Q4K])
@pytest.mark.parametrize("per_route", [False, True])
def test_expert_product_is_the_reference_definition(fmt, per_route):
    """conformity.rs:975-990: [5, K] or [5, 3, K] by 3 of 4 experts of
    [7, 256]; against kapel-ref/src/experts.rs:64-90 (the f64 definition,
    written here over the dequantized weights), and each route bitwise the
    f32 product of its own row by its expert alone."""
    k, n, experts, tokens, topk = 256, 7, 4, 5, 3
    w = lcg_blocks(fmt, 0, experts * n * k // ko.block_len(fmt), 31)
    rng = np.random.default_rng(4)
    idx = rng.integers(0, experts, size=(tokens, topk))
    shape = (tokens, topk, k) if per_route else (tokens, k)
    x = rng.uniform(-1, 1, size=shape).astype(np.float32)
    got = ko.expert_product(fmt, 0, w, experts, k, x, idx)
    dense = ko.dequantize(fmt, 0, w).reshape(experts, n, k)
    size = n * ko.row_bytes(fmt, 0, k)
    for t in range(tokens):
        for j in range(topk):
            row = x[t, j] if per_route else x[t]
            e = row.astype(np.float64) @ dense[idx[t, j]].T
            assert np.all(np.abs(got[t, j] - e) <= 1e-4 * (1 + np.abs(e))), (t, j)
            alone = ko.product_f32([(fmt, 0, w[idx[t, j] * size:(idx[t, j] + 1) * size], n)], k,
                                   row[None])
            assert np.array_equal(got[t, j].view(np.uint32), alone[0].view(np.uint32)), (t, j)


def test_expert_product_in_bytes():
    """The byte product by experts: within the bound of bytes.rs:753-770 of
    the exact product of the quantized activations."""
    k, n, experts = 512, 9, 3
    w = lcg_blocks(ko.Q4K, 0, experts * n * k // 256, 5)
    idx = np.array([[2, 0], [1, 2], [2, 2]])
    x = np.random.default_rng(8).uniform(-1, 1, size=(3, k)).astype(np.float32)
    got = ko.expert_product(ko.Q4K, 0, w, experts, k, x, idx, byte_activations=True)
    q, s, _ = ko.quantize_x(x)
    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    dense = ko.dequantize(ko.Q4K, 0, w).reshape(experts, n, k)
    for t in range(3):
        for j in range(2):
            d = dense[idx[t, j]]
            e = xq[t] @ d.T
            bound = 1e-5 * (np.abs(xq[t]) @ np.abs(d).T) + 1e-6
            assert np.all(np.abs(got[t, j] - e) <= bound), (t, j)


# ------------------------------------------- AVX-512 kernels (CPU baseline) ---

WIDE, VNNI = ko.wide_available()


@pytest.mark.skipif(not WIDE, reason="this host has no AVX-512")
@pytest.mark.parametrize("fmt", ko.WIDE_FORMATS)
def test_wide_products_match_the_dequantized_weights(fmt):
    # quantized.rs:1150-1191 run on the AVX-512 kernels: 11 rows take the
    # 8-, 2- and 1-row instances.
    n, k, rows = 37, 1280, 11
    i = np.arange(rows * k)
    x = (((i * 7919) % 201).astype(np.float32) / np.float32(100.0) - np.float32(1.0)).reshape(rows, k)
    w = lcg_blocks(fmt, 0, n * k // ko.block_len(fmt), 11)
    e = x.astype(np.float64) @ ko.dequantize(fmt, 0, w).reshape(n, k).T
    one = ko.product_wide([(fmt, 0, w, n)], k, x, threads=1)
    assert np.all(np.abs(one - e) <= 1e-4 * (1 + np.abs(e)))
    three = ko.product_wide([(fmt, 0, w, n)], k, x, threads=3)
    assert np.array_equal(one.view(np.uint32), three.view(np.uint32))
    # A dropped term or a wrong segment would be far from the portable kernel.
    port = ko.product_f32([(fmt, 0, w, n)], k, x)
    assert np.all(np.abs(one - port) <= 1e-4 * (1 + np.abs(port)))


@pytest.mark.skipif(not VNNI, reason="this host has no AVX-512 VNNI")
@pytest.mark.parametrize("fmt", ko.WIDE_FORMATS)
@pytest.mark.parametrize("rows", [7, 6])
def test_vnni_products_are_those_of_the_activations_in_bytes(fmt, rows):
    # bytes.rs:720-774 on the VNNI kernels (views of 4 and 3, or 4 and 2 rows).
    n, k = 13, 1024
    x = byte_x(rows, k)
    w = byte_blocks(fmt, 0, n * k // ko.block_len(fmt), 3)
    dense = ko.dequantize(fmt, 0, w).reshape(n, k)
    q, s, _ = ko.quantize_x(x)
    xq = np.repeat(s.astype(np.float64), 32, axis=1) * q.astype(np.float64)
    e, size = xq @ dense.T, np.abs(xq) @ np.abs(dense).T
    out = ko.product_vnni([(fmt, 0, w, n)], k, x, threads=3)
    assert np.all(np.abs(out - e) <= 1e-5 * size + 1e-6)
    port = ko.product_bytes([(fmt, 0, w, n)], k, x)
    assert np.all(np.abs(out - port) <= 1e-5 * size + 1e-6)
    again = ko.product_vnni([(fmt, 0, w, n)], k, x, threads=1)
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32))
