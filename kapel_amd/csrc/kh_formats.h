// Device readers of the quantized block formats, shaped for the int8 MFMA
// v_mfma_i32_16x16x64_i8 of gfx950.
//
// The product walks each weight row by "steps" of 64 elements.  In a step,
// lane group g (lanes 16g .. 16g+15, one weight row each) supplies 16 byte
// codes, four dwords d = 0..3, as the B operand.  Each dword holds the codes
// of four consecutive elements, which belong to one "group": a run of 32 (or
// 16) elements sharing a scale and a minimum, and lying in one block of 32
// activations.  A format says, for each (step, lane group, dword), which
// elements the codes are (`xoff`) and which of its NGRP groups they are in
// (`grp`), and gives each group's scale and minimum:
//
//     w = scale * code - minimum.
//
// Codes are the format's stored codes, made unsigned where the format
// subtracts an offset (Q6_K's 32, Q3_K's 4, Q5_0's 16): the offset goes into
// the minimum.  Q4_0 and int4 keep codes 0..15 with minimum 8 * scale, as
// kapel-cpu/src/bytes.rs:296-303, :342-348 does.
//
// Scales and minimums are the f32 products of kapel-cpu/src/quantized.rs
// (k_scales :603-616 and the per-format decoders :403-682).  Element layouts
// follow kapel-core/src/dtype.rs:342-520.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kh {

typedef int v4i __attribute__((ext_vector_type(4)));

// Loads.  Every load reads exactly its bytes at their natural alignment:
// blocks of 18, 22, 34, 110 and 210 bytes start at even addresses only, and
// Kapel's groups of odd size at any address.
__device__ __forceinline__ uint16_t ld16(const uint8_t *p) {  // p even
    return *reinterpret_cast<const uint16_t *>(p);
}
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {  // p a multiple of 4
    return *reinterpret_cast<const uint32_t *>(p);
}
__device__ __forceinline__ uint2 ld64(const uint8_t *p) {  // p a multiple of 4
    if (((uintptr_t)p & 7u) == 0) return *reinterpret_cast<const uint2 *>(p);
    return uint2{ld32(p), ld32(p + 4)};
}
// p even.
__device__ __forceinline__ uint32_t ld32e(const uint8_t *p) {
    if (((uintptr_t)p & 3u) == 0) return ld32(p);
    return (uint32_t)ld16(p) | ((uint32_t)ld16(p + 2) << 16);
}
__device__ __forceinline__ uint2 ld64e(const uint8_t *p) {
    if (((uintptr_t)p & 3u) == 0) return ld64(p);
    uint32_t mid = ld32(p + 2);
    return uint2{(uint32_t)ld16(p) | (mid << 16), (mid >> 16) | ((uint32_t)ld16(p + 6) << 16)};
}
// Any address.
__device__ __forceinline__ uint32_t ld32b(const uint8_t *p) {
    if (((uintptr_t)p & 3u) == 0) return ld32(p);
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ __forceinline__ float ldf32(const uint8_t *p) { return __uint_as_float(ld32b(p)); }

// IEEE half to f32, exactly, with integer operations only (independent of
// the denormal mode): kapel-cpu/src/quantized.rs:386-396 gives the same value.
__device__ __forceinline__ float h2f(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1fu) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e == 0) return __uint_as_float(sign) + (sign ? -1.0f : 1.0f) * __builtin_ldexpf((float)m, -24);
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

__device__ __forceinline__ float half_at(const uint8_t *p) { return h2f(ld16(p)); }

constexpr uint32_t LO4 = 0x0f0f0f0fu;

// ------------------------------------------------------------------ Q4_K
// 256 elements, 144 bytes: d, dmin, 12 bytes of 6-bit scales/minimums, 128
// bytes of nibbles (dtype.rs:441-457).  Step t: super-block t/4, chunk c = t%4
// of 32 bytes, whose low nibbles are sub-block 2c and high nibbles 2c+1.
// Lane group g takes bytes 8g .. 8g+7 of the chunk.
struct Q4K {
    static constexpr int LEN = 256, BYTES = 144, NGRP = 2, GS = 32;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        uint2 w = ld64(blk + 16 + (t & 3) * 32 + 8 * g);
        return v4i{(int)(w.x & LO4), (int)(w.y & LO4), (int)((w.x >> 4) & LO4),
                   (int)((w.y >> 4) & LO4)};
    }
    __device__ static int xoff(int t, int g, int d) {
        return (t >> 2) * 256 + (t & 3) * 64 + (d >> 1) * 32 + 8 * g + (d & 1) * 4;
    }
    __device__ static int gelem(int t, int grp) { return (t >> 2) * 256 + (t & 3) * 64 + 32 * grp; }
    // k_scales (quantized.rs:603-616) for sub-block j.
    __device__ static void kscale(const uint8_t *blk, int j, float &s, float &m) {
        float d = half_at(blk), dmin = half_at(blk + 2);
        const uint8_t *p = blk + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = p[j] & 63u;
            mn = p[j + 4] & 63u;
        } else {
            sc = (p[j + 4] & 15u) | ((p[j - 4] >> 6) << 4);
            mn = (p[j + 4] >> 4) | ((p[j] >> 6) << 4);
        }
        s = d * (float)sc;
        m = dmin * (float)mn;
    }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        kscale(row + (t >> 2) * BYTES, 2 * (t & 3) + grp, s, m);
    }
};

// ------------------------------------------------------------------ Q5_K
// 176 bytes: as Q4_K, with 32 bytes of fifth bits after the scales: bit
// e / 32 of byte e % 32 (dtype.rs:441-457).
struct Q5K {
    static constexpr int LEN = 256, BYTES = 176, NGRP = 2, GS = 32;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        int c = t & 3;
        uint2 w = ld64(blk + 48 + c * 32 + 8 * g);
        uint2 h = ld64(blk + 16 + 8 * g);
        uint32_t h0 = (h.x >> (2 * c)) & 0x01010101u, h1 = (h.y >> (2 * c)) & 0x01010101u;
        uint32_t k0 = (h.x >> (2 * c + 1)) & 0x01010101u, k1 = (h.y >> (2 * c + 1)) & 0x01010101u;
        return v4i{(int)((w.x & LO4) | (h0 << 4)), (int)((w.y & LO4) | (h1 << 4)),
                   (int)(((w.x >> 4) & LO4) | (k0 << 4)), (int)(((w.y >> 4) & LO4) | (k1 << 4))};
    }
    __device__ static int xoff(int t, int g, int d) { return Q4K::xoff(t, g, d); }
    __device__ static int gelem(int t, int grp) { return Q4K::gelem(t, grp); }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        Q4K::kscale(row + (t >> 2) * BYTES, 2 * (t & 3) + grp, s, m);
    }
};

// ------------------------------------------------------------------ Q6_K
// 210 bytes: 128 bytes of low nibbles, 64 of 2-bit highs, 16 signed scales,
// d (dtype.rs:458-469).  Element h*128 + s*32 + l: low nibble s/2 of byte
// h*64 + (s%2)*32 + l, high bits 2s of byte 128 + h*32 + l; scale of group
// (h*128 + 32s + l) / 16.  Step t: super-block t/4, h = (t%4)/2, u = t%2: the
// 64 elements h*128 + 32s + 16u + (0..15), s = 0..3, in four groups of 16;
// lane group g takes l = 16u + 4g .. +3 of each s (dword d = s).
struct Q6K {
    static constexpr int LEN = 256, BYTES = 210, NGRP = 4, GS = 16;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        int h = (t >> 1) & 1, l0 = 16 * (t & 1) + 4 * g;
        uint32_t a0 = ld32e(blk + h * 64 + l0), a1 = ld32e(blk + h * 64 + 32 + l0);
        uint32_t q = ld32e(blk + 128 + h * 32 + l0);
        return v4i{(int)((a0 & LO4) | ((q << 4) & 0x30303030u)),
                   (int)((a1 & LO4) | ((q << 2) & 0x30303030u)),
                   (int)(((a0 >> 4) & LO4) | (q & 0x30303030u)),
                   (int)(((a1 >> 4) & LO4) | ((q >> 2) & 0x30303030u))};
    }
    __device__ static int xoff(int t, int g, int d) {
        return (t >> 2) * 256 + ((t >> 1) & 1) * 128 + 32 * d + 16 * (t & 1) + 4 * g;
    }
    __device__ static int gelem(int t, int grp) {
        return (t >> 2) * 256 + ((t >> 1) & 1) * 128 + 32 * grp + 16 * (t & 1);
    }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        int index = ((t >> 1) & 1) * 8 + 2 * grp + (t & 1);
        s = half_at(blk + 208) * (float)(int8_t)blk[192 + index];
        m = 32.0f * s;  // codes stored with +32
    }
};

// ------------------------------------------------------------------ Q2_K
// 84 bytes: 16 scale bytes (low nibble scale, high nibble minimum), 64 bytes
// of 2-bit codes, d, dmin (dtype.rs:413-422).  Element h*128 + s*32 + l: bits
// 2s of byte 16 + h*32 + l; group e / 16.  Steps as Q6_K.
struct Q2K {
    static constexpr int LEN = 256, BYTES = 84, NGRP = 4, GS = 16;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        uint32_t q = ld32(blk + 16 + ((t >> 1) & 1) * 32 + 16 * (t & 1) + 4 * g);
        return v4i{(int)(q & 0x03030303u), (int)((q >> 2) & 0x03030303u),
                   (int)((q >> 4) & 0x03030303u), (int)((q >> 6) & 0x03030303u)};
    }
    __device__ static int xoff(int t, int g, int d) { return Q6K::xoff(t, g, d); }
    __device__ static int gelem(int t, int grp) { return Q6K::gelem(t, grp); }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        uint32_t k = blk[((t >> 1) & 1) * 8 + 2 * grp + (t & 1)];
        s = half_at(blk + 80) * (float)(k & 15u);
        m = half_at(blk + 82) * (float)(k >> 4);
    }
};

// ------------------------------------------------------------------ Q3_K
// 110 bytes: 32 bytes of high-bit masks, 64 of 2-bit codes, 12 of packed
// 6-bit scales, d (dtype.rs:423-440).  Element h*128 + s*32 + l: low bits 2s
// of byte 32 + h*32 + l, high bit 4h + s of byte l; the value is
// d * scale * (low - 4 (1 - high)) = d * scale * ((low | high << 2) - 4).
struct Q3K {
    static constexpr int LEN = 256, BYTES = 110, NGRP = 4, GS = 16;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        int h = (t >> 1) & 1, l0 = 16 * (t & 1) + 4 * g;
        uint32_t q = ld32e(blk + 32 + h * 32 + l0), mk = ld32e(blk + l0) >> (4 * h);
        return v4i{(int)((q & 0x03030303u) | ((mk << 2) & 0x04040404u)),
                   (int)(((q >> 2) & 0x03030303u) | ((mk << 1) & 0x04040404u)),
                   (int)(((q >> 4) & 0x03030303u) | (mk & 0x04040404u)),
                   (int)(((q >> 6) & 0x03030303u) | ((mk >> 1) & 0x04040404u))};
    }
    __device__ static int xoff(int t, int g, int d) { return Q6K::xoff(t, g, d); }
    __device__ static int gelem(int t, int grp) { return Q6K::gelem(t, grp); }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        const uint8_t *blk = row + (t >> 2) * BYTES;
        const uint8_t *packed = blk + 96;
        int i = ((t >> 1) & 1) * 8 + 2 * grp + (t & 1);
        uint32_t lo = (packed[i % 8] >> (4 * (i / 8))) & 15u;
        uint32_t hi = (packed[8 + i % 4] >> (2 * (i / 4))) & 3u;
        s = half_at(blk + 108) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
        m = 4.0f * s;  // codes stored with +4
    }
};

// ------------------------------------------------------ 32-element blocks
// A step is two blocks, 2t and 2t+1 (the second absent when K % 64 == 32:
// `two` is false and its codes are zero).  Groups are the blocks.

// Codes of a Q4_0-like block (a byte holds element j low, j + 16 high), lane
// group g: dword 4g .. 4g+3 -> elements 4g+i (low) and 16+4g+i (high).
__device__ __forceinline__ int2 nib32(uint32_t w) {
    return int2{(int)(w & LO4), (int)((w >> 4) & LO4)};
}
__device__ __forceinline__ v4i join(int2 a, int2 b) { return v4i{a.x, a.y, b.x, b.y}; }
__device__ __forceinline__ int xoff_nib32(int t, int g, int d) {
    return 64 * t + 32 * (d >> 1) + 16 * (d & 1) + 4 * g;
}
__device__ __forceinline__ int xoff_seq32(int t, int g, int d) {
    return 64 * t + 32 * (d >> 1) + 8 * g + 4 * (d & 1);
}

// Q4_0: 18 bytes, d then 16 bytes of nibbles; w = d (q - 8) (dtype.rs:379-391).
struct Q4_0 {
    static constexpr int LEN = 32, BYTES = 18, NGRP = 2, GS = 32;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        const uint8_t *b0 = row + 2 * t * BYTES;
        return join(nib32(ld32e(b0 + 2 + 4 * g)),
                    two ? nib32(ld32e(b0 + BYTES + 2 + 4 * g)) : int2{0, 0});
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_nib32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        s = half_at(row + (2 * t + grp) * BYTES);
        m = 8.0f * s;
    }
};

// Q4_1: 20 bytes, d, m then nibbles; w = d q + m.
struct Q4_1 {
    static constexpr int LEN = 32, BYTES = 20, NGRP = 2, GS = 32;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        const uint8_t *b0 = row + 2 * t * BYTES;
        return join(nib32(ld32(b0 + 4 + 4 * g)),
                    two ? nib32(ld32(b0 + BYTES + 4 + 4 * g)) : int2{0, 0});
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_nib32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        const uint8_t *blk = row + (2 * t + grp) * BYTES;
        s = half_at(blk);
        m = -half_at(blk + 2);
    }
};

// Fifth bits of Q5_0/Q5_1: bits j .. j+3 of `high` spread to bit 4 of bytes.
__device__ __forceinline__ uint32_t spread4(uint32_t high, int j) {
    uint32_t x = (high >> j) & 15u;
    return ((x * 0x00204081u) & 0x01010101u) << 4;
}

template <int OFFSET, bool MIN>
struct Q5x {
    static constexpr int LEN = 32, BYTES = MIN ? 24 : 22, NGRP = 2, GS = 32;
    __device__ static int2 one(const uint8_t *blk, int g) {
        uint32_t high = ld32e(blk + OFFSET), w = ld32e(blk + OFFSET + 4 + 4 * g);
        return int2{(int)((w & LO4) | spread4(high, 4 * g)),
                    (int)(((w >> 4) & LO4) | spread4(high, 16 + 4 * g))};
    }
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        const uint8_t *b0 = row + 2 * t * BYTES;
        return join(one(b0, g), two ? one(b0 + BYTES, g) : int2{0, 0});
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_nib32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        const uint8_t *blk = row + (2 * t + grp) * BYTES;
        s = half_at(blk);
        m = MIN ? -half_at(blk + 2) : 16.0f * s;
    }
};
using Q5_0 = Q5x<2, false>;  // 22 bytes: d, qh, nibbles; w = d (q - 16)
using Q5_1 = Q5x<4, true>;   // 24 bytes: d, m, qh, nibbles; w = d q + m

// Q8_0: 34 bytes, d then 32 signed bytes (dtype.rs:375-378).
struct Q8_0 {
    static constexpr int LEN = 32, BYTES = 34, NGRP = 2, GS = 32;
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        const uint8_t *b0 = row + 2 * t * BYTES;
        uint2 a = ld64e(b0 + 2 + 8 * g);
        uint2 b = two ? ld64e(b0 + BYTES + 2 + 8 * g) : uint2{0u, 0u};
        return v4i{(int)a.x, (int)a.y, (int)b.x, (int)b.y};
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_seq32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        s = half_at(row + (2 * t + grp) * BYTES);
        m = 0.0f;
    }
};

// Kapel int8 / int4 with groups of G (a multiple of 32): an f32 scale then
// G bytes, or G/2 bytes of nibbles (element 2i low, 2i+1 high)
// (dtype.rs:364-374).  Piece p (32 elements) is in block 32p / G.
template <int G>
struct Int8G {
    static constexpr int LEN = G, BYTES = 4 + G, NGRP = 2, GS = 32;
    __device__ static const uint8_t *piece(const uint8_t *row, int p) {
        return row + (32 * p / G) * BYTES + 4 + (32 * p) % G;
    }
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        uint2 a = ld64(piece(row, 2 * t) + 8 * g);
        uint2 b = two ? ld64(piece(row, 2 * t + 1) + 8 * g) : uint2{0u, 0u};
        return v4i{(int)a.x, (int)a.y, (int)b.x, (int)b.y};
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_seq32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        s = ldf32(row + (32 * (2 * t + grp) / G) * BYTES);
        m = 0.0f;
    }
};

template <int G>
struct Int4G {
    static constexpr int LEN = G, BYTES = 4 + G / 2, NGRP = 2, GS = 32;
    __device__ static const uint8_t *piece(const uint8_t *row, int p) {
        return row + (32 * p / G) * BYTES + 4 + ((32 * p) % G) / 2;
    }
    // Bytes 4g .. 4g+3 of the piece: elements 8g .. 8g+7, interleaved
    // low/high; put back in order.
    __device__ static int2 one(const uint8_t *pc, int g) {
        uint32_t w = ld32(pc + 4 * g);
        uint32_t lo = w & LO4, hi = (w >> 4) & LO4;
        return int2{(int)__builtin_amdgcn_perm(hi, lo, 0x05010400u),
                    (int)__builtin_amdgcn_perm(hi, lo, 0x07030602u)};
    }
    __device__ static v4i codes(const uint8_t *row, int t, int g, bool two) {
        return join(one(piece(row, 2 * t), g), two ? one(piece(row, 2 * t + 1), g) : int2{0, 0});
    }
    __device__ static int xoff(int t, int g, int d) { return xoff_seq32(t, g, d); }
    __device__ static int gelem(int t, int grp) { return 64 * t + 32 * grp; }
    __device__ static void scale_min(const uint8_t *row, int t, int grp, float &s, float &m) {
        s = ldf32(row + (32 * (2 * t + grp) / G) * BYTES);
        m = 8.0f * s;
    }
};

}  // namespace kh
