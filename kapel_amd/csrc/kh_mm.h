// The product by quantized weights for many activation rows (batched decode
// and prefill) on gfx950.
//
// The activations come prepared (prep_x_kernel): per row, int8 planes over K
// (one plane: the CPU's bytes, kapel-cpu/src/bytes.rs:144-158; three planes:
// a 23-bit fixed-point image of f32 activations) with per-32 scales and
// per-group sums.  Output element y[m, n] is then, group g by group,
//
//     y[m, n] = sum_g xscale[m, g] * wscale[n, g] * dot_g(m, n)
//             - sum_g minimum[n, g] * xsum[m, g]
//
// (bytes.rs:200-241), with dot_g the integer dot of the group's codes and
// activation bytes.  A workgroup of four waves takes 32 or 64 activation rows
// by 256 weight rows; each wave 32 or 64 rows by 64 weight rows, in tiles of
// 32 x 32.  Per group of 32 (or 16) elements and tile:
//
//   - dot_g for the whole tile: v_mfma_i32_32x32x32_i8 (32x32x16 for the
//     groups of 16), exact;
//   - the scale of each (m, n): xscale (x) wscale as an outer product,
//     v_mfma_f32_32x32x2_f32 with the second k-slot zero; exact f32
//     products, in the same lane layout as the dots;
//   - one cvt and one fma per element on the VALU;
//   - the minimum term of the formats that have one: a product over pairs
//     of groups, v_mfma_f32_32x32x2_f32 into a sum of the unit's, added to
//     the sums at the end of the unit.
//
// Weights, activation planes, scales and sums of a unit are copied from
// memory into a ring of two or three LDS stages by direct loads (buffer_load
// ... lds), the loads of later units in flight while a unit is multiplied
// (one barrier per unit); the lane readers below read the weights from LDS.
// Codes are signed where the format's offset is fixed (Q4_0 - 8, Q5_0 - 16,
// Q6_K - 32, Q3_K - 4, int4 - 8), so those formats have no minimum term.
//
// Every sum runs in an order fixed by the shapes: groups in K order within a
// workgroup, then the K splits (chosen from the shapes alone) in order by
// the reduction kernel.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_gemv.h"
#include "kh_internal.h"
#include "kh_lanes.h"

namespace kh {
namespace mm {

using lanes::f16;
using lanes::LO4;
using lanes::NONE;
using lanes::Src;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Lane (c, h) of a wave, c = lane % 32, h = lane / 32, supplies weight row c
// of a 32-row tile and half h of each group: elements 16h .. 16h + 15 of a
// group of 32 (v_mfma_i32_32x32x32_i8: 16 bytes), or 8h .. 8h + 7 of a group
// of 16 (32x32x16: 8 bytes).  The activations (A operand) take the same
// elements from their row, so each MFMA gives the group's dot.
//
// A reader: U elements a unit, groups of G, NG = U / G groups a unit, MIN
// (a minimum term), Regs, load(R, src, row, u, h) (row: byte offset of the
// weight row, or NONE), codes(R, j, h) (group j of the unit),
// scales(R, sc, mn).  Layouts: kapel-core/src/dtype.rs:342-520; scales and
// minimums as the CPU's byte decoders (bytes.rs:258-353).

// Each byte b (< 128) of x minus o (< 128), as signed bytes.
__device__ __forceinline__ uint32_t sub_bytes(uint32_t x, uint32_t o) {
    return ((x | 0x80808080u) - o) ^ 0x80808080u;
}
__device__ __forceinline__ uint64_t pair(uint32_t lo, uint32_t hi) { return (uint64_t)hi << 32 | lo; }

// The bytes of a workgroup's stage in LDS, read as dwords (offsets a multiple
// of 4 for ld, of 2 for rn).
struct Lds {
    const uint8_t *p;
};

template <int N>
__device__ __forceinline__ void ld(uint32_t (&v)[N], const Lds &s, uint32_t off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(s.p + off);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = w[i];
}
template <int R>
__device__ __forceinline__ void rn(uint32_t (&w)[(R + 3) / 4], const Lds &s, uint32_t off) {
    static_assert(R % 2 == 0, "even runs only");
    constexpr int D = (R + 5) / 4, W = (R + 3) / 4;
    const uint32_t a = off & 2u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(s.p + (off - a));
    uint32_t v[D + 1];
#pragma unroll
    for (int i = 0; i < D; i++) v[i] = p[i];
    v[D] = 0u;
#pragma unroll
    for (int i = 0; i < W; i++) w[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], a);
}

// The same reads straight from the weight matrix (buffer loads; offsets
// past its end read zeros).
template <int N>
__device__ __forceinline__ void ld(uint32_t (&v)[N], const Src &s, uint32_t off) {
    lanes::ldb<N>(v, s, off);
}
template <int R>
__device__ __forceinline__ void rn(uint32_t (&w)[(R + 3) / 4], const Src &s, uint32_t off) {
    lanes::run<R>(w, s, off);
}

// ------------------------------------------------ 256-element super-blocks
// Q4_K: nibbles of sub-block 2c (low) and 2c + 1 (high) at 16 + 32c + l.
struct Q4K {
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 144, BLEN = 256;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t h[4], q[4][4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
        ld<4>(r.h, s, b);
#pragma unroll
        for (int c = 0; c < 4; c++) ld<4>(r.q[c], s, b + 16 + 32 * c + 16 * h);
    }
    __device__ static v4i codes(const Regs &r, int j, int) {
        return (j & 1) ? lanes::hi4(r.q[j >> 1]) : lanes::lo4(r.q[j >> 1]);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&mn)[NG]) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float s[2], m[2];
            lanes::k_pair(r.h, g, s, m);
            sc[2 * g] = s[0], sc[2 * g + 1] = s[1];
            mn[2 * g] = m[0], mn[2 * g + 1] = m[1];
        }
    }
};

// Q5_K: as Q4_K, fifth bit of element 32j + l in bit j of byte 16 + l,
// nibbles at 48.
struct Q5K {
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 176, BLEN = 256;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t h[4], qh[4], q[4][4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
        ld<4>(r.h, s, b);
        ld<4>(r.qh, s, b + 16 + 16 * h);
#pragma unroll
        for (int c = 0; c < 4; c++) ld<4>(r.q[c], s, b + 48 + 32 * c + 16 * h);
    }
    __device__ static v4i codes(const Regs &r, int j, int) {
        v4i c = (j & 1) ? lanes::hi4(r.q[j >> 1]) : lanes::lo4(r.q[j >> 1]);
#pragma unroll
        for (int i = 0; i < 4; i++) c[i] |= (int)(((r.qh[i] >> j) & 0x01010101u) << 4);
        return c;
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&mn)[NG]) {
        Q4K::scales(*reinterpret_cast<const Q4K::Regs *>(&r), sc, mn);
    }
};

// Element 128a + 32t + l of the 2-bit formats is group 8a + 2t + l / 16:
// group j has a = j / 8, t = j / 2 % 4 and l from 16 (j % 2); its half h is
// l = 16 (j % 2) + 8h .. + 7.

// Q6_K (210 bytes): low nibble t / 2 of byte 64a + 32 (t % 2) + l, high bits
// 2t of byte 128 + 32a + l, signed scales at 192, d at 208; codes - 32.
struct Q6K {
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 210, BLEN = 256;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t ql[8][2], qh[4][2], sc[5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
#pragma unroll
        for (int i = 0; i < 8; i++)  // (a, t % 2, j % 2)
            rn<8>(r.ql[i], s, b + 64 * (i >> 2) + 32 * ((i >> 1) & 1) + 16 * (i & 1) + 8 * h);
#pragma unroll
        for (int i = 0; i < 4; i++)  // (a, j % 2)
            rn<8>(r.qh[i], s, b + 128 + 32 * (i >> 1) + 16 * (i & 1) + 8 * h);
        rn<18>(r.sc, s, b + 192);
    }
    __device__ static uint64_t codes(const Regs &r, int j, int) {
        const int a = j >> 3, t = (j >> 1) & 3, lh = j & 1;
        const uint32_t *l = r.ql[4 * a + 2 * (t & 1) + lh], *q = r.qh[2 * a + lh];
        uint32_t c[2];
#pragma unroll
        for (int i = 0; i < 2; i++)
            c[i] = sub_bytes(((l[i] >> (4 * (t >> 1))) & LO4) | (((q[i] >> (2 * t)) & 0x03030303u) << 4),
                             0x20202020u);
        return pair(c[0], c[1]);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
        const float d = f16(r.sc[4] & 0xffffu);
#pragma unroll
        for (int j = 0; j < 16; j++) sc[j] = d * (float)(int8_t)lanes::byte_of(r.sc[j >> 2], j & 3);
    }
};

// Q2_K (84 bytes): scale bytes at 0 (low nibble scale, high minimum), codes
// bits 2t of byte 16 + 32a + l, d and dmin at 80.
struct Q2K {
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 84, BLEN = 256;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t q[4][2], sc[4], dd[1];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
#pragma unroll
        for (int i = 0; i < 4; i++) ld<2>(r.q[i], s, b + 16 + 32 * (i >> 1) + 16 * (i & 1) + 8 * h);
        ld<4>(r.sc, s, b);
        ld<1>(r.dd, s, b + 80);
    }
    __device__ static uint64_t codes(const Regs &r, int j, int) {
        const int a = j >> 3, t = (j >> 1) & 3, lh = j & 1;
        const uint32_t *q = r.q[2 * a + lh];
        return pair((q[0] >> (2 * t)) & 0x03030303u, (q[1] >> (2 * t)) & 0x03030303u);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&mn)[NG]) {
        const float d = f16(r.dd[0] & 0xffffu), dmin = f16(r.dd[0] >> 16);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            uint32_t k = lanes::byte_of(r.sc[j >> 2], j & 3);
            sc[j] = d * (float)(k & 15u);
            mn[j] = dmin * (float)(k >> 4);
        }
    }
};

// Q3_K (110 bytes): high bit 4a + t of byte l, low bits 2t of byte 32 + 32a
// + l, 12 bytes of 6-bit scales at 96, d at 108; codes - 4.
struct Q3K {
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 110, BLEN = 256;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t hm[2][2], q[4][2], sc[4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
#pragma unroll
        for (int i = 0; i < 2; i++) rn<8>(r.hm[i], s, b + 16 * i + 8 * h);
#pragma unroll
        for (int i = 0; i < 4; i++) rn<8>(r.q[i], s, b + 32 + 32 * (i >> 1) + 16 * (i & 1) + 8 * h);
        rn<14>(r.sc, s, b + 96);
    }
    __device__ static uint64_t codes(const Regs &r, int j, int) {
        const int a = j >> 3, t = (j >> 1) & 3, lh = j & 1;
        const uint32_t *q = r.q[2 * a + lh], *m = r.hm[lh];
        uint32_t c[2];
#pragma unroll
        for (int i = 0; i < 2; i++)
            c[i] = sub_bytes(((q[i] >> (2 * t)) & 0x03030303u) | (((m[i] >> (4 * a + t)) & 0x01010101u) << 2),
                             0x04040404u);
        return pair(c[0], c[1]);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
        const float d = f16(r.sc[3] & 0xffffu);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int a = i % 8, c = 8 + i % 4;
            uint32_t lo = (lanes::byte_of(r.sc[a >> 2], a & 3) >> (4 * (i / 8))) & 15u;
            uint32_t hi = (lanes::byte_of(r.sc[c >> 2], c & 3) >> (2 * (i / 4))) & 3u;
            sc[i] = d * (float)((int)(lo | (hi << 4)) - 32);
        }
    }
};

// ----------------------------------------------------- blocks of 32
// A unit is four blocks (or pieces of 32 of Kapel's groups): group j of unit
// u is block 4u + j.  Blocks past K are read from wherever their offset
// lands and their scales cleared by the kernel (their activations are zero).

// Q8_0: d, 32 signed bytes.
struct Q8_0 {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 34, BLEN = 32;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[4][4], d[4][1];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t b = row + (4 * u + j) * BYTES;
            rn<16>(r.c[j], s, b + 2 + 16 * h);
            rn<2>(r.d[j], s, b);
        }
    }
    __device__ static v4i codes(const Regs &r, int j, int) {
        return v4i{(int)r.c[j][0], (int)r.c[j][1], (int)r.c[j][2], (int)r.c[j][3]};
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = f16(r.d[j][0] & 0xffffu);
    }
};

__device__ __forceinline__ v4i nibbles(const uint32_t *q, int h, uint32_t offset) {
    v4i c;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t v = h ? (q[i] >> 4) & LO4 : q[i] & LO4;
        c[i] = (int)(offset ? sub_bytes(v, offset) : v);
    }
    return c;
}

// Q4_0: d, 16 bytes (byte i: element i low nibble, i + 16 high); codes - 8.
struct Q4_0 {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 18, BLEN = 32;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t w[4][5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int) {
#pragma unroll
        for (int j = 0; j < 4; j++) rn<18>(r.w[j], s, row + (4 * u + j) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int j, int h) {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[j][i + 1], r.w[j][i], 2);
        return nibbles(q, h, 0x08080808u);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = f16(r.w[j][0] & 0xffffu);
    }
};

// Q4_1: d, m, 16 bytes of nibbles; w = d q + m (minimum -m).
struct Q4_1 {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 20, BLEN = 32;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t w[4][5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int) {
#pragma unroll
        for (int j = 0; j < 4; j++) ld<5>(r.w[j], s, row + (4 * u + j) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int j, int h) { return nibbles(r.w[j] + 1, h, 0u); }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&mn)[NG]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sc[j] = f16(r.w[j][0] & 0xffffu);
            mn[j] = -f16(r.w[j][0] >> 16);
        }
    }
};

// Q5_0: d, 4 bytes of fifth bits (bit e: element e), nibbles; codes - 16.
// Q5_1: d, m, fifth bits, nibbles; w = d q + m.
template <bool ONE>
struct Q5x {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = ONE ? 24 : 22, BLEN = 32;
    static constexpr bool MIN = ONE;
    struct Regs {
        uint32_t w[4][6];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t b = row + (4 * u + j) * BYTES;
            if (ONE) ld<6>(r.w[j], s, b);
            else rn<22>(r.w[j], s, b);
        }
    }
    __device__ static v4i codes(const Regs &r, int j, int h) {
        const uint32_t *w = r.w[j];
        uint32_t high, q[4];
        if (ONE) {
            high = w[1];
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = w[2 + i];
        } else {
            high = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(w[2 + i], w[1 + i], 2);
        }
        v4i c;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t v = (h ? (q[i] >> 4) & LO4 : q[i] & LO4) | lanes::spread4(high, 16 * h + 4 * i);
            c[i] = (int)(ONE ? v : sub_bytes(v, 0x10101010u));
        }
        return c;
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&mn)[NG]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sc[j] = f16(r.w[j][0] & 0xffffu);
            if (ONE) mn[j] = -f16(r.w[j][0] >> 16);
        }
    }
};

// Kapel int8 / int4 in groups of GR (a multiple of 32): an f32 scale, then GR
// bytes, or GR / 2 bytes of nibbles (element 2i low, 2i + 1 high); int4
// codes - 8.  A unit is 128 elements, or one group of 256; group j of unit
// u is the piece of 32 elements p = NG u + j.
template <int GR>
struct Int8G {
    static constexpr int U = GR > 128 ? GR : 128, G = 32, NG = U / 32, BYTES = 4 + GR, BLEN = GR;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[NG][4], sc[NG][1];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
#pragma unroll
        for (int j = 0; j < NG; j++) {
            const int p = NG * u + j;
            const uint32_t b = row + (uint32_t)(32 * p / GR) * BYTES;
            ld<1>(r.sc[j], s, b);
            ld<4>(r.c[j], s, b + 4 + (32 * p) % GR + 16 * h);
        }
    }
    __device__ static v4i codes(const Regs &r, int j, int) {
        return v4i{(int)r.c[j][0], (int)r.c[j][1], (int)r.c[j][2], (int)r.c[j][3]};
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
#pragma unroll
        for (int j = 0; j < NG; j++) sc[j] = __uint_as_float(r.sc[j][0]);
    }
};

template <int GR>
struct Int4G {
    static constexpr int U = GR > 128 ? GR : 128, G = 32, NG = U / 32, BYTES = 4 + GR / 2, BLEN = GR;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[NG][2], sc[NG][1];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
#pragma unroll
        for (int j = 0; j < NG; j++) {
            const int p = NG * u + j;
            const uint32_t b = row + (uint32_t)(32 * p / GR) * BYTES;
            ld<1>(r.sc[j], s, b);
            ld<2>(r.c[j], s, b + 4 + ((32 * p) % GR) / 2 + 8 * h);
        }
    }
    __device__ static v4i codes(const Regs &r, int j, int) {
        v4i c;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t w = r.c[j][i], lo = w & LO4, hi = (w >> 4) & LO4;
            c[2 * i] = (int)sub_bytes(__builtin_amdgcn_perm(hi, lo, 0x05010400u), 0x08080808u);
            c[2 * i + 1] = (int)sub_bytes(__builtin_amdgcn_perm(hi, lo, 0x07030602u), 0x08080808u);
        }
        return c;
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
#pragma unroll
        for (int j = 0; j < NG; j++) sc[j] = __uint_as_float(r.sc[j][0]);
    }
};

// ------------------------------------------------- the non-linear formats
// Codes become their signed values (kh_iq.h); no minimum; f32 activations
// only (bytes.rs:51-77 has no byte reader for them).
__device__ __forceinline__ v4i iq4_nibbles(const uint32_t *q, int h) {
    v4i c;
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = (int)iq4_bytes(h ? (q[i] >> 4) & LO4 : q[i] & LO4);
    return c;
}

// IQ4_NL: d, 16 bytes of codes as Q4_0's.
struct IQ4NL {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 18, BLEN = 32;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t w[4][5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int) {
#pragma unroll
        for (int j = 0; j < 4; j++) rn<18>(r.w[j], s, row + (4 * u + j) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int j, int h) {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[j][i + 1], r.w[j][i], 2);
        return iq4_nibbles(q, h);
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = f16(r.w[j][0] & 0xffffu);
    }
};

// IQ4_XS: d, 16 high scale bits, 4 bytes of low scale nibbles, group j's 16
// code bytes at 8 + 16j (half h: nibble h of each); scale d (s - 32).
struct IQ4XS {
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 136, BLEN = 256;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t h[2], q[8][4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int) {
        const uint32_t b = row + u * BYTES;
        ld<2>(r.h, s, b);
#pragma unroll
        for (int j = 0; j < 8; j++) ld<4>(r.q[j], s, b + 8 + 16 * j);
    }
    __device__ static v4i codes(const Regs &r, int j, int h) { return iq4_nibbles(r.q[j], h); }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
        const float d = f16(r.h[0] & 0xffffu);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int s = (int)((lanes::byte_of(r.h[1], j >> 1) >> (4 * (j & 1))) & 15u) |
                          (int)(((r.h[0] >> (16 + 2 * j)) & 3u) << 4);
            sc[j] = d * (float)(s - 32);
        }
    }
};

// IQ3_S: d; group j's 8 index bytes at 2 + 8j (half h: bytes 4h .. 4h + 3,
// ninth bits 4h .. 4h + 3 of byte 66 + j); its 4 sign bytes at 74 + 4j (half
// h: bytes 2h, 2h + 1); scale nibble j of 106: d (1 + 2s).
struct IQ3S {
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 110, BLEN = 256;
    static constexpr bool MIN = false, GRID = true;
    struct Regs {
        uint32_t c[8], hi[2], sg[8], sc, d;
    };
    template <class S>
    __device__ static void load(Regs &r, const S &s, uint32_t row, int u, int h) {
        const uint32_t b = row + u * BYTES;
        uint32_t t[1];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            rn<4>(t, s, b + 2 + 8 * j + 4 * h);
            r.c[j] = t[0];
        }
        rn<8>(r.hi, s, b + 66);
        rn<32>(r.sg, s, b + 74);
        rn<4>(t, s, b + 106);
        r.sc = t[0];
        rn<2>(t, s, b);
        r.d = t[0] & 0xffffu;
    }
    __device__ static v4i codes(const Regs &r, int j, int h) {
        const uint32_t hb = lanes::byte_of(r.hi[j >> 2], j & 3) >> (4 * h), sg = r.sg[j] >> (16 * h);
        v4i c;
#pragma unroll
        for (int i = 0; i < 4; i++)
            c[i] = (int)iq3s_bytes(lanes::byte_of(r.c[j], i) | (((hb >> i) & 1u) << 8), (sg >> (4 * i)) & 15u);
        return c;
    }
    __device__ static void scales(const Regs &r, float (&sc)[NG], float (&)[NG]) {
        const float d = f16(r.d);
#pragma unroll
        for (int j = 0; j < 8; j++) sc[j] = d * (float)(1u + 2u * ((lanes::byte_of(r.sc, j >> 1) >> (4 * (j & 1))) & 15u));
    }
};

// ---------------------------------------------------------- the kernel
constexpr int LDS_MAX = 160 * 1024;      // LDS of a CU (gfx950)


// The LDS stage of one unit, filled by direct loads to LDS (each wave
// instruction writes 64 lanes x 16 bytes, or x 4 bytes, consecutive): the
// activation rows [P][RM] of the unit's U bytes (16-byte chunks in a
// swizzled order: chunk o of row r at o ^ swz(r), so that an LDS read of one
// chunk by 16 rows touches every bank once), the weight rows [NCOLS] of CWP
// chunks (the unit's UB bytes from the dword at or below their start), the
// activation scales [RM][U / 32] and sums [RM][U / G].  Every region is a
// whole number of instructions for each wave.  A workgroup is WMG x 4 waves:
// WMG groups of WM row tiles of 32, by 4 x WN weight tiles of 32.
template <class F, int P, int WM, int WMG, int WN>
struct Plan {
    static constexpr int WAVES = 4 * WMG;
    static constexpr int U = F::U, G = F::G, RM = 32 * WM * WMG, NS = U / 32, NX = U / G;
    static constexpr int UB = U / F::BLEN * F::BYTES;
    static constexpr bool ODD = F::BYTES % 4 != 0;  // blocks at even offsets
    static constexpr int CW = (UB + (ODD ? 2 : 0) + 15) / 16;
    // Chunks a weight row takes in LDS: an odd number (the last one, past
    // CW, loads nothing), so that the rows read by the 32 lanes of a tile
    // start 4 banks apart modulo 64 and not on the same few banks (Q6_K's 14
    // chunks put every fourth row on one bank: 3 % shorter layer at M = 64).
    static constexpr int CWP = CW | 1;
    static constexpr int AW = U / 16;
    static constexpr int NCOLS = 4 * WN * 32;
    static constexpr int up(int x) { return (x + WAVES - 1) / WAVES * WAVES; }
    static constexpr int IA = up((P * RM * AW + 63) / 64);
    static constexpr int IW = up((NCOLS * CWP + 63) / 64);
    static constexpr int IS = up((RM * NS + 63) / 64);
    static constexpr int IX = F::MIN ? up((RM * NX + 63) / 64) : 0;
    static constexpr int OA = 0, OW = IA * 1024, OS = OW + IW * 1024, OX = OS + IS * 256;
    static constexpr int SB = OX + IX * 256;
    static constexpr int D = (IA + IW + IS + IX) / WAVES;  // instructions a wave issues a stage
    static constexpr int STAGES = 3 * SB + grid_lds<F>() <= LDS_MAX ? 3 : 2;
    static constexpr bool FITS = 2 * SB + grid_lds<F>() <= LDS_MAX;
    static_assert(D * (STAGES - 2) <= 63, "the later stages' loads fit vmcnt");
    // The position of chunk o of activation row r.
    static constexpr int swz(int r) { return U == 128 ? (r >> 1) & 7 : r & 15; }
};

// Weight tiles of a wave: two with byte activations, or one for three planes
// (their three dot sums a tile do not leave room for a second tile without
// spills), for the formats with a minimum term or more than 24 dwords of a
// unit's lane bytes (their registers would not fit two waves a SIMD) and
// where two stages of two would not fit in LDS.
template <class F, int P, int WM, int WMG>
constexpr int wn_of() {
    return P == 1 && !F::MIN && sizeof(typename F::Regs) <= 96 && Plan<F, P, WM, WMG, 2>::FITS ? 2 : 1;
}

// An empty asm through which a value must pass (its order among the others
// is kept).
#ifndef KH_PIN
#define KH_PIN(x) asm volatile("" : "+v"(x))
#endif
// A direct load to LDS: `size` bytes of each lane at buffer offset voff, to
// lds + size * lane.
#ifndef KH_LDS_LOAD
#define KH_LDS_LOAD(rsrc, lds, size, voff) \
    __builtin_amdgcn_raw_ptr_buffer_load_lds((rsrc), (__attribute__((address_space(3))) void *)(lds), (size), (int)(voff), 0, 0, 0)
#endif

__device__ __forceinline__ v16i mfma_dot(v4i a, v4i b) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
}
__device__ __forceinline__ v16i mfma_dot(uint64_t a, uint64_t b) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8((long)a, (long)b, v16i{}, 0, 0, 0);
}

// s_waitcnt with vmcnt <= n (and no outstanding LDS work).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
}

template <class F, int P, int WM, int WMG>
__global__ __launch_bounds__(256 * WMG) void mm_kernel(MmArgs a) {
    constexpr int WN = wn_of<F, P, WM, WMG>();
    using L = Plan<F, P, WM, WMG, WN>;
    constexpr int WAVES = L::WAVES;
    constexpr int U = F::U, G = F::G, NG = F::NG, RM = L::RM, NS = L::NS, NX = L::NX;
    constexpr int S = L::STAGES, AW = L::AW, CW = L::CW, CWP = L::CWP;
    using CodeT = decltype(F::codes(*(const typename F::Regs *)nullptr, 0, 0));
    extern __shared__ __align__(16) uint8_t lds[];

    // Workgroup -> (row tile, column group, K split): the row tiles of a
    // column group run together on one XCD, sharing its weights in L2.
    const int b = blockIdx.x, local = b / XCDS;
    const int mt = local % a.mtiles;
    const int rest = (local / a.mtiles) * XCDS + b % XCDS;
    if (rest >= a.ngroups * a.ks) return;
    grid_fill<F>();
    const int kz = rest / a.ngroups, ng = rest % a.ngroups;
    const int u0 = kz * a.ups, u1 = min(a.units, u0 + a.ups);
    const int m0 = mt * RM;

    const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = (wave >> 2) * WM * 32;  // this wave's first activation row in the stage
    const int wc = (wave & 3) * WN * 32;   // and first weight row
    int mat = 0;
    for (int i = 1; i < a.count; i++)
        if (ng >= a.ng0[i]) mat = i;
    const int64_t g0 = (int64_t)(ng - a.ng0[mat]) * L::NCOLS;  // first weight row of the group
    const int64_t nmat = (int64_t)a.n[mat];
    const uint32_t row_bytes = (uint32_t)a.row_bytes;

    // What each lane loads into a stage, by instruction: the offset of its
    // piece for unit 0 (or NONE) and what moves with the unit.
    const Src wsrc = lanes::source(a.w[mat], a.wbytes[mat]);
    const Src psrc = lanes::source(a.planes, a.planes_bytes);
    const Src ssrc = lanes::source(a.xscale, (uint32_t)(a.rows * (a.k / 32) * 4));
    const Src xsrc = lanes::source(a.xsum, (uint32_t)(a.rows * (a.k / G) * 4));
    constexpr int DA = L::IA / WAVES, DW = L::IW / WAVES, DS = L::IS / WAVES, DX = L::IX / WAVES;
    uint32_t a_base[DA], a_col[DA], w_row[DW], w_piece[DW], s_base[DS], s_j[DS];
    uint32_t x_base[DX > 0 ? DX : 1], x_j[DX > 0 ? DX : 1];
#pragma unroll
    for (int i = 0; i < DA; i++) {
        const int ci = (i * WAVES + wave) * 64 + lane, pr = ci / AW, o = (ci % AW) ^ L::swz(pr % RM);
        const int p = pr / RM, r = pr % RM;
        const bool on = ci < P * RM * AW && m0 + r < a.rows;
        a_base[i] = on ? (uint32_t)(((uint64_t)(m0 + r) * P + p) * a.kpad + 16 * o) : NONE;
        a_col[i] = 16 * o;
    }
#pragma unroll
    for (int i = 0; i < DW; i++) {
        const int ci = (i * WAVES + wave) * 64 + lane, col = ci / CWP;
        const int64_t n = g0 + col;
        w_row[i] = ci < L::NCOLS * CWP && ci % CWP < CW && n < nmat ? (uint32_t)n * row_bytes : NONE;
        w_piece[i] = 16 * (ci % CWP);
    }
#pragma unroll
    for (int i = 0; i < DS; i++) {
        const int di = (i * WAVES + wave) * 64 + lane, r = di / NS;
        const bool on = di < RM * NS && m0 + r < a.rows;
        s_base[i] = on ? (uint32_t)(((uint64_t)(m0 + r) * (a.k / 32) + di % NS) * 4) : NONE;
        s_j[i] = di % NS;
    }
#pragma unroll
    for (int i = 0; i < DX; i++) {
        const int di = (i * WAVES + wave) * 64 + lane, r = di / NX;
        const bool on = di < RM * NX && m0 + r < a.rows;
        x_base[i] = on ? (uint32_t)(((uint64_t)(m0 + r) * (a.k / G) + di % NX) * 4) : NONE;
        x_j[i] = di % NX;
    }
    // The loads of unit u into stage buffer `slot` (units past the range
    // load nothing: NONE, zeros written, no memory read), D instructions.
    auto issue = [&](int u, int slot) __attribute__((always_inline)) {
        uint8_t *st = lds + slot * L::SB;
        const bool on = u < u1;
#pragma unroll
        for (int i = 0; i < DA; i++) {
            const bool in = on && a_base[i] != NONE && u * U + (int)a_col[i] < a.k;
            KH_LDS_LOAD(psrc.r, st + L::OA + (i * WAVES + wave) * 1024, 16, in ? a_base[i] + u * U : NONE);
        }
#pragma unroll
        for (int i = 0; i < DW; i++) {
            const uint32_t at = w_row[i] + (uint32_t)u * L::UB;
            KH_LDS_LOAD(wsrc.r, st + L::OW + (i * WAVES + wave) * 1024, 16,
                        on && w_row[i] != NONE ? (at & ~3u) + w_piece[i] : NONE);
        }
#pragma unroll
        for (int i = 0; i < DS; i++) {
            const bool in = on && s_base[i] != NONE && u * NS + (int)s_j[i] < a.k / 32;
            KH_LDS_LOAD(ssrc.r, st + L::OS + (i * WAVES + wave) * 256, 4, in ? s_base[i] + u * NS * 4 : NONE);
        }
#pragma unroll
        for (int i = 0; i < DX; i++) {
            const bool in = on && x_base[i] != NONE && u * NX + (int)x_j[i] < a.k / G;
            KH_LDS_LOAD(xsrc.r, st + L::OX + (i * WAVES + wave) * 256, 4, in ? x_base[i] + u * NX * 4 : NONE);
        }
    };

    v16f acc[WM][WN], low[F::MIN ? WM : 1][F::MIN ? WN : 1];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int t = 0; t < WN; t++) acc[i][t] = v16f{};

    using Regs = typename F::Regs;
    // Unit u from stage `slot`; `then` (the next unit's loads) runs once this
    // unit's first LDS reads are issued.
    auto compute = [&](int u, int slot, auto then) __attribute__((always_inline)) {
        const uint8_t *st = lds + slot * L::SB;
        const float *sx = reinterpret_cast<const float *>(st + L::OS);
        const float *xs = reinterpret_cast<const float *>(st + L::OX);
        Regs R[WN];
        float sc[WN][NG], mn[WN][NG];
#pragma unroll
        for (int t = 0; t < WN; t++) {
            const int col = wc + t * 32 + c;
            const uint32_t shift = L::ODD ? (((uint32_t)(g0 + col) * row_bytes + (uint32_t)u * L::UB) & 3u) : 0u;
            F::load(R[t], Lds{st + L::OW}, (uint32_t)(col * CWP * 16) + shift, 0, h);
        }
        // The steps (group j, weight tile t, row tile i) in order, as a
        // pipeline: the MFMAs of a step are issued before the VALU work of
        // the one before.  Operands and sums pass through KH_PIN (an empty
        // asm), which keeps the compiler from hoisting the MFMAs of every
        // step ahead of all VALU work, whose results would not fit in the
        // registers.
        constexpr int NQ = NG * WN * WM;
        CodeT av[WM][P], an[WM][P], bw;
        float xa[WM], xn[WM], sw;
        v16i dp[P];
        v16f sp;
        // The unit's activation scales of each row, read whole (16-byte
        // reads: a read of one scale by the 32 rows of a tile would hit the
        // same banks four or eight times).
        float xrow[WM][NS];
#pragma unroll
        for (int i = 0; i < WM; i++) {
            const float4 *q = reinterpret_cast<const float4 *>(sx + (wr + i * 32 + c) * NS);
#pragma unroll
            for (int v = 0; v < NS / 4; v++) {
                const float4 t4 = q[v];
                xrow[i][4 * v] = t4.x, xrow[i][4 * v + 1] = t4.y, xrow[i][4 * v + 2] = t4.z, xrow[i][4 * v + 3] = t4.w;
            }
        }
        // The A operands and activation scales of group j, read a group
        // ahead of their use.
        auto a_operands = [&](int j) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
                const int r = wr + i * 32 + c;
                // Group j, half h: chunk 2j + h (groups of 32) or bytes 8h of
                // chunk j (groups of 16).
                const int o = G == 32 ? 2 * j + h : j, within = G == 32 ? 0 : 8 * h;
#pragma unroll
                for (int p = 0; p < P; p++)
                    an[i][p] = *reinterpret_cast<const CodeT *>(
                        st + L::OA + (p * RM + r) * AW * 16 + (o ^ L::swz(r)) * 16 + within);
                xn[i] = h ? 0.0f : xrow[i][j * G / 32];
            }
        };
        a_operands(0);
        then();
#pragma unroll
        for (int t = 0; t < WN; t++) {
            F::scales(R[t], sc[t], mn[t]);
            if (U == 128)
#pragma unroll
                for (int j = 0; j < NG; j++)
                    if (u * U + j * G >= a.k) sc[t][j] = 0.0f, mn[t][j] = 0.0f;
        }
        auto finish = [&](int i, int t) __attribute__((always_inline)) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                float dot;
                if (P == 3) dot = fmaf((float)dp[0][v], a.hi, (float)((dp[1][v] << a.shift) + dp[2][v]));
                else dot = (float)dp[0][v];
                acc[i][t][v] = fmaf(dot, sp[v], acc[i][t][v]);
            }
            KH_PIN(acc[i][t]);
        };
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int j = q / (WN * WM), t = (q / WM) % WN, i = q % WM;
            if (t == 0 && i == 0) {
#pragma unroll
                for (int ii = 0; ii < WM; ii++) {
#pragma unroll
                    for (int p = 0; p < P; p++) av[ii][p] = an[ii][p];
                    xa[ii] = xn[ii];
                }
                if (j + 1 < NG) a_operands(j + 1);
            }
            if (i == 0) {
                bw = F::codes(R[t], j, h);
                sw = h ? 0.0f : sc[t][j];
            }
            v16i dq[P];
#pragma unroll
            for (int p = 0; p < P; p++) {
                KH_PIN(av[i][p]);
                KH_PIN(bw);
                dq[p] = mfma_dot(av[i][p], bw);
            }
            KH_PIN(xa[i]);
            KH_PIN(sw);
            const v16f sq = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[i], sw, v16f{}, 0, 0, 0);
            if (q > 0) finish((q - 1) % WM, ((q - 1) / WM) % WN);
#pragma unroll
            for (int p = 0; p < P; p++) dp[p] = dq[p];
            sp = sq;
            if constexpr (F::MIN) {
                if ((j & 1) && t == WN - 1 && i == WM - 1) {
                    // Groups j - 1 (k-slot 0) and j (k-slot 1).
#pragma unroll
                    for (int ii = 0; ii < WM; ii++) {
                        float xm = xs[(wr + ii * 32 + c) * NX + j - 1 + h];
                        KH_PIN(xm);
#pragma unroll
                        for (int tt = 0; tt < WN; tt++) {
                            float m = -(h ? mn[tt][j] : mn[tt][j - 1]);
                            KH_PIN(m);
                            low[ii][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(xm, m, j == 1 ? v16f{} : low[ii][tt],
                                                                               0, 0, 0);
                        }
                    }
                }
            }
        }
        finish(WM - 1, WN - 1);
        if constexpr (F::MIN) {
            // The unit's minimum term joins the sums unit by unit: two
            // separate sums over all of K would cancel in the end.
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int t = 0; t < WN; t++) {
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[i][t][v] = acc[i][t][v] + low[i][t][v];
                    KH_PIN(acc[i][t]);
                }
        }
    };

    // The K loop over a ring of S stages: unit u waits for its own loads
    // (the D (S - 2) loads of the later units may still run), meets the
    // other waves at a barrier (their loads of u are in; their reads of u - 1
    // are done), loads unit u + S - 1 into the stage u - 1 used, multiplies.
    // A bare s_barrier: a fenced one would wait for every load in flight.
#pragma unroll
    for (int s = 0; s + 1 < S; s++) issue(u0 + s, s);
    for (int u = u0; u < u1; u += S) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            if (u + s < u1) {
                wait_vm<L::D * (S - 2)>();
                __builtin_amdgcn_s_barrier();
                compute(u + s, s, [&]() __attribute__((always_inline)) { issue(u + s + S - 1, (s + S - 1) % S); });
            }
        }
    }
    // No load may still write LDS when the workgroup ends.
    wait_vm<0>();

    // Lane (c, h), register v of a tile holds row 8 (v / 4) + 4h + v % 4,
    // column c.  The workgroup's sums go through LDS ([RM][NCOLS + 8]
    // floats: the two halves of a wave 32 banks apart), then out as 16-byte
    // stores of 4 consecutive columns: whole rows of 512 or 1024 bytes
    // instead of two 128-byte pieces an instruction (config 4's layer 2-3 %
    // shorter).
    constexpr int TS = L::NCOLS + 8;
    if constexpr (RM * TS * 4 <= S * L::SB) {
        float *tile = reinterpret_cast<float *>(lds);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int t = 0; t < WN; t++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    tile[(wr + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3)) * TS + wc + t * 32 + c] = acc[i][t][v];
        __syncthreads();
        const bool partial = a.ks > 1;
        float *dst = partial ? a.partials + (uint64_t)kz * a.rows * a.width : static_cast<float *>(a.out);
        const uint64_t stride = partial ? a.width : a.out_stride;
        const bool f32 = partial || a.out_kind == KH_F32;
        const bool vec = f32 && (((uintptr_t)dst & 15u) == 0) && stride % 4 == 0 && a.col0[mat] % 4 == 0;
        for (int idx = threadIdx.x; idx < RM * (L::NCOLS / 4); idx += 64 * WAVES) {
            const int r = idx / (L::NCOLS / 4), c4 = 4 * (idx % (L::NCOLS / 4));
            const int m = m0 + r;
            const int64_t n = g0 + c4;
            if (m >= a.rows || n >= nmat) continue;
            const float4 y = *reinterpret_cast<const float4 *>(tile + r * TS + c4);
            const uint64_t at = (uint64_t)m * stride + a.col0[mat] + (uint64_t)n;
            if (vec && n + 4 <= nmat) {
                *reinterpret_cast<float4 *>(dst + at) = y;
            } else {
                const float ys[4] = {y.x, y.y, y.z, y.w};
                for (int e = 0; e < 4 && n + e < nmat; e++) {
                    if (f32) dst[at + e] = ys[e];
                    else store_out(a.out_kind, a.out, at + e, ys[e]);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int t = 0; t < WN; t++) {
            const int64_t n = g0 + wc + t * 32 + c;
            if (n >= nmat) continue;
            const uint64_t col = a.col0[mat] + (uint64_t)n;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + wr + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m >= a.rows) continue;
                const float y = acc[i][t][v];
                if (a.ks == 1) store_out(a.out_kind, a.out, (uint64_t)m * a.out_stride + col, y);
                else a.partials[((uint64_t)kz * a.rows + m) * a.width + col] = y;
            }
        }
}

// The kernels of a format: bytes take two groups of waves of 64 rows each
// above 64 rows, two of 32 rows above 32 rows, one of 32 rows below; three
// planes take one group of 32 rows (LDS).
template <class F, int P, int WM, int WMG>
hipError_t launch_w(const MmArgs &a, hipStream_t s) {
    using L = Plan<F, P, WM, WMG, wn_of<F, P, WM, WMG>()>;
    static_assert(L::FITS, "two stages fit in LDS");
    constexpr size_t bytes = (size_t)L::STAGES * L::SB;
    static OncePerDevice once;
    hipError_t e = set_lds_limit(once, reinterpret_cast<const void *>(&mm_kernel<F, P, WM, WMG>), (int)bytes);
    if (e != hipSuccess) return e;
    const int groups = a.ngroups * a.ks;
    dim3 grid((unsigned)((groups + XCDS - 1) / XCDS * XCDS * a.mtiles)), block(64 * L::WAVES);
    hipLaunchKernelGGL((mm_kernel<F, P, WM, WMG>), grid, block, bytes, s, a);
    return hipGetLastError();
}

// The shapes of the kernel a launch of `rows` rows takes: (wm, wmg).
inline void shape_of(int planes, int rows, int &wm, int &wmg) {
    if (planes == 1) {
        wm = rows > 64 ? 2 : 1;
        wmg = rows > 32 ? 2 : 1;
    } else {
        wm = 1;
        wmg = 1;
    }
}

template <class F, int P>
hipError_t launch_fp(const MmArgs &a, hipStream_t s) {
    if constexpr (P == 1) {
        if (a.wm == 2 && a.wmg == 2) return launch_w<F, 1, 2, 2>(a, s);
        if (a.wm == 1 && a.wmg == 2) return launch_w<F, 1, 1, 2>(a, s);
        if (a.wm == 1 && a.wmg == 1) return launch_w<F, 1, 1, 1>(a, s);
    } else {
        if (a.wm == 1 && a.wmg == 1) return launch_w<F, 3, 1, 1>(a, s);
    }
    return hipErrorInvalidValue;
}

// Weight rows of a column group (a workgroup's).
template <class F>
int cols_f(int planes, int wm, int wmg) {
    if (planes == 3) return Plan<F, 3, 1, 1, wn_of<F, 3, 1, 1>()>::NCOLS;
    if (wm == 2) return Plan<F, 1, 2, 2, wn_of<F, 1, 2, 2>()>::NCOLS;
    if (wmg == 2) return Plan<F, 1, 1, 2, wn_of<F, 1, 1, 2>()>::NCOLS;
    return Plan<F, 1, 1, 1, wn_of<F, 1, 1, 1>()>::NCOLS;
}

// cols >= 0: the weight rows of a column group instead of a launch.
template <class F>
hipError_t launch_f(const MmArgs &a, int planes, hipStream_t s, int *cols) {
    if (cols) {
        *cols = cols_f<F>(planes, a.wm, a.wmg);
        return hipSuccess;
    }
    if (planes == 1) return launch_fp<F, 1>(a, s);
    if (planes == 3) return launch_fp<F, 3>(a, s);
    return hipErrorInvalidValue;
}

// The formats read with f32 activations only.
template <class F>
hipError_t launch_f3(const MmArgs &a, int planes, hipStream_t s, int *cols) {
    if (planes != 3) return hipErrorInvalidValue;
    if (cols) {
        *cols = cols_f<F>(planes, a.wm, a.wmg);
        return hipSuccess;
    }
    return launch_fp<F, 3>(a, s);
}

}  // namespace mm
}  // namespace kh
