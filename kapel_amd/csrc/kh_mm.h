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
// Weights are read straight from HBM by each wave through buffer loads (the
// lane readers below), one unit ahead; activations are staged per unit in
// LDS (double-buffered, one barrier per unit) and shared by the four waves.
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
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 144;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t h[4], q[4][4];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 256, G = 32, NG = 8, BYTES = 176;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t h[4], qh[4], q[4][4];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 210;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t ql[8][2], qh[4][2], sc[5];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 84;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t q[4][2], sc[4], dd[1];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 256, G = 16, NG = 16, BYTES = 110;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t hm[2][2], q[4][2], sc[4];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 34;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[4][4], d[4][1];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
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
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 18;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t w[4][5];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int) {
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
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 20;
    static constexpr bool MIN = true;
    struct Regs {
        uint32_t w[4][5];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int) {
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
    static constexpr int U = 128, G = 32, NG = 4, BYTES = ONE ? 24 : 22;
    static constexpr bool MIN = ONE;
    struct Regs {
        uint32_t w[4][6];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int) {
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
// codes - 8.  Group j of unit u is the piece of 32 elements p = 4u + j.
template <int GR>
struct Int8G {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 4 + GR;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[4][4], sc[4][1];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = 4 * u + j;
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
        for (int j = 0; j < 4; j++) sc[j] = __uint_as_float(r.sc[j][0]);
    }
};

template <int GR>
struct Int4G {
    static constexpr int U = 128, G = 32, NG = 4, BYTES = 4 + GR / 2;
    static constexpr bool MIN = false;
    struct Regs {
        uint32_t c[4][2], sc[4][1];
    };
    __device__ static void load(Regs &r, const Src &s, uint32_t row, int u, int h) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = 4 * u + j;
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
        for (int j = 0; j < 4; j++) sc[j] = __uint_as_float(r.sc[j][0]);
    }
};

// ---------------------------------------------------------- the kernel
constexpr int WAVES = 4;         // waves of a workgroup
constexpr int WN = 2;            // weight tiles of 32 rows a wave
constexpr int NCOLS = WAVES * WN * 32;  // weight rows of a workgroup

// Bytes of one row of a staged plane: the unit plus a pad that spreads the
// rows of an LDS read over all banks.
template <class F>
constexpr int row_stride() { return F::U + (F::G == 32 ? 16 : 8); }

// LDS bytes of one stage buffer: planes [P][RM][stride], scales [U/32][RM],
// sums [U/G][RM] (MIN).
template <class F, int P, int RM>
constexpr int stage_bytes() {
    return P * RM * row_stride<F>() + (F::U / 32) * RM * 4 + (F::MIN ? (F::U / F::G) * RM * 4 : 0);
}

// An empty asm through which a value must pass (its order among the others
// is kept).
#ifndef KH_PIN
#define KH_PIN(x) asm volatile("" : "+v"(x))
#endif

__device__ __forceinline__ v16i mfma_dot(v4i a, v4i b) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
}
__device__ __forceinline__ v16i mfma_dot(uint64_t a, uint64_t b) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8((long)a, (long)b, v16i{}, 0, 0, 0);
}

template <class F, int P, int WM>
__global__ __launch_bounds__(64 * WAVES) void mm_kernel(MmArgs a) {
    constexpr int U = F::U, G = F::G, NG = F::NG, RM = WM * 32;
    constexpr int RS = row_stride<F>(), NS = U / 32, NX = U / G;
    constexpr int T = 64 * WAVES;
    constexpr int CC = P * RM * U / 16;            // 16-byte pieces of a stage
    constexpr int CPT = (CC + T - 1) / T;
    constexpr int SPT = (RM * NS + T - 1) / T;
    constexpr int XPT = F::MIN ? (RM * NX + T - 1) / T : 0;
    constexpr int SB = stage_bytes<F, P, RM>();
    using CodeT = decltype(F::codes(*(const typename F::Regs *)nullptr, 0, 0));
    extern __shared__ __align__(16) uint8_t lds[];

    // Workgroup -> (row tile, column group, K split): the row tiles of a
    // column group run together on one XCD, sharing its weights in L2.
    const int b = blockIdx.x, local = b / XCDS;
    const int mt = local % a.mtiles;
    const int rest = (local / a.mtiles) * XCDS + b % XCDS;
    if (rest >= a.ngroups * a.ks) return;
    const int kz = rest / a.ngroups, ng = rest % a.ngroups;
    const int u0 = kz * a.ups, u1 = min(a.units, u0 + a.ups);
    const int m0 = mt * RM;

    const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int mat = 0;
    for (int i = 1; i < a.count; i++)
        if (ng >= a.ng0[i]) mat = i;
    const int64_t n0 = (int64_t)(ng - a.ng0[mat]) * NCOLS + wave * WN * 32;
    const Src src = lanes::source(a.w[mat], a.wbytes[mat]);
    uint32_t ro[WN];
#pragma unroll
    for (int t = 0; t < WN; t++) {
        const int64_t n = n0 + t * 32 + c;
        ro[t] = n < (int64_t)a.n[mat] ? (uint32_t)n * (uint32_t)a.row_bytes : NONE;
    }

    // Staging of the activations of a unit: every thread loads its pieces
    // (zeros past the rows or K), then stores them to a stage buffer.
    const Src psrc = lanes::source(a.planes, a.planes_bytes);
    const Src ssrc = lanes::source(a.xscale, (uint32_t)(a.rows * (a.k / 32) * 4));
    const Src xsrc = lanes::source(a.xsum, (uint32_t)(a.rows * (a.k / G) * 4));
    struct Stage {
        lanes::u32x4 c[CPT];
        uint32_t s[SPT];
        uint32_t x[XPT > 0 ? XPT : 1];
    };
    auto stage_load = [&](Stage &st, int u) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int ci = threadIdx.x + i * T;
            const int o = ci % (U / 16), rp = ci / (U / 16), r = rp % RM, p = rp / RM;
            const bool on = ci < CC && m0 + r < a.rows && u * U + 16 * o < a.k;
            const uint32_t off = on ? (uint32_t)(((m0 + r) * P + p) * a.kpad + u * U + 16 * o) : NONE;
            st.c[i] = __builtin_amdgcn_raw_buffer_load_b128(psrc.r, (int)off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int ci = threadIdx.x + i * T, j = ci % NS, r = ci / NS;
            const bool on = ci < RM * NS && m0 + r < a.rows && u * NS + j < a.k / 32;
            const uint32_t off = on ? (uint32_t)(((m0 + r) * (a.k / 32) + u * NS + j) * 4) : NONE;
            st.s[i] = __builtin_amdgcn_raw_buffer_load_b32(ssrc.r, (int)off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int ci = threadIdx.x + i * T, j = ci % NX, r = ci / NX;
            const bool on = ci < RM * NX && m0 + r < a.rows && u * NX + j < a.k / G;
            const uint32_t off = on ? (uint32_t)(((m0 + r) * (a.k / G) + u * NX + j) * 4) : NONE;
            st.x[i] = __builtin_amdgcn_raw_buffer_load_b32(xsrc.r, (int)off, 0, 0);
        }
    };
    auto stage_store = [&](const Stage &st, int buf) __attribute__((always_inline)) {
        uint8_t *base = lds + buf * SB;
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int ci = threadIdx.x + i * T;
            const int o = ci % (U / 16), rp = ci / (U / 16);
            if (ci >= CC) continue;
            uint8_t *to = base + rp * RS + 16 * o;
            if (RS % 16 == 0) {
                *reinterpret_cast<lanes::u32x4 *>(to) = st.c[i];
            } else {  // rows 8-byte aligned
                reinterpret_cast<lanes::u32x2 *>(to)[0] = lanes::u32x2{st.c[i].x, st.c[i].y};
                reinterpret_cast<lanes::u32x2 *>(to)[1] = lanes::u32x2{st.c[i].z, st.c[i].w};
            }
        }
        float *sx = reinterpret_cast<float *>(base + P * RM * RS);
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const int ci = threadIdx.x + i * T, j = ci % NS, r = ci / NS;
            if (ci < RM * NS) sx[j * RM + r] = __uint_as_float(st.s[i]);
        }
        float *xs = sx + NS * RM;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int ci = threadIdx.x + i * T, j = ci % NX, r = ci / NX;
            if (ci < RM * NX) xs[j * RM + r] = __uint_as_float(st.x[i]);
        }
    };

    v16f acc[WM][WN], low[F::MIN ? WM : 1][F::MIN ? WN : 1];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int t = 0; t < WN; t++) acc[i][t] = v16f{};

    using Regs = typename F::Regs;
    auto compute = [&](const Regs (&R)[WN], int u, int buf) __attribute__((always_inline)) {
        const uint8_t *base = lds + buf * SB;
        const float *sx = reinterpret_cast<const float *>(base + P * RM * RS);
        const float *xs = sx + NS * RM;
        float sc[WN][NG], mn[WN][NG];
#pragma unroll
        for (int t = 0; t < WN; t++) {
            F::scales(R[t], sc[t], mn[t]);
            if (U == 128)
#pragma unroll
                for (int j = 0; j < NG; j++)
                    if (u * U + j * G >= a.k) sc[t][j] = 0.0f, mn[t][j] = 0.0f;
        }
        // The steps (group j, weight tile t, row tile i) in order, as a
        // pipeline: the MFMAs of a step are issued before the VALU work of
        // the one before.  Operands and sums pass through KH_PIN (an empty
        // asm), which keeps the compiler from hoisting the MFMAs of every
        // step ahead of all VALU work, whose results would not fit in the
        // registers.
        constexpr int NQ = NG * WN * WM;
        CodeT av[WM][P], bw;
        float xa[WM], sw;
        v16i dp[P];
        v16f sp;
        auto a_operands = [&](int j) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
#pragma unroll
                for (int p = 0; p < P; p++)
                    av[i][p] = *reinterpret_cast<const CodeT *>(base + (p * RM + i * 32 + c) * RS + j * G +
                                                                (G / 2) * h);
                xa[i] = h ? 0.0f : sx[(j * G / 32) * RM + i * 32 + c];
            }
        };
        // The unit's sums start from its first group's products; they join
        // the running sums at the end of the unit (a sum in two levels).
        v16f part[WM][WN];
        auto finish = [&](int i, int t, bool first) __attribute__((always_inline)) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                float dot;
                if (P == 3) dot = fmaf((float)dp[0][v], a.hi, (float)((dp[1][v] << a.shift) + dp[2][v]));
                else dot = (float)dp[0][v];
                part[i][t][v] = first ? dot * sp[v] : fmaf(dot, sp[v], part[i][t][v]);
            }
            KH_PIN(part[i][t]);
        };
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int j = q / (WN * WM), t = (q / WM) % WN, i = q % WM;
            if (t == 0 && i == 0) a_operands(j);
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
            if (q > 0) finish((q - 1) % WM, ((q - 1) / WM) % WN, q - 1 < WN * WM);
#pragma unroll
            for (int p = 0; p < P; p++) dp[p] = dq[p];
            sp = sq;
            if constexpr (F::MIN) {
                if ((j & 1) && t == WN - 1 && i == WM - 1) {
                    // Groups j - 1 (k-slot 0) and j (k-slot 1).
#pragma unroll
                    for (int ii = 0; ii < WM; ii++) {
                        float xm = xs[(j - 1 + h) * RM + ii * 32 + c];
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
        finish(WM - 1, WN - 1, NQ == WN * WM);
        // The unit's minimum term joins with it: two separate sums over all
        // of K would cancel in the end.
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int t = 0; t < WN; t++) {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    float y = part[i][t][v];
                    if constexpr (F::MIN) y = y + low[i][t][v];
                    acc[i][t][v] = acc[i][t][v] + y;
                }
                KH_PIN(acc[i][t]);
            }
    };

    // The K loop: stage u + 1 and the weights of u + 1 load while u is
    // multiplied.
    Regs R0[WN], R1[WN];
    Stage st;
    auto wload = [&](Regs (&R)[WN], int u) __attribute__((always_inline)) {
        const bool on = u < u1;
#pragma unroll
        for (int t = 0; t < WN; t++) F::load(R[t], src, on ? ro[t] : NONE, on ? u : 0, h);
    };
    if (u0 < u1) {
        stage_load(st, u0);
        wload(R0, u0);
        stage_store(st, 0);
        __syncthreads();
    }
    auto step = [&](Regs (&Rc)[WN], Regs (&Rn)[WN], int u) __attribute__((always_inline)) {
        const bool more = u + 1 < u1;
        if (more) stage_load(st, u + 1);
        wload(Rn, u + 1);
        compute(Rc, u, (u - u0) & 1);
        if (more) stage_store(st, (u + 1 - u0) & 1);
        __syncthreads();
    };
    for (int u = u0; u < u1; u += 2) {
        step(R0, R1, u);
        if (u + 1 < u1) step(R1, R0, u + 1);
    }

    // Lane (c, h), register v of a tile holds row 8 (v / 4) + 4h + v % 4,
    // column c.
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int t = 0; t < WN; t++) {
            const int64_t n = n0 + t * 32 + c;
            if (n >= (int64_t)a.n[mat]) continue;
            const uint64_t col = a.col0[mat] + (uint64_t)n;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m >= a.rows) continue;
                const float y = acc[i][t][v];
                if (a.ks == 1) store_out(a.out_kind, a.out, (uint64_t)m * a.out_stride + col, y);
                else a.partials[((uint64_t)kz * a.rows + m) * a.width + col] = y;
            }
        }
}

// Rows of activations a workgroup takes: 64 with bytes, 32 with three
// planes (LDS).
template <class F, int P>
hipError_t launch_fp(const MmArgs &a, hipStream_t s) {
    const int groups = a.ngroups * a.ks;
    dim3 grid((unsigned)((groups + XCDS - 1) / XCDS * XCDS * a.mtiles)), block(64 * WAVES);
    constexpr size_t lds1 = 2 * stage_bytes<F, P, 32>(), lds2 = 2 * stage_bytes<F, P, 64>();
    if constexpr (P == 1)
        if (a.wm == 2) {
            hipLaunchKernelGGL((mm_kernel<F, P, 2>), grid, block, lds2, s, a);
            return hipGetLastError();
        }
    if (a.wm == 1)
        hipLaunchKernelGGL((mm_kernel<F, P, 1>), grid, block, lds1, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <class F>
hipError_t launch_f(const MmArgs &a, int planes, hipStream_t s) {
    if (planes == 1) return launch_fp<F, 1>(a, s);
    if (planes == 3) return launch_fp<F, 3>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace mm
}  // namespace kh
