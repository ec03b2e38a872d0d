// Lane readers of the quantized formats for the small-M product (kh_gemv.hip).
//
// A wave takes 16 weight rows; lane l serves row n = l % 16 as "lane group"
// g = l / 16.  The product walks a row by units (256 elements for the
// 256-element super-blocks, 128 for the 32-element blocks and Kapel's
// int8/int4 groups).  In a unit, each lane group owns its own elements: for
// every MFMA step s the 16 codes a lane gives as B operand of
// v_mfma_i32_16x16x64_i8 are 16 elements of ONE scale group of that lane
// group, and the activations (A operand) of that step are the 16 elements at
// unit offset xpos(g, s), consecutive.  Each lane therefore gets back in C
// exactly the dots of its own groups and applies their scales itself.
//
// A reader loads its lane's bytes with the widest buffer loads the alignment
// allows (16-byte loads at 4-byte-aligned offsets; formats whose blocks start
// at even offsets only are read from the 4-byte-aligned offset below and put
// back in place with v_alignbyte).
// Scales and minimums are the f32 products of the CPU decoders
// (kapel-cpu/src/quantized.rs:403-682, k_scales :603-616); element layouts
// follow kapel-core/src/dtype.rs:342-520.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_iq.h"

namespace kh {
namespace lanes {

typedef int v4i __attribute__((ext_vector_type(4)));
constexpr uint32_t LO4 = 0x0f0f0f0fu;

// ---------------------------------------------------------------- loads
// A weight matrix is read through a buffer resource: raw buffer loads at
// 32-bit byte offsets, bounds-checked by the hardware against the matrix
// size rounded up to whole dwords.  An offset past the end reads zeros and
// touches no memory, which lets a lane with nothing to read still issue its
// loads (NONE), so every wave issues the same loads in the same order.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x3 __attribute__((ext_vector_type(3)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t NONE = 0x80000000u;  // past every matrix (< 2 GiB each)

struct Src {
    __amdgpu_buffer_rsrc_t r;
};

__device__ __forceinline__ Src source(const void *base, uint32_t bytes) {
    return Src{__builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)((bytes + 3u) & ~3u),
                                                 0x00020000)};
}

// N dwords at byte offset off (a multiple of 4, or NONE).
template <int N>
__device__ __forceinline__ void ldb(uint32_t (&v)[N], const Src &s, uint32_t off) {
    int i = 0;
#pragma unroll
    for (; i + 4 <= N; i += 4) {
        u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(s.r, (int)(off + 4 * i), 0, 0);
        v[i] = t.x, v[i + 1] = t.y, v[i + 2] = t.z, v[i + 3] = t.w;
    }
    if (N - i == 3) {
        u32x3 t = __builtin_amdgcn_raw_buffer_load_b96(s.r, (int)(off + 4 * i), 0, 0);
        v[i] = t.x, v[i + 1] = t.y, v[i + 2] = t.z;
    } else if (N - i == 2) {
        u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(s.r, (int)(off + 4 * i), 0, 0);
        v[i] = t.x, v[i + 1] = t.y;
    } else if (N - i == 1) {
        v[i] = __builtin_amdgcn_raw_buffer_load_b32(s.r, (int)(off + 4 * i), 0, 0);
    }
}

// The bytes [off, off + R) at an even offset, as ceil(R / 4) dwords in
// place: the dwords from off - (off % 4) on, then shifted by v_alignbyte.
// The two bytes below an odd-halfword offset belong to the matrix (which
// starts at a multiple of 4); the bytes past the run are in the matrix's
// last dword or beyond it (zeros).
template <int R>
__device__ __forceinline__ void run(uint32_t (&w)[(R + 3) / 4], const Src &src, uint32_t off) {
    static_assert(R % 2 == 0, "even runs only");
    constexpr int D = (R + 5) / 4, W = (R + 3) / 4;
    const uint32_t s = off & 2u;
    uint32_t v[D + 1];
    ldb<D>(*reinterpret_cast<uint32_t(*)[D]>(v), src, off - s);
    v[D] = 0u;
#pragma unroll
    for (int i = 0; i < W; i++) w[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], s);
}

// The same reads from LDS (a workgroup's copy of the bytes): N dwords at a
// multiple of 4, runs at even offsets.
struct LdsSrc {
    const uint8_t *p;
};

template <int N>
__device__ __forceinline__ void ldb(uint32_t (&v)[N], const LdsSrc &s, uint32_t off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(s.p + off);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = w[i];
}

template <int R>
__device__ __forceinline__ void run(uint32_t (&w)[(R + 3) / 4], const LdsSrc &src, uint32_t off) {
    static_assert(R % 2 == 0, "even runs only");
    constexpr int D = (R + 5) / 4, W = (R + 3) / 4;
    const uint32_t s = off & 2u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(src.p + (off - s));
    uint32_t v[D + 1];
#pragma unroll
    for (int i = 0; i < D; i++) v[i] = p[i];
    v[D] = 0u;
#pragma unroll
    for (int i = 0; i < W; i++) w[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], s);
}

__device__ __forceinline__ float f16(uint32_t h) { return __half2float(__ushort_as_half((uint16_t)h)); }
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }
// Dword i of a 16-byte vector held as four dwords.
__device__ __forceinline__ v4i vec(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return v4i{(int)a, (int)b, (int)c, (int)d};
}
__device__ __forceinline__ v4i lo4(const uint32_t *q) {
    return vec(q[0] & LO4, q[1] & LO4, q[2] & LO4, q[3] & LO4);
}
__device__ __forceinline__ v4i hi4(const uint32_t *q) {
    return vec((q[0] >> 4) & LO4, (q[1] >> 4) & LO4, (q[2] >> 4) & LO4, (q[3] >> 4) & LO4);
}

// ------------------------------------------------------------- Q4_K
// 144 bytes: d, dmin, 12 bytes of 6-bit scales/minimums, 128 bytes of
// nibbles (dtype.rs:441-457): byte 16 + 32c + l holds element 64c + l (low
// nibble) and 64c + 32 + l (high).  Lane group g takes c = g: its sub-blocks
// are 2g (steps 0, 1) and 2g + 1 (steps 2, 3).
// The scales and minimums of sub-blocks 2g and 2g + 1 at once: bytes 2g,
// 2g + 1 of the 6-bit fields (k_scales, quantized.rs:603-616), two lanes of
// 16 bits each, then each byte to f32.
__device__ __forceinline__ void k_pair(const uint32_t (&h)[4], int g, float (&s)[2], float (&m)[2]) {
    // Both forms computed and one selected: lane groups 0-1 and 2-3 of a
    // wave take different ones, and a branch would run both in turn.
    const int sh = 16 * (g & 1);
    const uint32_t lo = h[3] >> sh;
    const uint32_t sc_low = (h[1] >> sh) & 0x3f3fu, mn_low = (h[2] >> sh) & 0x3f3fu;
    const uint32_t sc_high = (lo & 0x0f0fu) | ((h[1] >> (sh + 2)) & 0x3030u);
    const uint32_t mn_high = ((lo >> 4) & 0x0f0fu) | ((h[2] >> (sh + 2)) & 0x3030u);
    const uint32_t sc = g < 2 ? sc_low : sc_high, mn = g < 2 ? mn_low : mn_high;
    const float d = f16(h[0] & 0xffffu), dmin = f16(h[0] >> 16);
    s[0] = d * (float)(sc & 0xffu);
    s[1] = d * (float)(sc >> 8);
    m[0] = dmin * (float)(mn & 0xffu);
    m[1] = dmin * (float)(mn >> 8);
}

struct Q4K {
    static constexpr int U = 256, STEPS = 4, GS = 32, BYTES = 144, BLEN = 256;
    struct Regs {
        uint32_t h[4], q[8];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        ldb<4>(r.h, src, b);
        ldb<8>(r.q, src, b + 16 + 32 * g);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        const uint32_t *q = r.q + 4 * (s & 1);
        return (s >> 1) ? hi4(q) : lo4(q);
    }
    __device__ static int xpos(int g, int s) { return 64 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int g, float (&sc)[2], float (&mn)[2]) {
        k_pair(r.h, g, sc, mn);
    }
};

// ------------------------------------------------------------- Q5_K
// 176 bytes: as Q4_K with 32 bytes of fifth bits at 16: bit j of byte l is
// the fifth bit of element 32j + l; nibbles at 48.
struct Q5K {
    static constexpr int U = 256, STEPS = 4, GS = 32, BYTES = 176, BLEN = 256;
    struct Regs {
        uint32_t h[4], qh[8], q[8];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        ldb<4>(r.h, src, b);
        ldb<8>(r.qh, src, b + 16);
        ldb<8>(r.q, src, b + 48 + 32 * g);
    }
    __device__ static v4i codes(const Regs &r, int s, int g) {
        const uint32_t *q = r.q + 4 * (s & 1), *h = r.qh + 4 * (s & 1);
        int j = 2 * g + (s >> 1);
        v4i c = (s >> 1) ? hi4(q) : lo4(q);
        for (int i = 0; i < 4; i++) c[i] |= (int)(((h[i] >> j) & 0x01010101u) << 4);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 64 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int g, float (&sc)[2], float (&mn)[2]) {
        k_pair(r.h, g, sc, mn);
    }
};

// ------------------------------------------------------------- Q6_K
// 210 bytes (dtype.rs:458-469): 128 bytes of low nibbles, 64 of 2-bit
// highs, 16 signed scales, d.  Element 128h + 32t + l: low nibble t / 2 of
// byte 64h + 32(t % 2) + l, high bits 2t of byte 128 + 32h + l, scale
// (128h + 32t + l) / 16.  Lane group g: h = g / 2, t % 2 = g % 2; step s:
// t = g % 2 + 2(s / 2), l = 16(s % 2) .. + 15.  Codes are stored + 32.
struct Q6K {
    static constexpr int U = 256, STEPS = 4, GS = 16, BYTES = 210, BLEN = 256;
    struct Regs {
        uint32_t ql[8], qh[8], sc[2], d;
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        int h = g >> 1, q = g & 1;
        run<32>(r.ql, src, b + 64 * h + 32 * q);
        run<32>(r.qh, src, b + 128 + 32 * h);
        run<8>(r.sc, src, b + 192 + 8 * h);
        uint32_t d[1];
        run<2>(d, src, b + 208);
        r.d = d[0] & 0xffffu;
    }
    __device__ static v4i codes(const Regs &r, int s, int g) {
        const uint32_t *l = r.ql + 4 * (s & 1), *h = r.qh + 4 * (s & 1);
        int ls = 4 * (s >> 1), hs = 2 * (g & 1) + 4 * (s >> 1);
        v4i c;
        for (int i = 0; i < 4; i++)
            c[i] = (int)(((l[i] >> ls) & LO4) | (((h[i] >> hs) & 0x03030303u) << 4));
        return c;
    }
    __device__ static int xpos(int g, int s) {
        return 128 * (g >> 1) + 32 * ((g & 1) + 2 * (s >> 1)) + 16 * (s & 1);
    }
    __device__ static void scales(const Regs &r, int g, float (&sc)[4], float (&mn)[4]) {
        const float d = f16(r.d);
        for (int s = 0; s < 4; s++) {
            int i = 2 * (g & 1) + 4 * (s >> 1) + (s & 1);  // byte of the 8 loaded
            sc[s] = d * (float)(int8_t)byte_of(r.sc[i >> 2], i & 3);
            mn[s] = 32.0f * sc[s];
        }
    }
    static constexpr int SIGNED_OFFSET = 32;
};

// ------------------------------------------------------------- Q2_K
// 84 bytes (dtype.rs:413-422): 16 scale bytes (low nibble scale, high
// minimum), 64 bytes of 2-bit codes, d, dmin.  Element 128h + 32t + l: bits
// 2t of byte 16 + 32h + l; group e / 16.  Lane group g: h = g / 2, l =
// 16(g % 2) .. + 15; step s: t = s.
struct Q2K {
    static constexpr int U = 256, STEPS = 4, GS = 16, BYTES = 84, BLEN = 256;
    struct Regs {
        uint32_t q[4], sc[2], dd;
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        int h = g >> 1;
        ldb<4>(r.q, src, b + 16 + 32 * h + 16 * (g & 1));
        ldb<2>(r.sc, src, b + 8 * h);
        uint32_t dd[1];
        ldb<1>(dd, src, b + 80);
        r.dd = dd[0];
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        v4i c;
        for (int i = 0; i < 4; i++) c[i] = (int)((r.q[i] >> (2 * s)) & 0x03030303u);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 128 * (g >> 1) + 32 * s + 16 * (g & 1); }
    __device__ static void scales(const Regs &r, int g, float (&sc)[4], float (&mn)[4]) {
        const float d = f16(r.dd & 0xffffu), dmin = f16(r.dd >> 16);
        for (int s = 0; s < 4; s++) {
            int i = 2 * s + (g & 1);
            uint32_t k = byte_of(r.sc[i >> 2], i & 3);
            sc[s] = d * (float)(k & 15u);
            mn[s] = dmin * (float)(k >> 4);
        }
    }
};

// ------------------------------------------------------------- Q3_K
// 110 bytes (dtype.rs:423-440): 32 bytes of high-bit masks, 64 of 2-bit
// codes, 12 of packed 6-bit scales, d.  Element 128h + 32t + l: low bits 2t
// of byte 32 + 32h + l, high bit 4h + t of byte l; value d scale ((low |
// high << 2) - 4).  Lanes as Q2_K.
struct Q3K {
    static constexpr int U = 256, STEPS = 4, GS = 16, BYTES = 110, BLEN = 256;
    struct Regs {
        uint32_t hm[4], q[4], sc[3], d;
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        int h = g >> 1;
        run<16>(r.hm, src, b + 16 * (g & 1));
        run<16>(r.q, src, b + 32 + 32 * h + 16 * (g & 1));
        run<12>(r.sc, src, b + 96);
        uint32_t d[1];
        run<2>(d, src, b + 108);
        r.d = d[0] & 0xffffu;
    }
    __device__ static v4i codes(const Regs &r, int s, int g) {
        int hs = 4 * (g >> 1) + s;
        v4i c;
        for (int i = 0; i < 4; i++)
            c[i] = (int)(((r.q[i] >> (2 * s)) & 0x03030303u) | (((r.hm[i] >> hs) & 0x01010101u) << 2));
        return c;
    }
    __device__ static int xpos(int g, int s) { return Q2K::xpos(g, s); }
    __device__ static void scales(const Regs &r, int g, float (&sc)[4], float (&mn)[4]) {
        const float d = f16(r.d);
        for (int s = 0; s < 4; s++) {
            int i = 8 * (g >> 1) + 2 * s + (g & 1);
            int a = i % 8, c = 8 + i % 4;
            uint32_t lo = (byte_of(r.sc[a >> 2], a & 3) >> (4 * (i / 8))) & 15u;
            uint32_t hi = (byte_of(r.sc[c >> 2], c & 3) >> (2 * (i / 4))) & 3u;
            sc[s] = d * (float)((int)(lo | (hi << 4)) - 32);
            mn[s] = 4.0f * sc[s];
        }
    }
};

// ----------------------------------------------- blocks of 32 elements
// A unit is 4 blocks: lane group g takes block 4u + g (steps 0 and 1: its
// elements 0..15 and 16..31).  Lanes whose block lies beyond K load nothing.
__device__ __forceinline__ void nib_codes(v4i &c, const uint32_t *q, int s) {
    c = s ? hi4(q) : lo4(q);
}

// Q4_0: 18 bytes, d then 16 bytes (byte j: element j low, j + 16 high).
struct Q4_0 {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 18, BLEN = 32;
    struct Regs {
        uint32_t w[5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        run<18>(r.w, src, row + (4 * u + g) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        uint32_t q[4];
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
        v4i c;
        nib_codes(c, q, s);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = f16(r.w[0] & 0xffffu);
        mn[0] = 8.0f * sc[0];
    }
};

// Q4_1: 20 bytes, d, m, then nibbles; w = d q + m.
struct Q4_1 {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 20, BLEN = 32;
    struct Regs {
        uint32_t w[5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        ldb<5>(r.w, src, row + (4 * u + g) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        v4i c;
        nib_codes(c, r.w + 1, s);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = f16(r.w[0] & 0xffffu);
        mn[0] = -f16(r.w[0] >> 16);
    }
};

// Fifth bits of Q5_0 / Q5_1: bits j .. j + 3 of `high` to bit 4 of bytes.
__device__ __forceinline__ uint32_t spread4(uint32_t high, int j) {
    uint32_t x = (high >> j) & 15u;
    return ((x * 0x00204081u) & 0x01010101u) << 4;
}

// Q5_0: 22 bytes, d, 4 bytes of fifth bits (bit j: element j), nibbles;
// w = d (q - 16).  Q5_1: 24 bytes, d, m, fifth bits, nibbles; w = d q + m.
template <bool ONE>
struct Q5x {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = ONE ? 24 : 22, BLEN = 32;
    struct Regs {
        uint32_t w[(BYTES + 3) / 4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + (4 * u + g) * BYTES;
        if (ONE) ldb<6>(*reinterpret_cast<uint32_t(*)[6]>(r.w), src, b);
        else run<22>(*reinterpret_cast<uint32_t(*)[6]>(r.w), src, b);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        uint32_t high, q[4];
        if (ONE) {
            high = r.w[1];
            for (int i = 0; i < 4; i++) q[i] = r.w[2 + i];
        } else {
            high = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2);
            for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[2 + i], r.w[1 + i], 2);
        }
        v4i c;
        nib_codes(c, q, s);
        for (int i = 0; i < 4; i++) c[i] |= (int)spread4(high, 16 * s + 4 * i);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = f16(r.w[0] & 0xffffu);
        mn[0] = ONE ? -f16(r.w[0] >> 16) : 16.0f * sc[0];
    }
};
using Q5_0 = Q5x<false>;
using Q5_1 = Q5x<true>;

// Q8_0: 34 bytes, d then 32 signed bytes (dtype.rs:375-378).
struct Q8_0 {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 34, BLEN = 32;
    struct Regs {
        uint32_t w[9];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        run<34>(r.w, src, row + (4 * u + g) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        v4i c;
        for (int i = 0; i < 4; i++)
            c[i] = (int)__builtin_amdgcn_alignbyte(r.w[4 * s + i + 1], r.w[4 * s + i], 2);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = f16(r.w[0] & 0xffffu);
        mn[0] = 0.0f;
    }
};

// Kapel int8 / int4 in groups of G (a multiple of 32): an f32 scale, then G
// bytes, or G / 2 bytes of nibbles (element 2i low, 2i + 1 high)
// (dtype.rs:364-374).  Lane group g takes the 32 elements of piece 4u + g.
template <int G>
struct Int8G {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 4 + G, BLEN = G;
    struct Regs {
        uint32_t scale, q[8];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        int p = 4 * u + g;
        const uint32_t b = row + (32 * p / G) * BYTES;
        uint32_t sc[1];
        ldb<1>(sc, src, b);
        r.scale = sc[0];
        ldb<8>(r.q, src, b + 4 + (32 * p) % G);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        return vec(r.q[4 * s], r.q[4 * s + 1], r.q[4 * s + 2], r.q[4 * s + 3]);
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = __uint_as_float(r.scale);
        mn[0] = 0.0f;
    }
};

template <int G>
struct Int4G {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 4 + G / 2, BLEN = G;
    struct Regs {
        uint32_t scale, q[4];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        int p = 4 * u + g;
        const uint32_t b = row + (32 * p / G) * BYTES;
        uint32_t sc[1];
        ldb<1>(sc, src, b);
        r.scale = sc[0];
        ldb<4>(r.q, src, b + 4 + ((32 * p) % G) / 2);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        v4i c;
        for (int i = 0; i < 2; i++) {
            uint32_t w = r.q[2 * s + i], lo = w & LO4, hi = (w >> 4) & LO4;
            c[2 * i] = (int)__builtin_amdgcn_perm(hi, lo, 0x05010400u);
            c[2 * i + 1] = (int)__builtin_amdgcn_perm(hi, lo, 0x07030602u);
        }
        return c;
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = __uint_as_float(r.scale);
        mn[0] = 8.0f * sc[0];
    }
};


// ------------------------------------------------- the non-linear formats
// Codes become their signed values (kh_iq.h); no minimum.  f32 activations
// only: the byte mode has no reader for them (bytes.rs:51-77).
__device__ __forceinline__ v4i iq4_vec(const uint32_t *q, int s) {
    v4i c;
    for (int i = 0; i < 4; i++) c[i] = (int)iq4_bytes(s ? (q[i] >> 4) & LO4 : q[i] & LO4);
    return c;
}

// IQ4_NL: 18 bytes, d then 16 bytes of codes as Q4_0's (quantized.rs:420-433).
struct IQ4NL {
    static constexpr int U = 128, STEPS = 2, GS = 32, BYTES = 18, BLEN = 32;
    struct Regs {
        uint32_t w[5];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        run<18>(r.w, src, row + (4 * u + g) * BYTES);
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        uint32_t q[4];
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
        return iq4_vec(q, s);
    }
    __device__ static int xpos(int g, int s) { return 32 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[1], float (&mn)[1]) {
        sc[0] = f16(r.w[0] & 0xffffu);
        mn[0] = 0.0f;
    }
};

// IQ4_XS: 136 bytes (quantized.rs:435-452): d, 16 high scale bits, 4 bytes of
// low scale nibbles, then group G's 16 bytes at 8 + 16G (element 32G + j:
// low nibble of byte j, 32G + 16 + j: high nibble); scale d (s - 32).  Lane
// group g takes groups 2g (steps 0, 1) and 2g + 1 (steps 2, 3).
struct IQ4XS {
    static constexpr int U = 256, STEPS = 4, GS = 32, BYTES = 136, BLEN = 256;
    struct Regs {
        uint32_t h[2], q[8];
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        ldb<2>(r.h, src, b);
        ldb<8>(r.q, src, b + 8 + 32 * g);
    }
    __device__ static v4i codes(const Regs &r, int s, int) { return iq4_vec(r.q + 4 * (s >> 1), s & 1); }
    __device__ static int xpos(int g, int s) { return 64 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int g, float (&sc)[2], float (&mn)[2]) {
        const float d = f16(r.h[0] & 0xffffu);
        for (int i = 0; i < 2; i++) {
            const int G = 2 * g + i;
            const int s = (int)((byte_of(r.h[1], g) >> (4 * i)) & 15u) | (int)(((r.h[0] >> (16 + 2 * G)) & 3u) << 4);
            sc[i] = d * (float)(s - 32);
            mn[i] = 0.0f;
        }
    }
};

// IQ3_S: 110 bytes (quantized.rs:454-485): d; 64 index bytes (group G's 8 at
// 2 + 8G); 8 bytes of ninth index bits (byte G, bit i for index i); 32 sign
// bytes (group G's 4 at 74 + 4G, byte l for elements 8l .. 8l + 7); 4 scale
// bytes (nibble G of 106: scale d (1 + 2s)).  Lane group g takes groups 2g
// and 2g + 1 as IQ4_XS; step s is dword s of its 16 index bytes: indices
// 4(s % 2) .. + 3 of group 2g + s / 2, 16 elements.
struct IQ3S {
    static constexpr int U = 256, STEPS = 4, GS = 32, BYTES = 110, BLEN = 256;
    static constexpr bool GRID = true;
    struct Regs {
        uint32_t c[4], hs, sg[2], sc, d;
    };
    template <class S>
    __device__ static void load(Regs &r, const S &src, uint32_t row, int u, int g) {
        const uint32_t b = row + u * BYTES;
        uint32_t t[1];
        run<16>(r.c, src, b + 2 + 16 * g);
        run<2>(t, src, b + 66 + 2 * g);
        r.hs = t[0] & 0xffffu;
        run<8>(r.sg, src, b + 74 + 8 * g);
        run<4>(t, src, b + 106);
        r.sc = byte_of(t[0], g);
        run<2>(t, src, b);
        r.d = t[0] & 0xffffu;
    }
    __device__ static v4i codes(const Regs &r, int s, int) {
        const uint32_t q = r.c[s], hb = byte_of(r.hs, s >> 1) >> (4 * (s & 1));
        const uint32_t sg = r.sg[s >> 1] >> (16 * (s & 1));
        v4i c;
        for (int i = 0; i < 4; i++)
            c[i] = (int)iq3s_bytes(byte_of(q, i) | (((hb >> i) & 1u) << 8), (sg >> (4 * i)) & 15u);
        return c;
    }
    __device__ static int xpos(int g, int s) { return 64 * g + 16 * s; }
    __device__ static void scales(const Regs &r, int, float (&sc)[2], float (&mn)[2]) {
        const float d = f16(r.d);
        for (int i = 0; i < 2; i++) {
            sc[i] = d * (float)(1u + 2u * ((r.sc >> (4 * i)) & 15u));
            mn[i] = 0.0f;
        }
    }
};

}  // namespace lanes
}  // namespace kh
