// The product by quantized weights for many rows of float activations (f32,
// bf16 or f16) on gfx950's bf16 matrix cores: the arithmetic of the CPU's
// many-row path (rows decoded to f32, then an f32 product:
// kapel-cpu/src/matmul.rs:198-239), each product to about f32's precision.
//
// The activations come as P exact bf16 planes x0 + .. (prep_bf16_kernel):
// bf16 rows as they are (P = 1; read in place when K is a multiple of 64 and
// x is 16-byte aligned), f16 rows in two planes, f32 rows in three.  The
// weights take one of two modes:
//
// - dot mode (blocks of 32 without a minimum term: Q8_0, Q4_0, Q5_0, IQ4_NL,
//   Kapel int8 / int4 in groups up to 128): the codes (at most 8 significant
//   bits) are exact bf16 B operands; each group's dot sum_k q x over the
//   planes is an f32 MFMA result (v_mfma_f32_32x32x16_bf16), then
//   acc += scale * dot, one fma per output and group;
// - split mode (the others): each weight's f32 value, scale * code - minimum
//   (the CPU decoders' value, kapel-cpu/src/quantized.rs:403-682), is split
//   into three bf16 parts w0 + w1 + w2 (the top 16 bits of the f32, the top
//   16 bits of what is left, the rest rounded to bf16: the f32 exactly), and
//       y[m, n] = sum_k x[m, k] w[n, k] ~= sum_k sum_{i + j <= 2} x_i w_j
//   in f32 MFMAs over all of K (3, 5 or 6 a tile and 16 elements for P = 1,
//   2, 3; the terms left out are below 2^-24 of the product).  Two parts a
//   side (16 bits) fail the CPU's tolerance 1e-4 (1 + |y|) where large terms
//   cancel.
//
// A workgroup of four waves takes RM = 32 WM activation rows by 4 x 32 WN
// weight rows; wave w the weight rows 32 WN w .. + 32 WN of the group, for
// all RM activation rows (WM x WN tiles of 32 x 32).  Lane (c, h) supplies
// row c of a tile and half h of each scale group: with groups of 32 the
// codes 16h .. 16h + 15 (two MFMAs of 8), with groups of 16 the codes 8h ..
// 8h + 7 (one MFMA).  The activations of an MFMA are the same 8 elements of
// the activation row, so every MFMA adds exact bf16 products of matching
// elements.
//
// K runs in steps of 64 elements.  The activations of a step ([P][RM][64]
// bf16, 16-byte chunks swizzled by row) are loaded into registers two steps
// ahead by every wave, written into one of two LDS slots one step ahead, and
// read by all four waves.  A wave's weight rows of a unit are copied by
// coalesced 16-byte loads into registers a unit ahead, then into the wave's
// own LDS slot, where the lane readers of kh_mm.h read them.  Every wait is
// the compiler's: no direct-to-LDS copies.  Sums run in an order fixed by the
// shapes (K in order within a workgroup, then the K splits in order by
// mm_reduce_kernel).
#pragma once
#include "kh_mm.h"

namespace kh {
namespace mmf {

using mm::v16f;
using lanes::NONE;
using lanes::Src;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v16f mfma(v4i a, v4i b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Two f32 as packed bf16 (a low), rounded to nearest even.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
#ifdef KH_EMU_LDS
    return (uint32_t)to_bf16(a) | ((uint32_t)to_bf16(b) << 16);
#else
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), b2));
#endif
}

// NB codes (bytes, two's complement) of one scale group's lane part as
// weights s * code + nm, split: part[j][NB / 2] packed bf16, element e in half
// e % 2 of dword e / 2.  The code is taken as the unsigned byte of code + 128
// (v_cvt_f32_ubyte), the 128 folded into the constant.
template <int NB>
__device__ __forceinline__ void split(const uint32_t (&q)[NB / 4], float s, float nm,
                                      uint32_t (&part)[3][NB / 2]) {
    const float c = fmaf(-128.0f, s, nm);
    // An infinite or NaN weight keeps its first part and no others (w - w0
    // would be NaN): every value of the group is finite or not with s and c.
    const uint32_t keep = isfinite(s) && isfinite(c) ? 0xffffffffu : 0u;
#pragma unroll
    for (int d = 0; d < NB / 4; d++) {
        const uint32_t u = q[d] ^ 0x80808080u;
        float w[4];
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = fmaf(s, (float)((u >> (8 * e)) & 0xffu), c);
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const uint32_t b0 = __float_as_uint(w[2 * p]), b1 = __float_as_uint(w[2 * p + 1]);
            const float r0 = w[2 * p] - __uint_as_float(b0 & 0xffff0000u);
            const float r1 = w[2 * p + 1] - __uint_as_float(b1 & 0xffff0000u);
            const uint32_t m0 = __float_as_uint(r0), m1 = __float_as_uint(r1);
            part[0][2 * d + p] = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
            part[1][2 * d + p] = keep & __builtin_amdgcn_perm(m1, m0, 0x07060302u);
            part[2][2 * d + p] = keep & pk_bf16(r0 - __uint_as_float(m0 & 0xffff0000u),
                                                r1 - __uint_as_float(m1 & 0xffff0000u));
        }
    }
}

// NB signed codes as exact bf16 (|code| <= 128 has at most 8 significant
// bits), packed as split() packs.
template <int NB>
__device__ __forceinline__ void codes_bf16(const uint32_t (&q)[NB / 4], uint32_t (&b)[NB / 2]) {
#pragma unroll
    for (int d = 0; d < NB / 4; d++)
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const float f0 = (float)(int8_t)(q[d] >> (16 * p)), f1 = (float)(int8_t)(q[d] >> (16 * p + 8));
            b[2 * d + p] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
        }
}

__device__ __forceinline__ void code_words(v4i c, uint32_t (&q)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = (uint32_t)c[i];
}
__device__ __forceinline__ void code_words(uint64_t c, uint32_t (&q)[2]) {
    q[0] = (uint32_t)c;
    q[1] = (uint32_t)(c >> 32);
}

constexpr int WAVES = 4;

// The dot mode (codes as the B operand, one scale fma per output and group):
// units of 128 elements without a minimum term (Q8_0, Q4_0, Q5_0, IQ4_NL,
// Kapel int8 / int4 in groups up to 128; the host's choice of kernel lists
// the same formats, mmf_dot_format in kh_api.cpp).
template <class F>
constexpr bool dot_mode() { return !F::MIN && F::U == 128; }

template <class F, int P, int WM, int WN>
struct Plan {
    static constexpr int U = F::U, G = F::G, NG = F::NG, SPU = U / 64, GS = 64 / G;
    static constexpr int RM = 32 * WM, NCOLS = WAVES * WN * 32;
    static constexpr int XB = P * RM * 128;          // bytes of an activation slot
    static constexpr int NXL = P * RM * 8 / (64 * WAVES);  // 16-byte loads a lane a step
    // A wave's weight rows of one unit in LDS: 32 WN rows of CWP 16-byte
    // chunks (the unit's UB bytes from the dword at or below their start),
    // copied by NWL coalesced 16-byte loads a lane.
    static constexpr int UB = U / F::BLEN * F::BYTES;
    static constexpr bool ODD = F::BYTES % 4 != 0;
    static constexpr int CW = (UB + (ODD ? 2 : 0) + 15) / 16, CWP = CW | 1;
    // Row stride in the slot: 8 bytes past the chunks, so that the 32 rows a
    // lane reader's dword read takes fall on 32 different banks (rows at a
    // multiple of 16 bytes took 16; measured 3-6 % shorter on the Q8_0 calls
    // of config 4).  The chunks are written as two 8-byte halves.
    static constexpr int RS = CWP * 16 + 8;
    static constexpr int WB = 32 * WN * RS;          // bytes of a wave's weight slot
    static constexpr int NWL = (32 * WN * CWP + 63) / 64;
    static constexpr int LDS = 2 * XB + WAVES * WB;
    static constexpr int NB = G / 2;                 // code bytes of a lane a group
    static_assert(U % 64 == 0 && P * RM * 8 % (64 * WAVES) == 0, "whole steps and loads");
};

// Two workgroups a CU (two waves a SIMD, at most 256 registers each) for one
// plane, and for every plane count in the dot mode: one wave's waits for LDS,
// loads and barriers are the other's MFMA time (measured: Q8_0 [gate; up]
// 24576 x 4096 at M = 512 with bf16 activations 415 us, against 479 us for one
// wave a SIMD with 256 rows a workgroup; in f32, three planes, 534 us with 10
// registers spilled against 667 us at one wave a SIMD).  One workgroup a CU
// for split weights with two or three planes (their registers would spill).
template <class F, int P>
constexpr int occupancy_of() { return P == 1 || dot_mode<F>() ? 2 : 1; }

template <class F, int P, int WM, int WN>
__global__ __launch_bounds__(256, (occupancy_of<F, P>())) void mmf_kernel(MmArgs a) {
    using L = Plan<F, P, WM, WN>;
    constexpr int U = F::U, G = F::G, NG = F::NG, SPU = L::SPU, GS = L::GS, RM = L::RM, NXL = L::NXL;
    constexpr int NB = L::NB;
    extern __shared__ __align__(16) uint8_t lds[];

    // Workgroup -> (row tile, column group, K split), as mm_kernel.
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
    const int wc = wave * WN * 32;
    int mat = 0;
    for (int i = 1; i < a.count; i++)
        if (ng >= a.ng0[i]) mat = i;
    const int64_t g0 = (int64_t)(ng - a.ng0[mat]) * L::NCOLS;
    const int64_t nmat = (int64_t)a.n[mat];
    const Src wsrc = lanes::source(a.w[mat], a.wbytes[mat]);
    const Src xsrc = lanes::source(a.planes, a.planes_bytes);
    uint32_t wrow[WN];
#pragma unroll
    for (int t = 0; t < WN; t++) {
        const int64_t n = g0 + wc + t * 32 + c;
        wrow[t] = n < nmat ? (uint32_t)n * (uint32_t)a.row_bytes : NONE;
    }

    // The activation chunks of a lane: chunk q = (i WAVES + wave) 64 + lane
    // of a slot is plane p, row r, position q % 8 holding chunk (q % 8) ^ (r
    // % 8) of the row's 128 bytes of the step.
    const uint32_t kbytes = (uint32_t)a.kpad * 2u;
    uint32_t xoff[NXL];
#pragma unroll
    for (int i = 0; i < NXL; i++) {
        const int q = (i * WAVES + wave) * 64 + lane, pr = q / 8, r = pr % RM, p = pr / RM;
        const int o = (q % 8) ^ (r & 7);
        xoff[i] = m0 + r < a.rows ? (uint32_t)(((uint64_t)(m0 + r) * P + p) * kbytes) + 16u * o : NONE;
    }
    const int steps_end = (int)(a.kpad / 64);
    auto load_x = [&](int step, v4i (&v)[NXL]) __attribute__((always_inline)) {
        const bool on = step < steps_end && step < u1 * SPU;
#pragma unroll
        for (int i = 0; i < NXL; i++) {
            const uint32_t off = on && xoff[i] != NONE ? xoff[i] + 128u * step : NONE;
            v[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xsrc.r, (int)off, 0, 0));
        }
    };
    auto store_x = [&](int slot, const v4i (&v)[NXL]) __attribute__((always_inline)) {
        v4i *d = reinterpret_cast<v4i *>(lds + slot * L::XB);
#pragma unroll
        for (int i = 0; i < NXL; i++) d[(i * WAVES + wave) * 64 + lane] = v[i];
    };
    // The A operand of tile i, plane p, chunk o of the step (8 elements).
    auto x_operand = [&](int slot, int i, int p, int o) __attribute__((always_inline)) {
        const int r = i * 32 + c;
        return *reinterpret_cast<const v4i *>(lds + slot * L::XB + ((p * RM + r) * 8 + (o ^ (r & 7))) * 16);
    };

    // The wave's weight rows, unit by unit: coalesced 16-byte loads (chunk
    // ci = i 64 + lane: row ci / CWP, piece ci % CWP) into registers a unit
    // ahead, written to the wave's LDS slot at the unit's start and read
    // back by the lane readers (a load of one lane per row would gather 64
    // rows an instruction: measured 2.4x slower on the Q8_0 layer).
    using Regs = typename F::Regs;
    Regs Rc[WN];
    uint32_t wbase[L::NWL], wpiece[L::NWL];
#pragma unroll
    for (int i = 0; i < L::NWL; i++) {
        const int ci = i * 64 + lane, r = ci / L::CWP, piece = ci % L::CWP;
        const int64_t n = g0 + wc + r;
        wbase[i] = ci < 32 * WN * L::CWP && piece < L::CW && n < nmat ? (uint32_t)n * (uint32_t)a.row_bytes : NONE;
        wpiece[i] = 16u * piece;
    }
    v4i Wn[L::NWL];
    auto load_w = [&](int u) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < L::NWL; i++) {
            const uint32_t at = wbase[i] + (uint32_t)u * L::UB;
            const uint32_t off = wbase[i] != NONE ? (at & ~3u) + wpiece[i] : NONE;
            Wn[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wsrc.r, (int)off, 0, 0));
        }
    };
    uint8_t *wslot = lds + 2 * L::XB + wave * L::WB;
    auto unit_regs = [&](int u) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < L::NWL; i++) {
            const int ci = i * 64 + lane;
            if (ci < 32 * WN * L::CWP) {
                uint8_t *at = wslot + (ci / L::CWP) * L::RS + (ci % L::CWP) * 16;
                if constexpr (L::RS % 16 == 0) {
                    *reinterpret_cast<v4i *>(at) = Wn[i];
                } else {
                    typedef int v2i __attribute__((ext_vector_type(2)));
                    reinterpret_cast<v2i *>(at)[0] = v2i{Wn[i][0], Wn[i][1]};
                    reinterpret_cast<v2i *>(at)[1] = v2i{Wn[i][2], Wn[i][3]};
                }
            }
        }
        // Lanes read rows other lanes wrote: one wave instruction writes for
        // all lanes before the next reads (the barrier only keeps the order).
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int t = 0; t < WN; t++) {
            const int r = t * 32 + c;
            const uint32_t shift =
                L::ODD ? (((uint32_t)(g0 + wc + r) * (uint32_t)a.row_bytes + (uint32_t)u * L::UB) & 3u) : 0u;
            F::load(Rc[t], mm::Lds{wslot}, (uint32_t)(r * L::RS) + shift, 0, h);
        }
    };

    v16f acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int t = 0; t < WN; t++) acc[i][t] = v16f{};

    // Prologue: step u0 SPU into slot 0; steps + 1 and + 2 in registers.
    const int s0 = u0 * SPU;
    v4i X[2][NXL];
    load_w(u0);
    load_x(s0, X[0]);
    load_x(s0 + 1, X[1]);
    store_x(0, X[0]);
    load_x(s0 + 2, X[0]);

    for (int u = u0; u < u1; u++) {
        unit_regs(u);
        if (u + 1 < u1) load_w(u + 1);
        float sc[WN][NG], mn[WN][NG];
#pragma unroll
        for (int t = 0; t < WN; t++) {
            F::scales(Rc[t], sc[t], mn[t]);
#pragma unroll
            for (int j = 0; j < NG; j++) {
                if (!F::MIN) mn[t][j] = 0.0f;
                if (U == 128 && u * U + j * G >= a.k) sc[t][j] = 0.0f, mn[t][j] = 0.0f;
                mn[t][j] = -mn[t][j];
            }
        }
        // The unit's groups in order, software-pipelined: the weights of
        // group j + 1 are decoded, and the activations of the next slot read,
        // while the MFMAs of the current slot run.
        //
        // Blocks of 32 without a minimum term (DOT): the codes themselves are the
        // B operand (exact in bf16); each group's dot of codes and
        // activations, sum_k q x (planes summed), is an f32 MFMA result, and
        // joins the sums as acc += scale * dot (one fma per output and group).
        // Other formats (a minimum term, or 256-element units, for which the
        // dot mode spills registers even at one wave a SIMD): the weights'
        // values in three bf16 parts (split).
        constexpr bool DOT = dot_mode<F>();
        constexpr int WPARTS = DOT ? 1 : 3;
        constexpr int SPG = NB / 8;  // slots (16 elements of K) a group
        uint32_t wcur[WN][WPARTS][NB / 2], wnxt[WN][WPARTS][NB / 2];
        v16f dot[DOT ? WM : 1][DOT ? WN : 1];
        auto decode = [&](int j, uint32_t (&wp)[WN][WPARTS][NB / 2]) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < WN; t++) {
                uint32_t q[NB / 4];
                code_words(F::codes(Rc[t], j, h), q);
                if constexpr (DOT) codes_bf16<NB>(q, wp[t][0]);
                else split<NB>(q, sc[t][j], mn[t][j], *reinterpret_cast<uint32_t(*)[3][NB / 2]>(wp[t]));
            }
        };
        auto read_x = [&](int slot, int o, v4i (&xv)[WM][P]) __attribute__((always_inline)) {
#pragma unroll
            for (int mi = 0; mi < WM; mi++)
#pragma unroll
                for (int p = 0; p < P; p++) xv[mi][p] = x_operand(slot, mi, p, o);
        };
        // Chunk of the step's 128 bytes holding slot z's 8 elements.
        auto chunk = [&](int z) __attribute__((always_inline)) {
            const int jj = z / SPG, s2 = z % SPG;
            return G == 32 ? 4 * jj + 2 * h + s2 : 2 * jj + h;
        };
        decode(0, wcur);
#pragma unroll
        for (int i = 0; i < SPU; i++) {
            const int s = u * SPU + i;
            // Slot s % 2 holds step s (written by every wave a step ago);
            // every wave is done with slot (s + 1) % 2.  SPU is even, so i
            // gives the slots and register sets.
            // (The empty asms keep the compiler from moving LDS accesses
            // across the barrier.)
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            store_x((i + 1) & 1, X[(i + 1) & 1]);
            load_x(s + 3, X[(i + 1) & 1]);
            const int slot = i & 1;
            v4i xc[WM][P], xn[WM][P];
            // Dot mode with one plane: the step's activations read at once
            // (one wait).
            constexpr bool ALL = DOT && P == 1;
            v4i xall[ALL ? 4 : 1][WM][P];
            if constexpr (ALL) {
#pragma unroll
                for (int z = 0; z < 4; z++) read_x(slot, chunk(z), xall[z]);
                asm volatile("" ::: "memory");
            } else {
                read_x(slot, chunk(0), xc);
            }
#pragma unroll
            for (int z = 0; z < 4; z++) {
                const int jj = z / SPG, s2 = z % SPG, j = i * GS + jj;
                if constexpr (ALL) {
#pragma unroll
                    for (int mi = 0; mi < WM; mi++)
#pragma unroll
                        for (int p = 0; p < P; p++) xc[mi][p] = xall[z][mi][p];
                } else if (z + 1 < 4) {
                    read_x(slot, chunk(z + 1), xn);
                }
                if (s2 == SPG - 1 && j + 1 < NG) decode(j + 1, wnxt);
#pragma unroll
                for (int mi = 0; mi < WM; mi++)
#pragma unroll
                    for (int t = 0; t < WN; t++) {
                        v4i bw[WPARTS];
#pragma unroll
                        for (int j3 = 0; j3 < WPARTS; j3++)
                            bw[j3] = v4i{(int)wcur[t][j3][4 * s2], (int)wcur[t][j3][4 * s2 + 1],
                                         (int)wcur[t][j3][4 * s2 + 2], (int)wcur[t][j3][4 * s2 + 3]};
                        if constexpr (DOT) {
#pragma unroll
                            for (int p = P - 1; p >= 0; p--)
                                dot[mi][t] = mfma(xc[mi][p], bw[0], s2 == 0 && p == P - 1 ? v16f{} : dot[mi][t]);
                        } else {
                            // x_i w_j for i + j <= 2, largest terms last.
#pragma unroll
                            for (int p = P - 1; p >= 0; p--)
#pragma unroll
                                for (int j3 = 2 - p; j3 >= 0; j3--)
                                    acc[mi][t] = mfma(xc[mi][p], bw[j3], acc[mi][t]);
                        }
                    }
                if constexpr (DOT) {
                    if (s2 == SPG - 1)
#pragma unroll
                        for (int mi = 0; mi < WM; mi++)
#pragma unroll
                            for (int t = 0; t < WN; t++)
#pragma unroll
                                for (int v = 0; v < 16; v++)
                                    acc[mi][t][v] = fmaf(dot[mi][t][v], sc[t][j], acc[mi][t][v]);
                }
                if (!ALL && z + 1 < 4)
#pragma unroll
                    for (int mi = 0; mi < WM; mi++)
#pragma unroll
                        for (int p = 0; p < P; p++) xc[mi][p] = xn[mi][p];
                if (s2 == SPG - 1 && j + 1 < NG)
#pragma unroll
                    for (int t = 0; t < WN; t++)
#pragma unroll
                        for (int j3 = 0; j3 < WPARTS; j3++)
#pragma unroll
                            for (int e = 0; e < NB / 2; e++) wcur[t][j3][e] = wnxt[t][j3][e];
            }
        }
    }

    // Lane (c, h), register v of tile (i, t): activation row i 32 + 8 (v / 4)
    // + 4h + v % 4, weight row wc + 32 t + c.
    const bool partial = a.ks > 1;
#pragma unroll
    for (int t = 0; t < WN; t++) {
        const int64_t n = g0 + wc + t * 32 + c;
        if (n >= nmat) continue;
        const uint64_t col = a.col0[mat] + (uint64_t)n;
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m >= a.rows) continue;
                if (partial) a.partials[((uint64_t)kz * a.rows + m) * a.width + col] = acc[i][t][v];
                else store_out(a.out_kind, a.out, (uint64_t)m * a.out_stride + col, acc[i][t][v]);
            }
    }
}

// Activation rows a workgroup takes: 256 for one or two planes, 128 for
// three (registers); one weight tile a wave (128 weight rows a workgroup).
// Activation rows a workgroup takes: 128 (four tiles a wave) where the
// weights are split into three parts, 64 (two tiles a wave) for the dot mode
// (its dot sums take the registers of two more tiles; measured on the Q8_0
// layer of config 4 at M = 512: 12 % shorter than four tiles a wave at one
// wave a SIMD); one weight tile a wave (128 weight rows a workgroup).
template <class F, int P>
constexpr int wm_of() { return dot_mode<F>() ? 2 : 4; }
constexpr int WN_ALL = 1;

template <class F, int P>
hipError_t launch_p(const MmArgs &a_in, hipStream_t s) {
    constexpr int WM = wm_of<F, P>(), WN = WN_ALL;
    using L = Plan<F, P, WM, WN>;
    MmArgs a = a_in;
    a.mtiles = (a.rows + L::RM - 1) / L::RM;
    constexpr int bytes = L::LDS;  // the IQ3_S grid is static LDS
    static OncePerDevice once;
    hipError_t e = set_lds_limit(once, reinterpret_cast<const void *>(&mmf_kernel<F, P, WM, WN>), bytes);
    if (e != hipSuccess) return e;
    const int groups = a.ngroups * a.ks;
    dim3 grid((unsigned)((groups + XCDS - 1) / XCDS * XCDS * a.mtiles)), block(64 * WAVES);
    hipLaunchKernelGGL((mmf_kernel<F, P, WM, WN>), grid, block, (size_t)bytes, s, a);
    return hipGetLastError();
}

// planes: 1 (bf16 activations), 2 (f16) or 3 (f32); cols: the weight rows of a column group
// instead of a launch.
template <class F>
hipError_t launch_f(const MmArgs &a, int planes, hipStream_t s, int *cols) {
    if (cols) {
        *cols = Plan<F, 1, wm_of<F, 1>(), WN_ALL>::NCOLS;
        return hipSuccess;
    }
    if (planes == 1) return launch_p<F, 1>(a, s);
    if (planes == 2) return launch_p<F, 2>(a, s);
    if (planes == 3) return launch_p<F, 3>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace mmf
}  // namespace kh
