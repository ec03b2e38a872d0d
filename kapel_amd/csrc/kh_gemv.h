// The product by quantized weights for few activation rows (decode: M <= 8
// with f32 activations, M <= 16 with byte activations) on gfx950.
//
// A workgroup is four waves taking 1, 2 or 4 tiles of 16 weight rows; the
// waves of a tile split K between them (units of 128 or 256 elements, dealt
// in turn).  For each chunk of K the workgroup:
//
//  1. issues the loads of each wave's first weights (lane readers,
//     kh_lanes.h);
//  2. prepares the chunk's activations in LDS: by blocks of 32, int8
//     "planes" and per-block scales and sums.  With byte activations the
//     one plane is the CPU's q and the scale its s (kapel-cpu/src/
//     bytes.rs:144-158).  With float activations each block becomes a
//     23-bit fixed-point number v = rint(x 2^sh) (sh = 22 - exponent of the
//     block's largest magnitude) in three signed bytes, v = a 2^16 + b 2^8 +
//     c, so that the integer dots of the planes give the dot of v exactly;
//  3. per unit and MFMA step, multiplies the codes of 16 rows (B) by the
//     planes (A) with v_mfma_i32_16x16x64_i8.  A row 4g + j of A holds plane
//     (or activation row) j only in the k-slice of lane group g, zero
//     elsewhere, so lane (n, g) gets back the dots of its own scale group
//     for every plane and row, and adds scale * xscale * dot - minimum * xsum
//     to its sums, group after group.
//
// At the end the four lane groups of a row are added in a fixed tree, then
// the waves of a tile in wave order, through LDS.  No workgroup waits for
// another (no atomics, no cache flushes).
//
// Every reduction is split by the shapes alone (units, chunks, lanes), never
// by timing or the number of CUs: results are bitwise the same run to run.
// Workgroups are numbered so that the chunks of one row range share an XCD.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_internal.h"
#include "kh_lanes.h"

namespace kh {
namespace {

using lanes::v4i;

constexpr int XCDS = 8;


// How the kernel reads the activations: f32 (16-byte aligned), bf16 or f16
// (8-byte aligned; which of the two is a runtime flag with no branch), or
// int8 (4-byte aligned, block dots).
enum XKind { X_F32 = 0, X_H16 = 1, X_I8 = 2 };

// Four consecutive activations, elements i .. i + 3 (i % 4 == 0).
template <int XK>
__device__ __forceinline__ void x4(const void *x, uint64_t i, bool bf16, float (&v)[4]) {
    if (XK == X_F32) {
        float4 f = *reinterpret_cast<const float4 *>(static_cast<const float *>(x) + i);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else if (XK == X_H16) {
        uint2 h = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(x) + i);
        uint32_t hs[4] = {h.x & 0xffffu, h.x >> 16, h.y & 0xffffu, h.y >> 16};
        for (int j = 0; j < 4; j++) {
            float b = __uint_as_float(hs[j] << 16), f = __half2float(__ushort_as_half((uint16_t)hs[j]));
            v[j] = bf16 ? b : f;
        }
    } else {
        uint32_t w = *reinterpret_cast<const uint32_t *>(static_cast<const int8_t *>(x) + i);
        for (int j = 0; j < 4; j++) v[j] = (float)(int8_t)(w >> (8 * j));
    }
}

__device__ __forceinline__ uint16_t to_bf16(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ void store_out(uint32_t kind, void *out, uint64_t i, float v) {
    if (kind == KH_F32) static_cast<float *>(out)[i] = v;
    else if (kind == KH_BF16) static_cast<uint16_t *>(out)[i] = to_bf16(v);
    else static_cast<uint16_t *>(out)[i] = __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d) {
    return ((uint32_t)a & 0xffu) | (((uint32_t)b & 0xffu) << 8) | (((uint32_t)c & 0xffu) << 16) |
           ((uint32_t)d << 24);
}

// Step 2: the chunk's activations into LDS, by the first waves of the
// workgroup (`nthreads` threads).  Thread t takes quads (4 elements) t, t +
// nthreads, ... (at most PASSES each); eight consecutive threads hold a block
// of 32.  x_load issues the loads (before any weight load of these waves, so
// that waiting for x does not wait for the weights), x_prepare
// writes planes: [rows][P][span] int8 and info: [rows][span / 32] of
// {xscale, xsum32, xsum16 (first half), xsum16 (second half)}, xsum = xscale
// * the integer sum of the block's (or half's) values.
constexpr int PASSES = 4;

// The activations a workgroup prepares: rows [rows, k] at x, of kind x_kind.
struct XIn {
    const void *x;
    int rows, k;
    uint32_t kind;
};

// Cross-lane steps inside a block of 32 activations (8 lanes): DPP quad
// permutations for lanes ^ 1 and ^ 2, ds_swizzle for lanes ^ 4.
__device__ __forceinline__ int lane_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, true); }
__device__ __forceinline__ int lane_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, true); }
__device__ __forceinline__ int lane_xor4(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x1f | (4 << 10)); }

// The row and quad of a thread's quad q (rows of qpr quads; rows <= 16).
__device__ __forceinline__ void quad_at(int q, int qpr, int &m, int &eq) {
    m = 0;
    eq = q;
    while (eq >= qpr) {
        eq -= qpr;
        m++;
    }
}

template <int XK>
__device__ __forceinline__ void x_load(const XIn &a, int e0, int span, int q0, int tid, int nthreads,
                                       float (&v)[PASSES][4]) {
    const int qpr = span / 4, quads = a.rows * qpr;
#pragma unroll
    for (int i = 0; i < PASSES; i++) {
        // Every thread loads (from the last quad when it has none), so that
        // the loads issued after these can be counted on.
        int q = q0 + tid + nthreads * i, m, eq;
        quad_at(q, qpr, m, eq);
        int e = e0 + 4 * eq;
        bool in = q < quads && e < a.k;
        x4<XK>(a.x, in ? (uint64_t)m * a.k + e : (uint64_t)a.rows * a.k - 4, a.kind == KH_BF16, v[i]);
        for (int j = 0; j < 4; j++) v[i][j] = in ? v[i][j] : 0.0f;
    }
}

template <int P, int XK>
__device__ void x_prepare(const XIn &a, int span, int q0, int tid, int nthreads,
                          const float (&v)[PASSES][4], int8_t *planes, float4 *info) {
    const int qpr = span / 4, quads = a.rows * qpr;
    const int wave0 = tid & ~63;
#pragma unroll
    for (int i = 0; i < PASSES; i++) {
        if (q0 + nthreads * i + wave0 >= quads) break;  // nothing for this wave
        int q = q0 + tid + nthreads * i, m, eq;
        quad_at(q, qpr, m, eq);
        // The block's largest magnitude as an integer maximum of the bit
        // patterns (their order for non-negative floats); NaN and infinity
        // are at or above 0x7f800000.
        uint32_t mag[4];
        for (int j = 0; j < 4; j++) {
            mag[j] = __float_as_uint(v[i][j]) & 0x7fffffffu;
            // f32::max ignores NaN (bytes.rs:148-151).
            if (P == 1 && XK != X_I8) mag[j] = mag[j] > 0x7f800000u ? 0u : mag[j];
        }
        uint32_t top = max(max(mag[0], mag[1]), max(mag[2], mag[3]));
        top = max(top, (uint32_t)lane_xor1((int)top));
        top = max(top, (uint32_t)lane_xor2((int)top));
        top = max(top, (uint32_t)lane_xor4((int)top));
        const float max = __uint_as_float(top);
        int val[4];
        float xscale;
        if (P == 1 && XK == X_I8) {
            xscale = 1.0f;
            for (int j = 0; j < 4; j++) val[j] = (int)v[i][j];
        } else if (P == 1) {
            // bytes.rs:152-156: s = max / 127, q = round-half-even(x (127 /
            // max)) clamped to +-127, NaN -> 0 (correctly rounded divisions).
            xscale = max / 127.0f;
            float inverse = max > 0.0f ? 127.0f / max : 0.0f;
            for (int j = 0; j < 4; j++) {
                float r = rintf(v[i][j] * inverse);
                r = r != r ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
                val[j] = (int)r;
            }
        } else {
            // v = rint(x 2^sh), |v| <= 2^22: max < 2^e, sh = 22 - e.  A block
            // with a NaN or an infinity has xscale NaN (its dots then give
            // NaN, as the product does); an all-zero block xscale 0.
            const bool bad = top >= 0x7f800000u;
            const int sh = 22 - __builtin_amdgcn_frexp_expf(max);
            for (int j = 0; j < 4; j++) val[j] = (int)rintf(ldexpf(v[i][j], sh));
            xscale = bad ? __uint_as_float(0x7fc00000u) : (top ? ldexpf(1.0f, -sh) : 0.0f);
        }
        int sum16 = (val[0] + val[1]) + (val[2] + val[3]);
        sum16 += lane_xor1(sum16);
        sum16 += lane_xor2(sum16);
        const int other = lane_xor4(sum16);
        if (q >= quads) continue;
        int8_t *dst = planes + (size_t)m * P * span + 4 * eq;
        // Planes of v = a 2^16 + b 2^8 + c with signed bytes a, b, c: c is
        // byte 0 of v, b byte 1 of v + 2^7, a byte 2 of v + 2^15 + 2^7.
        const uint32_t sel0 = 0x0c0c0400u, sel1 = 0x04000c0cu;
        auto pack = [&](uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t shift) {
            uint32_t lo = __builtin_amdgcn_perm(w1 >> shift, w0 >> shift, sel0);
            uint32_t hi = __builtin_amdgcn_perm(w3 >> shift, w2 >> shift, sel1);
            return lo | hi;
        };
        const uint32_t c = pack(val[0], val[1], val[2], val[3], 0);
        if (P == 1) {
            *reinterpret_cast<uint32_t *>(dst) = c;
        } else {
            const uint32_t b = pack(val[0] + 128, val[1] + 128, val[2] + 128, val[3] + 128, 8);
            const uint32_t hi = pack(val[0] + 32896, val[1] + 32896, val[2] + 32896, val[3] + 32896, 16);
            *reinterpret_cast<uint32_t *>(dst) = hi;
            *reinterpret_cast<uint32_t *>(dst + span) = b;
            *reinterpret_cast<uint32_t *>(dst + 2 * span) = c;
        }
        if ((eq & 7) == 0) {
            // bytes.rs:126-128: scale * (sum of the block's q as i32) as f32.
            info[(size_t)m * (span / 32) + eq / 8] =
                float4{xscale, xscale * (float)(sum16 + other), xscale * (float)sum16, xscale * (float)other};
        }
    }
}

}  // namespace

template <class F, int P, int MT, int W, int XK>
__global__ __launch_bounds__(64 * W) void gemv_kernel(GemvArgs a) {
    constexpr int U = F::U;
    constexpr int ACC = P == 3 ? MT : 4 * MT;     // activation rows a lane sums
    constexpr int NG = F::GS == 16 ? F::STEPS : F::STEPS / 2;  // groups per unit and lane
    extern __shared__ __align__(16) uint8_t lds[];

    // Workgroup -> (group of tiles, chunk of activation rows): the row chunks
    // of a group of tiles are dispatched together and on one XCD, so that the
    // weights the first reads are still in that XCD's L2 for the others.
    const int b = blockIdx.x, local = b / XCDS;
    const int mc = local % a.mchunks;
    const int group = (local / a.mchunks) * XCDS + b % XCDS;
    if (group * a.tiles >= a.total_tiles) return;
    grid_fill<F>();
    const int m0 = mc * a.rows;
    const int rows = min(a.rows, a.rows_total - m0);
    // A route of the experts' product (one row a chunk): its expert and
    // input row.
    const uint32_t expert = a.experts ? a.experts[m0] : 0u;
    const bool bad = a.experts && expert >= a.n_experts;
    const int64_t xrow = a.experts && !a.per_route ? m0 / a.topk : m0;
    const XIn xin{static_cast<const uint8_t *>(a.x) + (size_t)xrow * a.k * (XK == X_F32 ? 4 : XK == X_H16 ? 2 : 1),
                  rows, a.k, a.x_kind};
    void *const out = static_cast<uint8_t *>(a.out) + (size_t)m0 * a.out_stride * (a.out_kind == KH_F32 ? 4 : 2);
    int32_t *const dots = a.dots ? a.dots + (size_t)m0 * a.width * (a.k / 16) : nullptr;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n16 = lane & 15;
    const int tl = wave & (a.tiles - 1), kw = wave >> a.tiles_log2;
    const int tile = group * a.tiles + tl;
    // Waves past the last tile load nothing (their offsets are NONE) and
    // write nothing.
    const bool any = tile < a.total_tiles;
    const int ltile = any ? tile : a.total_tiles - 1;
    int mat = 0;
    for (int i = 0; i < a.count; i++)
        if (ltile >= a.tile0[i] && ltile < a.tile0[i] + (int)((a.n[i] + 15) / 16)) mat = i;
    const int64_t row = (int64_t)(ltile - a.tile0[mat]) * 16 + n16;
    const bool live = any && row < (int64_t)a.n[mat];
    const uint8_t *const wbase = a.experts ? a.w[0] + (size_t)(bad ? 0u : expert) * a.wbytes[0] : a.w[mat];
    const lanes::Src src = lanes::source(wbase, a.wbytes[mat]);
    const uint32_t ro = live && !bad ? (uint32_t)row * (uint32_t)a.row_bytes : lanes::NONE;
    const uint64_t col = a.col0[mat] + (uint64_t)row;
    const int blocks32 = a.k / 32;
    auto valid = [&](int u) { return U == 256 || 4 * u + g < blocks32; };
    // Every wave issues the same loads: a unit past the chunk, or a lane past
    // K, reads at NONE (zeros, no memory access).
    auto load = [&](typename F::Regs &R, int u, int c1) {
        const bool on = u < c1 && valid(u);
        F::load(R, src, on ? ro : lanes::NONE, on ? u : 0, g);
    };
    const int span = a.chunk * U;
    using Regs = typename F::Regs;

    // LDS: planes [rows][P][span], zeros [span] (the A operand of lanes
    // outside their slice), info [rows][span / 32], sums [waves][16][rows].
    int8_t *planes = reinterpret_cast<int8_t *>(lds + 16);
    int8_t *zeros = planes + (size_t)rows * P * span;
    float4 *info = reinterpret_cast<float4 *>(zeros + span);
    float *sums = reinterpret_cast<float *>(info + (size_t)rows * (span / 32));
    for (int i = threadIdx.x; i < span / 16; i += blockDim.x)
        reinterpret_cast<v4i *>(zeros)[i] = v4i{0, 0, 0, 0};

    float acc[ACC];
#pragma unroll
    for (int i = 0; i < ACC; i++) acc[i] = 0.0f;

    // The A operand this lane supplies: row i = lane % 16 of each MFMA is
    // (plane or activation row) j = i % 4 of lane group i / 4, and only in
    // that lane group's k-slice (lane / 16); elsewhere it reads zeros.
    const int ai = lane & 15, aj = ai & 3;
    const bool a_lane = (ai >> 2) == (lane >> 4);
    int a_off[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        int m = P == 3 ? mi : 4 * mi + aj, p = P == 3 ? aj : 0;
        bool on = a_lane && p < P && m < rows;
        a_off[mi] = (on ? (m * P + p) * span : (int)(zeros - planes)) + F::xpos(g, 0);
    }
    const float4 *my_info = info + F::xpos(g, 0) / 32;

    auto process = [&](const Regs &R, int u, int c0) {
        const int ul = u - c0;
        const bool ok = valid(u);
        float sc[NG], mn[NG];
        F::scales(R, g, sc, mn);
        v4i c[MT];
#pragma unroll
        for (int s = 0; s < F::STEPS; s++) {
            v4i bw = F::codes(R, s, g);
            if (U == 128 && !ok) bw = v4i{0, 0, 0, 0};
            // Block dots in the codes of kapel-cpu/src/bytes.rs:282-353, where
            // Q6_K's are signed: stored - 32 in each byte.
            if (F::BYTES == 210 && dots)
                for (int i = 0; i < 4; i++)
                    bw[i] = (int)((((uint32_t)bw[i] | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
            if (F::GS == 16 || (s & 1) == 0)
#pragma unroll
                for (int mi = 0; mi < MT; mi++) c[mi] = v4i{0, 0, 0, 0};
            const int xo = ul * U + F::xpos(g, s) - F::xpos(g, 0);
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                v4i av = *reinterpret_cast<const v4i *>(planes + a_off[mi] + xo);
                c[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bw, c[mi], 0, 0, 0);
            }
            if (!ok || !(F::GS == 16 || (s & 1) == 1)) continue;
            // The group of this step is complete: scale it.
            const int s0 = F::GS == 16 ? s : s - 1, gi = F::GS == 16 ? s : s / 2;
            const int xs = F::xpos(g, s0) - F::xpos(g, 0);
            const int blk = (ul * U + xs) / 32;
            const bool second = ((F::xpos(g, s0) / 16) & 1) != 0;
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
#pragma unroll
                for (int j = 0; j < (P == 3 ? 1 : 4); j++) {
                    int m = P == 3 ? mi : 4 * mi + j;
                    if (m >= rows) continue;
                    if (dots) {
                        if (live)
                            dots[((uint64_t)m * a.width + col) * (a.k / 16) + (u * U + F::xpos(g, s0)) / 16] =
                                c[mi][j];
                        continue;
                    }
                    float4 in = my_info[(size_t)m * (span / 32) + blk];
                    float dot;
                    if (P == 3) dot = fmaf((float)c[mi].x, a.hi, (float)((c[mi].y << a.shift) + c[mi].z));
                    else dot = (float)c[mi][j];
                    float xsum = F::GS == 32 ? in.y : (second ? in.w : in.z);
                    float t = fmaf(dot, sc[gi] * in.x, acc[m]);
                    acc[m] = fmaf(-mn[gi], xsum, t);
                }
            }
        }
    };

    // This wave's units of a chunk: c0 + kw, c0 + kw + a.kw, ... < c1, NB of
    // them loading while the oldest is multiplied.
    constexpr int RB = sizeof(Regs) / 4;
#ifdef KH_NB
    constexpr int NB = KH_NB;
#else
    constexpr int NB = RB <= 12 ? 3 : 2;
#endif
    Regs R[NB];
    // The first `npw` waves prepare each chunk's activations, from loads
    // issued before any of their own weight loads; the other waves start
    // loading weights at once and wait (on an LDS counter, not a barrier) for
    // the activations before their first multiplication.  A barrier behind
    // weight loads would hold every wave back: once the weights stream, a
    // wave's loads wait to issue.
    const int qpc = rows * span / 4;  // quads of a chunk
    const int npw = min((int)(blockDim.x >> 6), (qpc + 64 * PASSES - 1) / (64 * PASSES));
    const bool prep = wave < npw;
    bool stalled = false;
    int *ready = reinterpret_cast<int *>(lds);
    if (threadIdx.x == 0) *ready = 0;
    __syncthreads();
    for (int c0 = 0, ci = 1; c0 < a.units; c0 += a.chunk, ci++) {
        const int c1 = min(a.units, c0 + a.chunk);
        const int step = a.kw;
        if (c0) __syncthreads();  // the previous chunk's planes are consumed
        if (prep && a.pplanes) {
            // Copy this chunk of the prepared activations, row by row.
            const int nt = 64 * npw, kb = a.k / 32;
            for (int m = 0; m < rows; m++)
                for (int p = 0; p < P; p++) {
                    const int8_t *src = a.pplanes + ((size_t)(m0 + m) * P + p) * a.pkpad;
                    int8_t *dst = planes + (size_t)(m * P + p) * span;
                    for (int w = threadIdx.x; w < span / 4; w += nt) {
                        const int e = c0 * U + 4 * w;
                        *reinterpret_cast<uint32_t *>(dst + 4 * w) =
                            e < a.k ? *reinterpret_cast<const uint32_t *>(src + e) : 0u;
                    }
                }
            for (int m = 0; m < rows; m++) {
                const size_t r = (size_t)(m0 + m);
                for (int blk = threadIdx.x; blk < span / 32; blk += nt) {
                    const int bk = c0 * U / 32 + blk;
                    info[(size_t)m * (span / 32) + blk] =
                        bk < kb ? float4{a.pxscale[r * kb + bk], a.pxsum32[r * kb + bk],
                                         a.pxsum16[r * 2 * kb + 2 * bk], a.pxsum16[r * 2 * kb + 2 * bk + 1]}
                                : float4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) __hip_atomic_fetch_add(ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else if (prep) {
            for (int q0 = 0; q0 < qpc; q0 += 64 * npw * PASSES) {
                float xv[PASSES][4];
                x_load<XK>(xin, c0 * U, span, q0, threadIdx.x, 64 * npw, xv);
                x_prepare<P, XK>(xin, span, q0, threadIdx.x, 64 * npw, xv, planes, info);
            }
            __builtin_amdgcn_wave_barrier();  // every lane's writes before the release
            if (lane == 0) __hip_atomic_fetch_add(ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
#pragma unroll
        for (int j = 0; j < NB; j++) load(R[j], c0 + kw + j * step, c1);
        // Bounded: a wait that never ended would hang the device.  A wait
        // that gives up leaves the workgroup's outputs NaN (never silently
        // wrong numbers).
        for (int spin = 0; spin < a.spin_limit; spin++) {
            if (__hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= npw * ci) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (a.spin_limit < 0 ||
            __hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < npw * ci)
            stalled = true;
        for (int base = c0 + kw; base < c1; base += NB * step) {
#pragma unroll
            for (int j = 0; j < NB; j++) {
                int u = base + j * step;
                if (u >= c1) break;
                process(R[j], u, c0);
                load(R[j], u + NB * step, c1);
            }
        }
    }
    if (dots) return;

    // The four lane groups of each row, in a fixed tree; then the waves of a
    // tile in order.
#pragma unroll
    for (int i = 0; i < ACC; i++) {
        float v = acc[i];
        v = v + __shfl_xor(v, 16);
        acc[i] = v + __shfl_xor(v, 32);
    }
    if (bad || stalled)
#pragma unroll
        for (int i = 0; i < ACC; i++) acc[i] = __uint_as_float(0x7fc00000u);
    if (a.kw == 1) {
        if (live && g == 0)
#pragma unroll
            for (int i = 0; i < ACC; i++)
                if (i < rows) store_out(a.out_kind, out, (uint64_t)i * a.out_stride + col, acc[i]);
        return;
    }
    if (g == 0)
#pragma unroll
        for (int i = 0; i < ACC; i++)
            if (i < rows) sums[((kw * a.tiles + tl) * 16 + n16) * rows + i] = acc[i];
    __syncthreads();
    if (kw == 0 && live && g == 0) {
        for (int i = 0; i < rows; i++) {
            float v = sums[(tl * 16 + n16) * rows + i];
            for (int w = 1; w < a.kw; w++) v = v + sums[((w * a.tiles + tl) * 16 + n16) * rows + i];
            store_out(a.out_kind, out, (uint64_t)i * a.out_stride + col, v);
        }
    }
}

// ---------------------------------------------------------------------------
// The decode product with its weights staged in LDS by direct loads (few
// activation rows, every matrix format the lane readers know).
//
// A workgroup takes `tiles` tiles of 16 weight rows over all of K.  Its first
// `npw` waves prepare the activations in LDS (x_load / x_prepare); the other
// `kw` waves split the units of K between them (wave c takes units c, c + kw,
// ...).  Each of those waves first copies its own units of all its tiles
// from HBM into LDS with buffer_load ... lds (16 bytes a lane, consecutive
// lanes to consecutive LDS, so every copy is coalesced and holds no
// register), tile after tile: all of a workgroup's weight bytes are in flight
// at once.  It then meets the preparing waves at a barrier and multiplies
// each tile as soon as its own copies have landed (its own vmcnt: no wave
// waits for another's loads), reading the weights from LDS through the same
// lane readers.  The sums of the waves are added in wave order by the
// preparing waves, which write the outputs.
//
// LDS of a wave's weights: [tile][unit][row of 16][CW chunks] in TB copies
// of 64 chunks; a row's unit is its block (or blocks) from the dword at or
// below its start.

// s_waitcnt vmcnt(n) for a wave-uniform n (clamped to 63: waiting for more
// than needed is safe).
__device__ __forceinline__ void wait_vm_n(int n) {
#define KH_VM(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8)); break;
    switch (n < 63 ? n : 63) {
        KH_VM(0) KH_VM(1) KH_VM(2) KH_VM(3) KH_VM(4) KH_VM(5) KH_VM(6) KH_VM(7) KH_VM(8) KH_VM(9)
        KH_VM(10) KH_VM(11) KH_VM(12) KH_VM(13) KH_VM(14) KH_VM(15) KH_VM(16) KH_VM(17) KH_VM(18) KH_VM(19)
        KH_VM(20) KH_VM(21) KH_VM(22) KH_VM(23) KH_VM(24) KH_VM(25) KH_VM(26) KH_VM(27) KH_VM(28) KH_VM(29)
        KH_VM(30) KH_VM(31) KH_VM(32) KH_VM(33) KH_VM(34) KH_VM(35) KH_VM(36) KH_VM(37) KH_VM(38) KH_VM(39)
        KH_VM(40) KH_VM(41) KH_VM(42) KH_VM(43) KH_VM(44) KH_VM(45) KH_VM(46) KH_VM(47) KH_VM(48) KH_VM(49)
        KH_VM(50) KH_VM(51) KH_VM(52) KH_VM(53) KH_VM(54) KH_VM(55) KH_VM(56) KH_VM(57) KH_VM(58) KH_VM(59)
        KH_VM(60) KH_VM(61) KH_VM(62)
        default: KH_VM(63)
    }
#undef KH_VM
}

// LDS waits and a bare barrier (a fenced __syncthreads would also wait for
// every load in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

#ifndef KH_LDS_LOAD
#define KH_LDS_LOAD(rsrc, lds, size, voff) \
    __builtin_amdgcn_raw_ptr_buffer_load_lds((rsrc), (__attribute__((address_space(3))) void *)(lds), (size), (int)(voff), 0, 0, 0)
#endif

// Bytes of a unit's copy: its block (several blocks of 32-element formats,
// one block, shared by two units, for Kapel groups of 256), and 16-byte
// chunks of it from the dword below its start.
template <class F>
struct Unit {
    static constexpr int PER = F::BLEN >= F::U ? 1 : F::U / F::BLEN;  // blocks a copy
    static constexpr int UB = PER * F::BYTES;
    static constexpr bool ODD = F::BYTES % 4 != 0;
    static constexpr int CW = (UB + (ODD ? 2 : 0) + 15) / 16;
    // The first block of unit u, and u within that block's units.
    __device__ static uint32_t block(int u) { return (uint32_t)((int64_t)u * F::U / F::BLEN); }
    __device__ static int local(int u) { return F::BLEN > F::U ? u % (F::BLEN / F::U) : 0; }
};

// A build with -DKH_TRACE (and kh_debug_trace(buffer) before a call) has
// lane 0 of every wave of the decode kernels write s_memrealtime stamps (a
// 100 MHz clock) at its phases: 32 ints a wave at (workgroup * 16 + wave) *
// 32 -- start, loads issued or activations prepared, activations ready,
// first data, multiplication done, end, HW_ID, XCC_ID, then (streamed
// kernel) data ready and done for its first twelve units.  Off by default.
#ifdef KH_TRACE
#define KH_T(i)                                                                      \
    do {                                                                              \
        if (a.trace && lane == 0) {                                                   \
            int *tr_ = a.trace + ((size_t)blockIdx.x * 16 + wave) * 32;                 \
            tr_[i] = (int)__builtin_amdgcn_s_memrealtime();                           \
            if (i == 0) {                                                             \
                unsigned hw_, xcc_;                                                   \
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw_));     \
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_));   \
                tr_[6] = (int)hw_;                                                    \
                tr_[7] = (int)xcc_;                                                   \
            }                                                                         \
        }                                                                             \
    } while (0)
#else
#define KH_T(i) do {} while (0)
#endif

template <class F, int P, int MT, int XK>
__global__ __launch_bounds__(1024) void gemv2_kernel(GemvArgs a) {
    using UN = Unit<F>;
    constexpr int U = F::U, CW = UN::CW;
    constexpr int ACC = P == 3 ? MT : 4 * MT;
    constexpr int NG = F::GS == 16 ? F::STEPS : F::STEPS / 2;
    extern __shared__ __align__(16) uint8_t lds[];

    const int group = blockIdx.x;
    const int t0 = group * a.tiles;
    if (t0 >= a.total_tiles) return;
    grid_fill<F>();
    const int T = min(a.tiles, a.total_tiles - t0);
    const int rows = a.rows;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n16 = lane & 15;
    const int span = a.units * U;
    const int TB = a.tb;
    KH_T(0);

    // LDS: planes [rows][P][span], zeros [span], info [rows][span / 32],
    // sums [kw][tiles][16][rows], weights [kw][TB KiB].
    int8_t *planes = reinterpret_cast<int8_t *>(lds + 16);
    int8_t *zeros = planes + (size_t)rows * P * span;
    float4 *info = reinterpret_cast<float4 *>(zeros + span);
    float *sums = reinterpret_cast<float *>(info + (size_t)rows * (span / 32));
    uint8_t *wl = reinterpret_cast<uint8_t *>(
        ((uintptr_t)(sums + (size_t)a.kw * a.tiles * 16 * rows) + 15) & ~(uintptr_t)15);

    // The matrix and row of a tile's row.
    auto row_of = [&](int tile, int r, int &mat) {
        mat = 0;
        for (int i = 1; i < a.count; i++)
            if (tile >= a.tile0[i]) mat = i;
        return (int64_t)(tile - a.tile0[mat]) * 16 + r;
    };

    if (wave < a.npw) {
        // ---- the activations, then (after the multiplying waves) the sums
        for (int i = threadIdx.x; i < span / 16; i += 64 * a.npw)
            reinterpret_cast<v4i *>(zeros)[i] = v4i{0, 0, 0, 0};
        const XIn xin{a.x, rows, a.k, a.x_kind};
        const int qpc = rows * span / 4;
        for (int q0 = 0; q0 < qpc; q0 += 64 * a.npw * PASSES) {
            float xv[PASSES][4];
            x_load<XK>(xin, 0, span, q0, threadIdx.x, 64 * a.npw, xv);
            x_prepare<P, XK>(xin, span, q0, threadIdx.x, 64 * a.npw, xv, planes, info);
        }
        KH_T(1);
        lds_barrier();  // the activations are ready
        KH_T(2);
        lds_barrier();  // the sums are written
        KH_T(3);
        for (int o = threadIdx.x; o < T * 16 * rows; o += 64 * a.npw) {
            const int t = o / (16 * rows), r = (o / rows) % 16, m = o % rows;
            int mat;
            const int64_t n = row_of(t0 + t, r, mat);
            if (n >= (int64_t)a.n[mat]) continue;
            float v = sums[((0 * a.tiles + t) * 16 + r) * rows + m];
            for (int c = 1; c < a.kw; c++) v = v + sums[((c * a.tiles + t) * 16 + r) * rows + m];
            store_out(a.out_kind, a.out, (uint64_t)m * a.out_stride + a.col0[mat] + (uint64_t)n, v);
        }
        KH_T(5);
        return;
    }

    // ---- a multiplying wave: copy its units of every tile, then multiply
    const int cw = wave - a.npw;
    const int upw = (a.units - cw + a.kw - 1) / a.kw;  // its units
    const int upm = (a.units + a.kw - 1) / a.kw;       // units of the wave with most
    const int tchunks = 16 * upm * CW;                  // chunks of one tile's block
    uint8_t *mine = wl + (size_t)cw * TB * 1024;
    // TB copies of 64 chunks over [tile][unit][row][CW], in order.  The
    // tiles of a workgroup lie in one matrix (the host takes several only
    // when every matrix is a whole number of them).
    int wmat;
    const int64_t row0 = row_of(t0, 0, wmat);
    const lanes::Src src = lanes::source(a.w[wmat], a.wbytes[wmat]);
    const int64_t nmat = (int64_t)a.n[wmat];
    for (int i = 0; i < TB; i++) {
        // A copy spans at most two tiles (a tile's block is over 64 chunks).
        const int ti = __builtin_amdgcn_readfirstlane(i * 64 / tchunks);
        const int ci = i * 64 + lane, t = ci >= (ti + 1) * tchunks ? ti + 1 : ti, rem = ci - t * tchunks;
        const int j = rem / (16 * CW), r = (rem / CW) % 16, c = rem % CW;
        const int64_t n = row0 + t * 16 + r;
        const int u = cw + j * a.kw;
        const bool on = t < T && j < upw && n < nmat;
        const uint32_t at = (uint32_t)n * (uint32_t)a.row_bytes + UN::block(u) * F::BYTES;
        KH_LDS_LOAD(src.r, mine + i * 1024, 16, on ? (at & ~3u) + 16u * c : lanes::NONE);
    }
    KH_T(1);
    lds_barrier();  // the activations are ready
    KH_T(2);

    // The A operand of this lane: row i = lane % 16 of each MFMA is (plane
    // or activation row) j = i % 4 of lane group i / 4, in that lane group's
    // k-slice only; elsewhere it reads zeros.
    const int ai = lane & 15, aj = ai & 3;
    const bool a_lane = (ai >> 2) == (lane >> 4);
    int a_off[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        int m = P == 3 ? mi : 4 * mi + aj, p = P == 3 ? aj : 0;
        bool on = a_lane && p < P && m < rows;
        a_off[mi] = (on ? (m * P + p) * span : (int)(zeros - planes)) + F::xpos(g, 0);
    }
    const float4 *my_info = info + F::xpos(g, 0) / 32;
    const int blocks32 = a.k / 32;

    // One unit of one tile into acc.
    auto unit = [&](int t, int jj, float (&acc)[ACC]) __attribute__((always_inline)) {
        int mat;
        const int64_t n = row_of(t0 + t, n16, mat);
        const int u = cw + jj * a.kw;
        const bool ok = U == 256 || 4 * u + g < blocks32;
        const uint32_t at = (uint32_t)n * (uint32_t)a.row_bytes + UN::block(u) * F::BYTES;
        typename F::Regs R;
        F::load(R, lanes::LdsSrc{mine}, (uint32_t)((t * tchunks + (jj * 16 + n16) * CW) * 16) + (at & 3u),
                UN::local(u), g);
        float sc[NG], mn[NG];
        F::scales(R, g, sc, mn);
        v4i c[MT];
#pragma unroll
        for (int s = 0; s < F::STEPS; s++) {
            v4i bw = F::codes(R, s, g);
            if (U == 128 && !ok) bw = v4i{0, 0, 0, 0};
            if (F::GS == 16 || (s & 1) == 0)
#pragma unroll
                for (int mi = 0; mi < MT; mi++) c[mi] = v4i{0, 0, 0, 0};
            const int xo = u * U + F::xpos(g, s) - F::xpos(g, 0);
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                v4i av = *reinterpret_cast<const v4i *>(planes + a_off[mi] + xo);
                c[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bw, c[mi], 0, 0, 0);
            }
            if (!(F::GS == 16 || (s & 1) == 1)) continue;
            // The group of this step is complete: scale it (nothing past K).
            const int s0 = F::GS == 16 ? s : s - 1, gi = F::GS == 16 ? s : s / 2;
            const int blk = (u * U + F::xpos(g, s0) - F::xpos(g, 0)) / 32;
            const bool second = ((F::xpos(g, s0) / 16) & 1) != 0;
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
#pragma unroll
                for (int j = 0; j < (P == 3 ? 1 : 4); j++) {
                    int m = P == 3 ? mi : 4 * mi + j;
                    if (m >= rows) continue;
                    float4 in = my_info[(size_t)m * (span / 32) + (ok ? blk : 0)];
                    float dot;
                    if (P == 3) dot = fmaf((float)c[mi].x, a.hi, (float)((c[mi].y << a.shift) + c[mi].z));
                    else dot = (float)c[mi][j];
                    float xsum = F::GS == 32 ? in.y : (second ? in.w : in.z);
                    float tt = fmaf(dot, sc[gi] * in.x, acc[m]);
                    tt = fmaf(-mn[gi], xsum, tt);
                    acc[m] = ok ? tt : acc[m];
                }
            }
        }
    };
    // The four lane groups of each row in a fixed tree, then to LDS.
    auto finish = [&](int t, float (&acc)[ACC]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < ACC; i++) {
            float v = acc[i];
            v = v + __shfl_xor(v, 16);
            acc[i] = v + __shfl_xor(v, 32);
        }
        if (g == 0)
#pragma unroll
            for (int i = 0; i < ACC; i++)
                if (i < rows) sums[((cw * a.tiles + t) * 16 + n16) * rows + i] = acc[i];
    };
    // Units two at a time, so that their LDS reads and MFMAs overlap: pairs
    // of units of a tile (then their sums added), or, with one unit a wave,
    // pairs of tiles.
    if (upw >= 2) {
        for (int t = 0; t < T; t++) {
            // This tile's copies are the first ceil((t + 1) tchunks / 64).
            wait_vm_n(TB - (((t + 1) * tchunks + 63) >> 6));
            if (t == 0) KH_T(3);
            float acc[ACC], acc2[ACC];
#pragma unroll
            for (int i = 0; i < ACC; i++) acc[i] = acc2[i] = 0.0f;
            int jj = 0;
            for (; jj + 1 < upw; jj += 2) {
                unit(t, jj, acc);
                unit(t, jj + 1, acc2);
            }
            if (jj < upw) unit(t, jj, acc);
#pragma unroll
            for (int i = 0; i < ACC; i++) acc[i] = acc[i] + acc2[i];
            finish(t, acc);
        }
    } else if (upw == 1) {
        int t = 0;
        for (; t + 1 < T; t += 2) {
            wait_vm_n(TB - (((t + 2) * tchunks + 63) >> 6));
            if (t == 0) KH_T(3);
            float acc[ACC], acc2[ACC];
#pragma unroll
            for (int i = 0; i < ACC; i++) acc[i] = acc2[i] = 0.0f;
            unit(t, 0, acc);
            unit(t + 1, 0, acc2);
            finish(t, acc);
            finish(t + 1, acc2);
        }
        if (t < T) {
            wait_vm_n(TB - (((t + 1) * tchunks + 63) >> 6));
            float acc[ACC];
#pragma unroll
            for (int i = 0; i < ACC; i++) acc[i] = 0.0f;
            unit(t, 0, acc);
            finish(t, acc);
        }
    } else {
        // No unit for this wave (more waves than units): zero sums.
        for (int t = 0; t < T; t++) {
            float acc[ACC];
#pragma unroll
            for (int i = 0; i < ACC; i++) acc[i] = 0.0f;
            finish(t, acc);
        }
    }
    KH_T(4);
    wait_vm_n(0);
    lds_barrier();  // the sums are written
    KH_T(5);
}

}  // namespace kh
#include "kh_gemv4.h"
namespace kh {

namespace {

template <class F, int P, int MT, int XK>
hipError_t launch4(const GemvArgs &a, hipStream_t s, size_t lds) {
    static OncePerDevice once;
    hipError_t e = set_lds_limit(once, reinterpret_cast<const void *>(&gemv4_kernel<F, P, MT, XK>),
                                 160 * 1024 - grid_lds<F>());
    if (e != hipSuccess) return e;
    const int threads = 64 * (a.npw + a.tiles * a.kw);
    const bool walk = a.kw == 1 && a.count == 1;
    // Workgroups a CU holds at once (registers, waves, LDS), from the runtime.
    int per_cu = 0;
    if ((walk || a.occupancy) &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&gemv4_kernel<F, P, MT, XK>),
                                                     threads, lds) != hipSuccess)
        per_cu = 0;
    if (a.occupancy) {
        *a.occupancy = per_cu;
        return hipSuccess;
    }
    int groups = (a.total_tiles + a.tiles - 1) / a.tiles;
    if (walk) {
        // Each wave walks its tiles: as many workgroups as are resident at once.
        if (per_cu < 1)
            per_cu = std::max(1, std::min((int)((160 * 1024) / std::max<size_t>(lds, 1)), 32 / (a.npw + a.tiles)));
        groups = std::min(groups, cu_count() * per_cu);
    }
    hipLaunchKernelGGL((gemv4_kernel<F, P, MT, XK>), dim3((unsigned)groups), dim3(threads), lds, s, a);
    return hipGetLastError();
}

template <class F, int P, int MT, int XK>
hipError_t launch2(const GemvArgs &a, hipStream_t s, size_t lds) {
    static OncePerDevice once;
    hipError_t e = set_lds_limit(once, reinterpret_cast<const void *>(&gemv2_kernel<F, P, MT, XK>),
                                 160 * 1024 - grid_lds<F>());
    if (e != hipSuccess) return e;
    const int groups = (a.total_tiles + a.tiles - 1) / a.tiles;
    hipLaunchKernelGGL((gemv2_kernel<F, P, MT, XK>), dim3((unsigned)groups), dim3(64 * (a.npw + a.kw)), lds, s, a);
    return hipGetLastError();
}

template <class F, int P, int XK>
hipError_t launch_fx(const GemvArgs &a, hipStream_t s) {
    int mt = P == 3 ? a.rows : (a.rows + 3) / 4;
    if (a.dma == 4) {
        // Host-side checks of what the kernel assumes: its waves, a ring
        // that holds the whole stream or whole units (at least two: a copy
        // never overwrites the unit being multiplied) in whole copies.  A
        // wave that walks several tiles has a stream longer than one tile's:
        // its ring must be whole units (a unit's chunks never wrap).
        constexpr int UC = 16 * Unit<F>::CW;
        const int upw = (a.units + a.kw - 1) / a.kw;
        const int whole = (upw * UC + 63) / 64;
        const bool walk = a.kw == 1 && a.count == 1;
        const bool ring_ok = (a.tb * 64) % UC == 0 ? a.tb >= whole || a.tb * 64 >= 2 * UC
                                                    : !walk && a.tb >= whole;
        const size_t lds = gemv4_lds(a.rows, P, a.units, F::U, a.tiles, a.kw, a.tb);
        if (a.npw < 1 || a.tiles < 1 || a.kw < 1 || a.npw + a.tiles * a.kw > 16 || a.tb < 1 || !ring_ok ||
            lds > (size_t)(160 * 1024 - grid_lds<F>()) || mt > 1)
            return hipErrorInvalidValue;
        return launch4<F, P, 1, XK>(a, s, lds);
    }
    if (a.dma) {
        if (a.tb * 64 < a.tiles * 16 * Unit<F>::CW * ((a.units + a.kw - 1) / a.kw) || a.npw + a.kw > 16)
            return hipErrorInvalidValue;
        size_t lds = gemv2_lds(a.rows, P, a.units, F::U, a.tiles, a.kw, a.tb);
        if (lds > (size_t)(160 * 1024 - grid_lds<F>())) return hipErrorInvalidValue;
        if (mt <= 1) return launch2<F, P, 1, XK>(a, s, lds);
        return hipErrorInvalidValue;
    }
    int waves = a.tiles * a.kw;
    size_t lds = gemv_lds(a.rows, P, a.chunk, F::U, waves);
    const int groups = (a.total_tiles + a.tiles - 1) / a.tiles;
    dim3 grid((unsigned)((groups + XCDS - 1) / XCDS * XCDS * a.mchunks)), block(64 * waves);
    if (waves < 1 || waves > gemv_max_waves(P, a.rows) || lds > 65536) return hipErrorInvalidValue;
    if (mt <= 1) hipLaunchKernelGGL((gemv_kernel<F, P, 1, P == 3 ? 16 : 8, XK>), grid, block, lds, s, a);
    else if (mt <= 2) hipLaunchKernelGGL((gemv_kernel<F, P, 2, 8, XK>), grid, block, lds, s, a);
    else if (mt <= 4) hipLaunchKernelGGL((gemv_kernel<F, P, 4, 8, XK>), grid, block, lds, s, a);
    else if constexpr (P == 3) {
        if (mt <= 8) hipLaunchKernelGGL((gemv_kernel<F, 3, 8, 8, XK>), grid, block, lds, s, a);
        else return hipErrorInvalidValue;
    } else return hipErrorInvalidValue;
    return hipGetLastError();
}

// The kernels of a format: f32 and 16-bit activations, and (bytes) int8.
template <class F, int P>
hipError_t launch_f(const GemvArgs &a, hipStream_t s) {
    if (a.x_kind == KH_F32) return launch_fx<F, P, X_F32>(a, s);
    if (a.x_kind == KH_BF16 || a.x_kind == KH_F16) return launch_fx<F, P, X_H16>(a, s);
    if constexpr (P == 1)
        if (a.x_kind == KH_I8_INTERNAL) return launch_fx<F, 1, X_I8>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

}  // namespace kh
