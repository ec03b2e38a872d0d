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
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_internal.h"
#include "kh_lanes.h"

namespace kh {
namespace {

using lanes::v4i;

constexpr int MAX_PASSES = 8;  // quads of activations per thread in step 2

__device__ __forceinline__ float x_at(uint32_t kind, const void *x, uint64_t i) {
    if (kind == KH_F32) return static_cast<const float *>(x)[i];
    if (kind == KH_I8_INTERNAL) return (float)static_cast<const int8_t *>(x)[i];
    uint32_t h = static_cast<const uint16_t *>(x)[i];
    if (kind == KH_BF16) return __uint_as_float(h << 16);
    return __half2float(__ushort_as_half((uint16_t)h));
}

// Four consecutive activations (i % 4 == 0); `vec`: x is 16-byte (f32) or
// 8-byte (16-bit types) aligned.
__device__ __forceinline__ void x4(uint32_t kind, const void *x, uint64_t i, bool vec, float (&v)[4]) {
    if (vec && kind == KH_F32) {
        float4 f = *reinterpret_cast<const float4 *>(static_cast<const float *>(x) + i);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else if (vec) {
        uint2 h = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(x) + i);
        uint32_t hs[4] = {h.x & 0xffffu, h.x >> 16, h.y & 0xffffu, h.y >> 16};
        for (int j = 0; j < 4; j++)
            v[j] = kind == KH_BF16 ? __uint_as_float(hs[j] << 16)
                                   : __half2float(__ushort_as_half((uint16_t)hs[j]));
    } else {
        for (int j = 0; j < 4; j++) v[j] = x_at(kind, x, i + j);
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

// Step 2: the chunk's activations into LDS.  Thread t takes quads (4
// elements) t, t + 256, ...; eight consecutive threads hold a block of 32.
// planes: [rows][P][span] int8; info: [rows][span / 32] of {xscale, xsum32,
// xsum16 (first half), xsum16 (second half)}, xsum = xscale * the integer sum
// of the block's (or half's) values.
template <int P>
__device__ void prepare(const GemvArgs &a, int e0, int span, int8_t *planes, float4 *info) {
    const int quads_per_row = span / 4;
    const int quads = a.rows * quads_per_row;
    float v[MAX_PASSES][4];
#pragma unroll
    for (int i = 0; i < MAX_PASSES; i++) {
        int q = threadIdx.x + 256 * i;
        int m = q / quads_per_row, e = e0 + 4 * (q % quads_per_row);
        if (q < quads && e < a.k) x4(a.x_kind, a.x, (uint64_t)m * a.k + e, a.x_vec, v[i]);
        else v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < MAX_PASSES; i++) {
        if (256 * i >= quads) break;  // uniform
        int q = threadIdx.x + 256 * i;
        bool live = q < quads;
        int m = q / quads_per_row, eq = q % quads_per_row;
        // f32::max ignores NaN, as fmaxf does (bytes.rs:148-151).
        float max = fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3])));
        for (int s = 1; s < 8; s <<= 1) max = fmaxf(max, __shfl_xor(max, s));
        int val[4];
        float xscale;
        if (P == 1 && a.x_kind == KH_I8_INTERNAL) {
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
            int bad = 0;
            for (int j = 0; j < 4; j++) bad |= v[i][j] != v[i][j];
            bad |= !isfinite(max);
            for (int s = 1; s < 8; s <<= 1) bad |= __shfl_xor(bad, s);
            int exponent = 0;
            bool scaled = max > 0.0f && !bad;
            if (scaled) frexpf(max, &exponent);  // max < 2^exponent
            int sh = 22 - exponent;
            for (int j = 0; j < 4; j++) val[j] = scaled ? (int)rintf(ldexpf(v[i][j], sh)) : 0;
            xscale = bad ? __uint_as_float(0x7fc00000u) : (scaled ? ldexpf(1.0f, -sh) : 0.0f);
        }
        int sum16 = (val[0] + val[1]) + (val[2] + val[3]);
        sum16 += __shfl_xor(sum16, 1);
        sum16 += __shfl_xor(sum16, 2);
        int other = __shfl_xor(sum16, 4);
        if (!live) continue;
        int8_t *dst = planes + (size_t)m * P * span + 4 * eq;
        if (P == 1) {
            *reinterpret_cast<uint32_t *>(dst) = pack_bytes(val[0], val[1], val[2], val[3]);
        } else {
            int r1[4], r0[4];
            for (int j = 0; j < 4; j++) {
                r1[j] = (val[j] + 128) >> 8;
                r0[j] = (r1[j] + 128) >> 8;
            }
            *reinterpret_cast<uint32_t *>(dst) = pack_bytes(r0[0], r0[1], r0[2], r0[3]);
            *reinterpret_cast<uint32_t *>(dst + span) = pack_bytes(r1[0], r1[1], r1[2], r1[3]);
            *reinterpret_cast<uint32_t *>(dst + 2 * span) = pack_bytes(val[0], val[1], val[2], val[3]);
        }
        if ((eq & 7) == 0) {
            // bytes.rs:126-128: scale * (sum of the block's q as i32) as f32.
            info[(size_t)m * (span / 32) + eq / 8] =
                float4{xscale, xscale * (float)(sum16 + other), xscale * (float)sum16, xscale * (float)other};
        }
    }
}

}  // namespace

template <class F, int P, int MT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    constexpr int U = F::U;
    constexpr int ACC = P == 3 ? MT : 4 * MT;  // activation rows a lane sums
    constexpr int PD = 2;                      // units in flight per batch
    extern __shared__ __align__(16) uint8_t lds[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, n16 = lane & 15;
    const int tl = wave % a.tiles, kw = wave / a.tiles;
    const int tile = blockIdx.x * a.tiles + tl;
    int mat = -1;
    for (int i = 0; i < a.count; i++)
        if (tile >= a.tile0[i] && tile < a.tile0[i] + (int)((a.n[i] + 15) / 16)) mat = i;
    int64_t row = 0;
    bool live = false;
    const uint8_t *rowp = nullptr;
    uint64_t col = 0;
    if (mat >= 0) {
        row = (int64_t)(tile - a.tile0[mat]) * 16 + n16;
        live = row < (int64_t)a.n[mat];
        rowp = a.w[mat] + (live ? row : (int64_t)a.n[mat] - 1) * (int64_t)a.row_bytes;
        col = a.col0[mat] + (uint64_t)row;
    }
    const int blocks32 = a.k / 32;
    auto valid = [&](int u) { return U == 256 || 4 * u + g < blocks32; };
    const int span = a.chunk * U;

    using Regs = typename F::Regs;
    Regs A[PD], B[PD];
    // This wave's units of a chunk: c0 + kw, c0 + kw + a.kw, ... < c1.
    auto load = [&](Regs(&R)[PD], int ub, int c1) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
            int u = ub + j * a.kw;
            if (u < c1 && valid(u)) F::load(R[j], rowp, u, g);
        }
    };

    int8_t *planes = reinterpret_cast<int8_t *>(lds + 16);
    float4 *info = reinterpret_cast<float4 *>(lds + 16 + (size_t)a.rows * P * span);
    float *sums = reinterpret_cast<float *>(lds + 16 + (size_t)a.rows * P * span +
                                            (size_t)a.rows * (span / 32) * 16);

    float acc[ACC];
#pragma unroll
    for (int i = 0; i < ACC; i++) acc[i] = 0.0f;

    // The A operand this lane supplies: row i = lane % 16 of each MFMA is
    // (plane or activation row) j = i % 4 of lane group i / 4, and only in
    // that lane group's k-slice (lane / 16).
    const int ai = lane & 15, aj = ai & 3;
    const bool a_lane = (ai >> 2) == (lane >> 4);
    int a_off[MT];
    bool a_on[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        int m = P == 3 ? mi : 4 * mi + aj, p = P == 3 ? aj : 0;
        a_on[mi] = a_lane && p < P && m < a.rows;
        a_off[mi] = (m * P + p) * span;
    }

    auto apply = [&](const Regs &R, const v4i (&c)[MT], int ul, int u, int s0) {
        float sc, mn;
        F::scale(R, g, s0, sc, mn);
        const int xs = F::xpos(g, s0);
        const int blk = (ul * U + xs) / 32;
        const bool second = (xs / 16) & 1;
#pragma unroll
        for (int mi = 0; mi < MT; mi++) {
#pragma unroll
            for (int j = 0; j < (P == 3 ? 1 : 4); j++) {
                int m = P == 3 ? mi : 4 * mi + j;
                if (m >= a.rows) continue;
                if (a.dots) {
                    if (live) a.dots[((uint64_t)m * a.width + col) * (a.k / 16) + (u * U + xs) / 16] = c[mi][j];
                    continue;
                }
                float4 in = info[(size_t)m * (span / 32) + blk];
                float dot;
                if (P == 3) dot = (float)c[mi].x * 65536.0f + (float)(c[mi].y * 256 + c[mi].z);
                else dot = (float)c[mi][j];
                float xsum = F::GS == 32 ? in.y : (second ? in.w : in.z);
                float t = fmaf(dot, sc * in.x, acc[P == 3 ? mi : 4 * mi + j]);
                acc[P == 3 ? mi : 4 * mi + j] = fmaf(-mn, xsum, t);
            }
        }
    };

    auto process = [&](const Regs &R, int u, int c0) {
        const int ul = u - c0;
        const bool ok = valid(u);
        v4i c[MT];
#pragma unroll
        for (int s = 0; s < F::STEPS; s++) {
            v4i bw = F::codes(R, s, g);
            if (U == 128 && !ok) bw = v4i{0, 0, 0, 0};
            // Block dots in the codes of kapel-cpu/src/bytes.rs:282-353, where
            // Q6_K's are signed: stored - 32 in each byte.
            if (F::BYTES == 210 && a.dots)
                for (int i = 0; i < 4; i++)
                    bw[i] = (int)((((uint32_t)bw[i] | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
            if (F::GS == 16 || (s & 1) == 0)
#pragma unroll
                for (int mi = 0; mi < MT; mi++) c[mi] = v4i{0, 0, 0, 0};
            const int xo = ul * U + F::xpos(g, s);
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                v4i av = v4i{0, 0, 0, 0};
                if (a_on[mi]) av = *reinterpret_cast<const v4i *>(planes + a_off[mi] + xo);
                c[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bw, c[mi], 0, 0, 0);
            }
            if (ok && (F::GS == 16 || (s & 1) == 1)) apply(R, c, ul, u, F::GS == 16 ? s : s - 1);
        }
    };

    for (int c0 = 0; c0 < a.units; c0 += a.chunk) {
        const int c1 = min(a.units, c0 + a.chunk);
        const int step = PD * a.kw;
        if (mat >= 0) load(A, c0 + kw, c1);
        if (c0) __syncthreads();  // the previous chunk's planes are consumed
        prepare<P>(a, c0 * U, span, planes, info);
        __syncthreads();
        if (mat >= 0) {
            for (int ub = c0 + kw; ub < c1; ub += 2 * step) {
                load(B, ub + step, c1);
#pragma unroll
                for (int j = 0; j < PD; j++)
                    if (ub + j * a.kw < c1) process(A[j], ub + j * a.kw, c0);
                if (ub + step >= c1) break;
                load(A, ub + 2 * step, c1);
#pragma unroll
                for (int j = 0; j < PD; j++)
                    if (ub + step + j * a.kw < c1) process(B[j], ub + step + j * a.kw, c0);
            }
        }
    }
    if (a.dots) return;

    // The four lane groups of each row, in a fixed tree; then the waves of a
    // tile in order.
#pragma unroll
    for (int i = 0; i < ACC; i++) {
        float v = acc[i];
        v = v + __shfl_xor(v, 16);
        acc[i] = v + __shfl_xor(v, 32);
    }
    if (a.kw == 1) {
        if (live && g == 0)
#pragma unroll
            for (int i = 0; i < ACC; i++)
                if (i < a.rows) store_out(a.out_kind, a.out, (uint64_t)i * a.out_stride + col, acc[i]);
        return;
    }
    // sums: [kw][tiles][16][rows]
    if (g == 0)
#pragma unroll
        for (int i = 0; i < ACC; i++)
            if (i < a.rows) sums[((kw * a.tiles + tl) * 16 + n16) * a.rows + i] = acc[i];
    __syncthreads();
    if (kw == 0 && live && g == 0) {
        for (int i = 0; i < a.rows; i++) {
            float v = sums[(tl * 16 + n16) * a.rows + i];
            for (int w = 1; w < a.kw; w++) v = v + sums[((w * a.tiles + tl) * 16 + n16) * a.rows + i];
            store_out(a.out_kind, a.out, (uint64_t)i * a.out_stride + col, v);
        }
    }
}

namespace {

template <class F, int P>
hipError_t launch_f(const GemvArgs &a, hipStream_t s) {
    int mt = P == 3 ? a.rows : (a.rows + 3) / 4;
    int waves = a.tiles * a.kw;
    size_t lds = gemv_lds(a.rows, P, a.chunk, F::U, waves);
    dim3 grid((unsigned)((a.total_tiles + a.tiles - 1) / a.tiles)), block(64 * waves);
    if (waves != 4) return hipErrorInvalidValue;
    if (mt <= 1) hipLaunchKernelGGL((gemv_kernel<F, P, 1>), grid, block, lds, s, a);
    else if (mt <= 2) hipLaunchKernelGGL((gemv_kernel<F, P, 2>), grid, block, lds, s, a);
    else if (mt <= 4) hipLaunchKernelGGL((gemv_kernel<F, P, 4>), grid, block, lds, s, a);
    else if (P == 3 && mt <= 8) hipLaunchKernelGGL((gemv_kernel<F, 3, 8>), grid, block, lds, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

int gemv_unit(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K: return 256;
    case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0: return 128;
    case KH_INT8: case KH_INT4:
        return (group == 32 || group == 64 || group == 128 || group == 256) ? 128 : 0;
    default: return 0;
    }
}

size_t gemv_lds(int rows, int planes, int chunk, int unit, int waves) {
    size_t span = (size_t)chunk * unit;
    return 16 + (size_t)rows * planes * span + (size_t)rows * (span / 32) * 16 +
           (size_t)waves * 16 * rows * 4;
}

hipError_t launch_gemv(uint32_t fmt, uint32_t group, int planes, const GemvArgs &a, hipStream_t s) {
    using namespace lanes;
    if (planes == 1) {
        switch (fmt) {
        case KH_Q4K: return launch_f<Q4K, 1>(a, s);
        case KH_Q5K: return launch_f<Q5K, 1>(a, s);
        case KH_Q6K: return launch_f<Q6K, 1>(a, s);
        case KH_Q4_0: return launch_f<Q4_0, 1>(a, s);
        case KH_Q8_0: return launch_f<Q8_0, 1>(a, s);
        case KH_INT8:
            if (group == 32) return launch_f<Int8G<32>, 1>(a, s);
            if (group == 64) return launch_f<Int8G<64>, 1>(a, s);
            if (group == 128) return launch_f<Int8G<128>, 1>(a, s);
            break;
        case KH_INT4:
            if (group == 32) return launch_f<Int4G<32>, 1>(a, s);
            if (group == 64) return launch_f<Int4G<64>, 1>(a, s);
            if (group == 128) return launch_f<Int4G<128>, 1>(a, s);
            break;
        }
        return hipErrorInvalidValue;
    }
    switch (fmt) {
    case KH_Q4K: return launch_f<Q4K, 3>(a, s);
    case KH_Q5K: return launch_f<Q5K, 3>(a, s);
    case KH_Q6K: return launch_f<Q6K, 3>(a, s);
    case KH_Q2K: return launch_f<Q2K, 3>(a, s);
    case KH_Q3K: return launch_f<Q3K, 3>(a, s);
    case KH_Q4_0: return launch_f<Q4_0, 3>(a, s);
    case KH_Q4_1: return launch_f<Q4_1, 3>(a, s);
    case KH_Q5_0: return launch_f<Q5_0, 3>(a, s);
    case KH_Q5_1: return launch_f<Q5_1, 3>(a, s);
    case KH_Q8_0: return launch_f<Q8_0, 3>(a, s);
    case KH_INT8:
        if (group == 32) return launch_f<Int8G<32>, 3>(a, s);
        if (group == 64) return launch_f<Int8G<64>, 3>(a, s);
        if (group == 128) return launch_f<Int8G<128>, 3>(a, s);
        if (group == 256) return launch_f<Int8G<256>, 3>(a, s);
        break;
    case KH_INT4:
        if (group == 32) return launch_f<Int4G<32>, 3>(a, s);
        if (group == 64) return launch_f<Int4G<64>, 3>(a, s);
        if (group == 128) return launch_f<Int4G<128>, 3>(a, s);
        if (group == 256) return launch_f<Int4G<256>, 3>(a, s);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
