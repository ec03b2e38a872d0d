// libkapel_hip: Kapel's product by quantized weights on MI355X (gfx950).
//
// One pipeline serves every format and every number of activation rows:
//
//  1. prep_x: the activations, by blocks of 32, become int8 "planes" in the
//     workspace.  With byte activations (kapel-cpu/src/bytes.rs:144-158) the
//     one plane is the CPU's q and the block scale its s.  With f32
//     activations, each block is a 23-bit fixed-point number x * 2^sh
//     (sh = 22 - exponent of the block's largest magnitude), split into three
//     signed bytes (planes) a * 2^16 + b * 2^8 + c: the integer dots of the
//     three planes recompose the dot, and the representation error is below
//     2^-23 of the block's largest value.
//
//  2. qmv: each wave takes 16 weight rows and a segment of K.  Per step of 64
//     elements it unpacks the weights' codes in registers into bytes (the B
//     operand) and multiplies them by the activation planes (A operand, read
//     from LDS) with v_mfma_i32_16x16x64_i8: exact i32 dots per group of 16 or
//     32 weights, which are then scaled: out += scale * xscale * dot -
//     minimum * sum(x).  A segment split of K (fixed by the shapes alone) is
//     reduced by the last workgroup of each row range to arrive, in segment
//     order: the bits do not depend on timing or on the number of CUs.
//
// Layouts of the formats: kh_formats.h.  Shapes and refusals: kh_api.cpp.
#include <hip/hip_fp16.h>
#include <algorithm>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_formats.h"
#include "kh_iq.h"
#include "kh_internal.h"

namespace kh {

// ------------------------------------------------------------------ floats
__device__ __forceinline__ float load_x(uint32_t kind, const void *x, uint64_t i) {
    if (kind == KH_F32) return static_cast<const float *>(x)[i];
    uint32_t h = static_cast<const uint16_t *>(x)[i];
    if (kind == KH_BF16) return __uint_as_float(h << 16);
    return h2f(h);
}

// f32 to bf16 / f16, round to nearest even.
__device__ __forceinline__ uint16_t to_bf16(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ uint16_t to_f16(float v) {
    return __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ void store_out(uint32_t kind, void *out, uint64_t i, float v) {
    if (kind == KH_F32) static_cast<float *>(out)[i] = v;
    else if (kind == KH_BF16) static_cast<uint16_t *>(out)[i] = to_bf16(v);
    else static_cast<uint16_t *>(out)[i] = to_f16(v);
}

// --------------------------------------------------------------- prep_x
// Eight consecutive elements a thread, four threads (consecutive lanes) a
// block of 32.  Writes the planes [rows][planes][kpad], xscale [rows][k/32],
// the sums of each group of 16 and 32 as floats (x's value: xsum = xscale *
// sum of the plane values) and of 16 as integers.
constexpr int PREP_E = 8;

__device__ __forceinline__ void load8(uint32_t kind, const void *x, uint64_t e, bool vec, float (&v)[PREP_E]) {
    if (vec && kind == KH_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + e);
        float4 a = p[0], b = p[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else if (vec) {
        uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + e);
        uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = d[i] & 0xffffu, hi = d[i] >> 16;
            v[2 * i] = kind == KH_BF16 ? __uint_as_float(lo << 16) : h2f(lo);
            v[2 * i + 1] = kind == KH_BF16 ? __uint_as_float(hi << 16) : h2f(hi);
        }
    } else {
#pragma unroll
        for (int i = 0; i < PREP_E; i++) v[i] = load_x(kind, x, e + i);
    }
}

__global__ __launch_bounds__(256) void prep_x_kernel(PrepArgs a) {
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t total = a.rows * a.k / PREP_E;
    const bool live = t < total;
    const uint64_t e = live ? t * PREP_E : 0;
    const uint64_t m = e / a.k, col = e % a.k;
    // Vector loads when x allows them (rows start at multiples of 32
    // elements).
    const bool vec = ((uintptr_t)a.x & 15u) == 0;
    float v[PREP_E];
    if (a.q_in || !live) {
#pragma unroll
        for (int i = 0; i < PREP_E; i++) v[i] = 0.0f;
    } else {
        load8(a.x_kind, a.x, e, vec, v);
    }
    float mag[PREP_E], max = 0.0f;
#pragma unroll
    for (int i = 0; i < PREP_E; i++) {
        mag[i] = fabsf(v[i]);
        // f32::max ignores NaN, as fmaxf does: bytes.rs:148-151.
        max = fmaxf(max, mag[i]);
    }
    max = fmaxf(max, __shfl_xor(max, 1));
    max = fmaxf(max, __shfl_xor(max, 2));
    int value[PREP_E];  // the integers these elements stand for: q, or x * 2^sh
    int digit[3][PREP_E];
    float xscale;      // their weight: element = xscale * value
    if (a.q_in) {
        // Bytes given (kh_block_dots): only their sums are wanted.
        xscale = 1.0f;
#pragma unroll
        for (int i = 0; i < PREP_E; i++) value[i] = digit[0][i] = live ? (int)a.q_in[e + i] : 0;
    } else if (a.planes == 1) {
        // bytes.rs:152-156: s = max / 127 (correctly rounded division),
        // q = round-half-even(x * (127 / max)) clamped to +-127; NaN -> 0.
        xscale = max / 127.0f;
        const float inverse = max > 0.0f ? 127.0f / max : 0.0f;
#pragma unroll
        for (int i = 0; i < PREP_E; i++) {
            float r = rintf(v[i] * inverse);
            r = r != r ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
            value[i] = digit[0][i] = (int)r;
        }
    } else {
        // 23-bit fixed point against the block's largest magnitude, in three
        // signed bytes: value = d0 * 2^16 + d1 * 2^8 + d2, |value| <= 2^22,
        // |d0| <= 64.
        const bool finite = isfinite(max);
        int exponent = 0;
        if (max > 0.0f && finite) frexpf(max, &exponent);  // max < 2^exponent
        const int sh = 22 - exponent;
        int bad = 0;
#pragma unroll
        for (int i = 0; i < PREP_E; i++) {
            const float f = (max > 0.0f && finite) ? rintf(__builtin_ldexpf(v[i], sh)) : 0.0f;
            value[i] = f != f ? 0 : (int)f;
            const int c = ((value[i] + 128) & 255) - 128;
            const int r1 = (value[i] - c) >> 8;
            const int b = ((r1 + 128) & 255) - 128;
            digit[0][i] = (r1 - b) >> 8;
            digit[1][i] = b;
            digit[2][i] = c;
            bad |= (!finite || mag[i] != mag[i]) ? 1 : 0;
        }
        // A block holding a NaN or an infinity gives NaN, as the product does.
        bad |= __shfl_xor(bad, 1);
        bad |= __shfl_xor(bad, 2);
        xscale = bad ? __uint_as_float(0x7fc00000u) : (max > 0.0f ? __builtin_ldexpf(1.0f, -sh) : 0.0f);
    }
    int v8 = 0;
#pragma unroll
    for (int i = 0; i < PREP_E; i++) v8 += value[i];
    const int v16 = v8 + __shfl_xor(v8, 1);
    const int other = __shfl_xor(v16, 2);
    if (!live) return;
    const int quarter = (int)(col % 32) / PREP_E;
    const uint64_t blk32 = m * (a.k / 32) + col / 32;
    const uint64_t g16 = m * (a.k / 16) + col / 16;
    if ((quarter & 1) == 0) {
        if (a.xsumi16) a.xsumi16[g16] = v16;
        if (a.xsum16) a.xsum16[g16] = xscale * (float)v16;
    }
    if (quarter == 0) {
        // bytes.rs:126-128: scale * (sum of the block's q as i32) as f32.
        const float sum32 = xscale * (float)(v16 + other);
        if (a.xscale) a.xscale[blk32] = xscale;
        if (a.xsum32) a.xsum32[blk32] = sum32;
        if (a.q_scale) a.q_scale[blk32] = xscale;
        if (a.q_sums) a.q_sums[blk32] = sum32;
    }
    auto pack = [&](const int (&d)[PREP_E]) {
        uint2 w;
        w.x = (uint32_t)(d[0] & 0xff) | (uint32_t)(d[1] & 0xff) << 8 | (uint32_t)(d[2] & 0xff) << 16 |
              (uint32_t)(d[3] & 0xff) << 24;
        w.y = (uint32_t)(d[4] & 0xff) | (uint32_t)(d[5] & 0xff) << 8 | (uint32_t)(d[6] & 0xff) << 16 |
              (uint32_t)(d[7] & 0xff) << 24;
        return w;
    };
    if (a.planes_out)
        for (int p = 0; p < a.planes; p++)
            *reinterpret_cast<uint2 *>(a.planes_out + (m * a.planes + p) * a.kpad + col) = pack(digit[p]);
    if (a.q_out)
#pragma unroll
        for (int i = 0; i < PREP_E; i++) a.q_out[e + i] = (int8_t)digit[0][i];
}

// Zero-fills `words` u32 (a graph-safe replacement for a memset).
__global__ void fill_kernel(uint32_t *p, uint64_t words) {
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < words) p[i] = 0u;
}

__global__ void fill_bytes_kernel(uint8_t *p, uint64_t bytes) {
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < bytes) p[i] = 0;
}

// ------------------------------------------------------------------ qmv
// LDS of a workgroup: a flag word (16 bytes), the segment's planes
// [rows][planes][span + 16], then xscale [rows][span/32], xsum32
// [rows][span/32], xsum16 [rows][span/16].
template <class F, int P, int MAXQ>
__global__ __launch_bounds__(256) void qmv_kernel(QmvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, n16 = lane & 15;
    const int seg = blockIdx.y;
    const int t0 = seg * a.seg_steps;
    const int t1 = min(a.steps, t0 + a.seg_steps);
    // The elements the segment covers, [e0, e0 + span).
    const int e0 = t0 * 64;
    const int span = a.seg_steps * 64;
    const int pstride = span + 16;
    int *last = reinterpret_cast<int *>(lds);
    int8_t *xp = reinterpret_cast<int8_t *>(lds + 16);
    float *xs = reinterpret_cast<float *>(lds + 16 + (size_t)a.rows * P * pstride);
    float *xs32 = xs + (size_t)a.rows * (span / 32);
    float *xs16 = xs32 + (size_t)a.rows * (span / 32);

    // Stage the segment of the activations, zero beyond K.
    {
        const int words = span / 4;
        for (int i = threadIdx.x; i < a.rows * P * words; i += 256) {
            int r = i / words, w = i % words;
            int el = e0 + 4 * w;
            uint32_t v = 0;
            if (el < a.k) v = *reinterpret_cast<const uint32_t *>(a.planes + (size_t)r * a.kpad + el);
            *reinterpret_cast<uint32_t *>(xp + (size_t)r * pstride + 4 * w) = v;
        }
        for (int i = threadIdx.x; i < a.rows * (span / 32); i += 256) {
            int r = i / (span / 32), b = i % (span / 32);
            int blk = e0 / 32 + b;
            bool in = blk < a.k / 32;
            xs[i] = in ? a.xscale[(size_t)r * (a.k / 32) + blk] : 0.0f;
            xs32[i] = in ? a.xsum32[(size_t)r * (a.k / 32) + blk] : 0.0f;
        }
        for (int i = threadIdx.x; i < a.rows * (span / 16); i += 256) {
            int r = i / (span / 16), b = i % (span / 16);
            int grp = e0 / 16 + b;
            xs16[i] = grp < a.k / 16 ? a.xsum16[(size_t)r * (a.k / 16) + grp] : 0.0f;
        }
    }
    __syncthreads();

    // This wave's 16 rows: tile blockIdx.x * 4 + wave of the launch.
    const int tile = blockIdx.x * 4 + wave;
    int mat = -1;
    for (int i = 0; i < a.count; i++)
        if (tile >= a.tile0[i] && tile < a.tile0[i] + (int)((a.n[i] + 15) / 16)) mat = i;
    constexpr int SG = slot_groups_per_mfma(P);
    const int nsg = a.rows * F::NGRP;                // slot groups in use
    const int nq = (nsg + SG - 1) / SG;
    float acc[MAXQ][4];  // P = 3 uses acc[q][0] only
#pragma unroll
    for (int q = 0; q < MAXQ; q++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[q][v] = 0.0f;

    int64_t row = 0;
    bool live = false;
    const uint8_t *rowp = nullptr;
    if (mat >= 0) {
        row = (int64_t)(tile - a.tile0[mat]) * 16 + n16;
        live = row < (int64_t)a.n[mat];
        int64_t safe = live ? row : (int64_t)a.n[mat] - 1;
        rowp = a.w[mat] + safe * (int64_t)a.row_bytes;
    }
    const bool k_tail = (a.k % 64) != 0;  // the last step has one block of 32
    if (mat >= 0) {
        // The A row this lane supplies: row i = lane % 16 of each MFMA.
        const int i = lane & 15;
        for (int t = t0; t < t1; t++) {
            const bool two = !(k_tail && t == a.steps - 1);
            v4i b = F::codes(rowp, t, g, two);
            int off[4];
            for (int d = 0; d < 4; d++) off[d] = F::xoff(t, g, d) - e0;
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                if (q >= nq) break;
                int sg, p;
                if (P == 3) {
                    sg = q * 4 + i / 4;
                    p = i % 4;
                } else {
                    sg = q * 16 + i;
                    p = 0;
                }
                v4i av = {0, 0, 0, 0};
                if (sg < nsg && p < P) {
                    int m = sg / F::NGRP, grp = sg % F::NGRP;
                    const int8_t *base = xp + (size_t)(m * P + p) * pstride;
                    if (F::NGRP == 2) {
                        if (grp == 0) {
                            av.x = *reinterpret_cast<const int *>(base + off[0]);
                            av.y = *reinterpret_cast<const int *>(base + off[1]);
                        } else {
                            av.z = *reinterpret_cast<const int *>(base + off[2]);
                            av.w = *reinterpret_cast<const int *>(base + off[3]);
                        }
                    } else {
                        int word = *reinterpret_cast<const int *>(base + off[grp]);
                        av.x = grp == 0 ? word : 0;
                        av.y = grp == 1 ? word : 0;
                        av.z = grp == 2 ? word : 0;
                        av.w = grp == 3 ? word : 0;
                    }
                }
                v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b, v4i{0, 0, 0, 0}, 0, 0, 0);
                // Output rows 4g .. 4g+3 of this MFMA, column n16.
                if (P == 3) {
                    int osg = q * 4 + g;
                    if (osg < nsg) {
                        int m = osg / F::NGRP, grp = osg % F::NGRP;
                        // d0 2^16 + d1 2^8 + d2 (the last two fit an int).
                        float dot = fmaf((float)c.x, 65536.0f, (float)((c.y << 8) + c.z));
                        bool present = two || F::gelem(t, grp) < a.k;
                        if (present) {
                            float s, mn;
                            F::scale_min(rowp, t, grp, s, mn);
                            int ge = F::gelem(t, grp) - e0;
                            float xsc = xs[m * (span / 32) + ge / 32];
                            float xsum = F::GS == 32 ? xs32[m * (span / 32) + ge / 32]
                                                     : xs16[m * (span / 16) + ge / 16];
                            acc[q][0] = fmaf(dot, s * xsc, acc[q][0]);
                            acc[q][0] = fmaf(-mn, xsum, acc[q][0]);
                        }
                    }
                } else {
                    int cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        int osg = q * 16 + 4 * g + v;
                        if (osg >= nsg) continue;
                        int m = osg / F::NGRP, grp = osg % F::NGRP;
                        bool present = two || F::gelem(t, grp) < a.k;
                        if (!present) continue;
                        if (a.dots) {
                            // Block dots in the codes of bytes.rs:282-353: Q6_K
                            // signed (stored - 32), the others as stored.
                            int dot = cv[v];
                            int ge = F::gelem(t, grp);
                            if (a.signed_offset)
                                dot -= a.signed_offset * a.xsumi16[(size_t)m * (a.k / 16) + ge / 16];
                            if (live)
                                a.dots[((size_t)m * a.width + a.col0[mat] + row) * (a.k / 16) + ge / 16] = dot;
                            continue;
                        }
                        float s, mn;
                        F::scale_min(rowp, t, grp, s, mn);
                        int ge = F::gelem(t, grp) - e0;
                        float xsc = xs[m * (span / 32) + ge / 32];
                        float xsum = F::GS == 32 ? xs32[m * (span / 32) + ge / 32]
                                                 : xs16[m * (span / 16) + ge / 16];
                        acc[q][v] = fmaf((float)cv[v], s * xsc, acc[q][v]);
                        acc[q][v] = fmaf(-mn, xsum, acc[q][v]);
                    }
                }
            }
        }
    }
    if (a.dots) return;

    // Sums over the groups of each activation row, in a fixed order, then out
    // (one segment) or the segment's partial sums.
    float *partial = a.partials + (size_t)seg * a.rows * a.pwidth;
    auto emit = [&](int m, float v) {
        if (!live) return;
        size_t col = (size_t)a.col0[mat] + row;
        if (a.segs == 1) store_out(a.out_kind, a.out, (size_t)m * a.out_stride + col, v);
        else partial[(size_t)m * a.pwidth + (size_t)tile * 16 + n16] = v;
    };
    if (mat >= 0) {
        if (P == 3) {
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                if (q >= nq) break;
                float v = acc[q][0];
                // slot group q*4 + g: NGRP 2 -> rows 2q + g/2, groups g%2;
                // NGRP 4 -> row q, groups g.
                v = v + __shfl_xor(v, 16);
                if (F::NGRP == 4) v = v + __shfl_xor(v, 32);
                int osg = q * 4 + g;
                if (osg < nsg && osg % F::NGRP == 0) emit(osg / F::NGRP, v);
            }
        } else {
#pragma unroll
            for (int q = 0; q < MAXQ; q++) {
                if (q >= nq) break;
                if (F::NGRP == 2) {
                    int m0 = (q * 16 + 4 * g) / 2;
                    if (2 * m0 < nsg) emit(m0, acc[q][0] + acc[q][1]);
                    if (2 * (m0 + 1) < nsg) emit(m0 + 1, acc[q][2] + acc[q][3]);
                } else {
                    int m0 = (q * 16 + 4 * g) / 4;
                    if (4 * m0 < nsg) emit(m0, (acc[q][0] + acc[q][1]) + (acc[q][2] + acc[q][3]));
                }
            }
        }
    }
    if (a.segs == 1) return;

    // The last workgroup of this row range to finish adds the segments.
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        int old = __hip_atomic_fetch_add(a.counters + blockIdx.x, 1, __ATOMIC_ACQ_REL,
                                         __HIP_MEMORY_SCOPE_AGENT);
        *last = old == a.segs - 1;
    }
    __syncthreads();
    if (!*last) return;
    __threadfence();
    for (int idx = threadIdx.x; idx < 64 * a.rows; idx += 256) {
        int m = idx / 64, r = idx % 64;
        int tl = blockIdx.x * 4 + r / 16;
        int mt = -1;
        for (int i = 0; i < a.count; i++)
            if (tl >= a.tile0[i] && tl < a.tile0[i] + (int)((a.n[i] + 15) / 16)) mt = i;
        if (mt < 0) continue;
        int64_t rr = (int64_t)(tl - a.tile0[mt]) * 16 + (r % 16);
        if (rr >= (int64_t)a.n[mt]) continue;
        size_t col = (size_t)a.col0[mt] + rr;
        float v = 0.0f;
        for (int s = 0; s < a.segs; s++)
            v = v + __hip_atomic_load(a.partials + ((size_t)s * a.rows + m) * a.pwidth + (size_t)tl * 16 + r % 16,
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        store_out(a.out_kind, a.out, (size_t)m * a.out_stride + col, v);
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(a.counters + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// --------------------------------------------------------- element decode
// The value of element e of a row, in f32, by the decoders of
// kapel-cpu/src/quantized.rs:403-682 (products in f32, not fused).
__device__ float element(uint32_t fmt, uint32_t group, const uint8_t *row, uint64_t e) {
    switch (fmt) {
    case KH_INT8: {
        const uint8_t *blk = row + (e / group) * (4 + group);
        return ldf32(blk) * (float)(int8_t)blk[4 + e % group];
    }
    case KH_INT4: {
        const uint8_t *blk = row + (e / group) * (4 + group / 2);
        uint32_t i = e % group;
        uint32_t byte = blk[4 + i / 2];
        return ldf32(blk) * ((float)((i & 1) ? byte >> 4 : byte & 15u) - 8.0f);
    }
    case KH_Q8_0: {
        const uint8_t *blk = row + (e / 32) * 34;
        return half_at(blk) * (float)(int8_t)blk[2 + e % 32];
    }
    case KH_Q4_0: case KH_Q4_1: {
        bool one = fmt == KH_Q4_1;
        const uint8_t *blk = row + (e / 32) * (one ? 20 : 18);
        uint32_t j = e % 32;
        uint32_t byte = blk[(one ? 4 : 2) + j % 16];
        float q = (float)(j < 16 ? byte & 15u : byte >> 4);
        return one ? half_at(blk) * q + half_at(blk + 2) : half_at(blk) * (q - 8.0f);
    }
    case KH_Q5_0: case KH_Q5_1: {
        bool one = fmt == KH_Q5_1;
        const uint8_t *blk = row + (e / 32) * (one ? 24 : 22);
        const uint8_t *rest = blk + (one ? 4 : 2);
        uint32_t j = e % 32, high = ld32e(rest), byte = rest[4 + j % 16];
        uint32_t q = (j < 16 ? byte & 15u : byte >> 4) | (((high >> j) & 1u) << 4);
        return one ? half_at(blk) * (float)q + half_at(blk + 2) : half_at(blk) * ((float)q - 16.0f);
    }
    case KH_Q2K: {
        const uint8_t *blk = row + (e / 256) * 84;
        uint32_t f = e % 256, h = f / 128, s = f % 128 / 32, l = f % 32;
        uint32_t k = blk[f / 16];
        float q = (float)((blk[16 + h * 32 + l] >> (2 * s)) & 3u);
        return half_at(blk + 80) * (float)(k & 15u) * q - half_at(blk + 82) * (float)(k >> 4);
    }
    case KH_Q3K: {
        const uint8_t *blk = row + (e / 256) * 110;
        uint32_t f = e % 256, i = f / 16, h = f / 128, s = f % 128 / 32, l = f % 32;
        const uint8_t *packed = blk + 96;
        uint32_t lo = (packed[i % 8] >> (4 * (i / 8))) & 15u, hi = (packed[8 + i % 4] >> (2 * (i / 4))) & 3u;
        float scale = half_at(blk + 108) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
        int low = (blk[32 + h * 32 + l] >> (2 * s)) & 3;
        int high = ((blk[l] >> (f / 32)) & 1) ^ 1;
        return scale * (float)(low - 4 * high);
    }
    case KH_Q4K: case KH_Q5K: {
        bool five = fmt == KH_Q5K;
        const uint8_t *blk = row + (e / 256) * (five ? 176 : 144);
        uint32_t f = e % 256, c = f / 64, t = f % 64 / 32, l = f % 32;
        float s, m;
        Q4K::kscale(blk, (int)(f / 32), s, m);
        uint32_t q = (blk[(five ? 48 : 16) + c * 32 + l] >> (4 * t)) & 15u;
        if (five) q |= ((blk[16 + l] >> (f / 32)) & 1u) << 4;
        return s * (float)q - m;
    }
    case KH_Q6K: {
        const uint8_t *blk = row + (e / 256) * 210;
        uint32_t f = e % 256, h = f / 128, t = f % 128 / 64, mm = f % 64, s = f % 128 / 32, l = f % 32;
        uint32_t ql = (blk[h * 64 + mm] >> (4 * t)) & 15u;
        uint32_t qh = (blk[128 + h * 32 + l] >> (2 * s)) & 3u;
        float scale = half_at(blk + 208) * (float)(int8_t)blk[192 + f / 16];
        return scale * ((float)(ql | (qh << 4)) - 32.0f);
    }
    case KH_IQ4_NL: {
        const uint8_t *blk = row + (e / 32) * 18;
        uint32_t j = e % 32, byte = blk[2 + j % 16];
        return half_at(blk) * (float)iq4nl_value(j < 16 ? byte & 15u : byte >> 4);
    }
    case KH_IQ4_XS: {
        const uint8_t *blk = row + (e / 256) * 136;
        uint32_t f = e % 256, g = f / 32, j = f % 32;
        int s = (int)((blk[4 + g / 2] >> (4 * (g % 2))) & 15u) | (int)(((ld16(blk + 2) >> (2 * g)) & 3u) << 4);
        uint32_t byte = blk[8 + 16 * g + j % 16];
        float scale = half_at(blk) * (float)(s - 32);
        return scale * (float)iq4nl_value(j < 16 ? byte & 15u : byte >> 4);
    }
    case KH_IQ3_S: {
        const uint8_t *blk = row + (e / 256) * 110;
        uint32_t f = e % 256, g = f / 32, l = f % 32 / 8, j = f % 8;
        uint32_t s = (blk[106 + g / 2] >> (4 * (g % 2))) & 15u;
        float db = half_at(blk) * (float)(1u + 2u * s);
        uint32_t index = blk[2 + 8 * g + 2 * l + j / 4] | (((uint32_t)blk[66 + g] << (8 - 2 * l - j / 4)) & 256u);
        float v = db * (float)((IQ3S_GRID[index] >> (8 * (j % 4))) & 255u);
        return ((blk[74 + 4 * g + l] >> j) & 1u) ? -v : v;
    }
    default:
        return __uint_as_float(0x7fc00000u);  // unknown code: NaN, never a fault
    }
}

// The product for the formats and groups the MFMA readers do not take
// (Kapel groups that are not a multiple of 32): one wave per weight row,
// f32 fused multiply-adds in a fixed lane order, then a fixed butterfly.
__global__ __launch_bounds__(256) void qmv_generic_kernel(GenericArgs a) {
    const int lane = threadIdx.x & 63;
    uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.n) return;
    if (a.experts) {
        // The experts' product: route r takes rows of expert experts[r].
        for (uint64_t r = blockIdx.y; r < a.rows; r += gridDim.y) {
            const uint32_t e = a.experts[r];
            const uint64_t xr = a.per_route ? r : r / (uint64_t)a.topk;
            float acc = 0.0f;
            if (e < a.n_experts) {
                const uint8_t *rowp = a.w + e * a.expert_bytes + row * a.row_bytes;
                for (uint64_t i = lane; i < a.k; i += 64)
                    acc = fmaf(element(a.format, a.group, rowp, i), load_x(a.x_kind, a.x, xr * a.k + i), acc);
                for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s);
            } else {
                acc = __uint_as_float(0x7fc00000u);
            }
            if (lane == 0) store_out(a.out_kind, a.out, r * a.out_stride + row, acc);
        }
        return;
    }
    const uint8_t *rowp = a.w + row * a.row_bytes;
    for (uint64_t m = 0; m < a.rows; m++) {
        float acc = 0.0f;
        for (uint64_t e = lane; e < a.k; e += 64)
            acc = fmaf(element(a.format, a.group, rowp, e), load_x(a.x_kind, a.x, m * a.k + e), acc);
        for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s);
        if (lane == 0) store_out(a.out_kind, a.out, m * a.out_stride + a.col0 + row, acc);
    }
}

// Dequantization to a float type: rows of a weight, or gathered rows.
__global__ __launch_bounds__(256) void dequantize_kernel(DequantArgs a) {
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.count * a.k) return;
    uint64_t r = i / a.k, e = i % a.k;
    uint64_t row = a.indices ? (uint64_t)a.indices[r] : a.first + r;
    float v = row < a.n ? element(a.format, a.group, a.w + row * a.row_bytes, e)
                        : __uint_as_float(0x7fc00000u);
    store_out(a.out_kind, a.out, i, v);
}

// ------------------------------------------------------------ launchers
// MFMAs per step: P = 3 takes 4 slot groups (row, group) per MFMA, P = 1 16.
template <class F, int P>
hipError_t launch_qmv_t(const QmvArgs &a, dim3 grid, size_t lds, hipStream_t stream) {
    constexpr int SG = slot_groups_per_mfma(P);
    int nq = (a.rows * F::NGRP + SG - 1) / SG;
    if (nq <= 1) hipLaunchKernelGGL((qmv_kernel<F, P, 1>), grid, dim3(256), lds, stream, a);
    else if (nq <= 4) hipLaunchKernelGGL((qmv_kernel<F, P, 4>), grid, dim3(256), lds, stream, a);
    else if (nq <= MAX_MFMAS) hipLaunchKernelGGL((qmv_kernel<F, P, MAX_MFMAS>), grid, dim3(256), lds, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int P>
hipError_t launch_qmv_p(uint32_t fmt, uint32_t group, const QmvArgs &a, dim3 grid, size_t lds,
                        hipStream_t s) {
    switch (fmt) {
    case KH_Q4K: return launch_qmv_t<Q4K, P>(a, grid, lds, s);
    case KH_Q5K: return launch_qmv_t<Q5K, P>(a, grid, lds, s);
    case KH_Q6K: return launch_qmv_t<Q6K, P>(a, grid, lds, s);
    case KH_Q2K: return launch_qmv_t<Q2K, P>(a, grid, lds, s);
    case KH_Q3K: return launch_qmv_t<Q3K, P>(a, grid, lds, s);
    case KH_Q4_0: return launch_qmv_t<Q4_0, P>(a, grid, lds, s);
    case KH_Q4_1: return launch_qmv_t<Q4_1, P>(a, grid, lds, s);
    case KH_Q5_0: return launch_qmv_t<Q5_0, P>(a, grid, lds, s);
    case KH_Q5_1: return launch_qmv_t<Q5_1, P>(a, grid, lds, s);
    case KH_Q8_0: return launch_qmv_t<Q8_0, P>(a, grid, lds, s);
    case KH_INT8:
        if (group == 32) return launch_qmv_t<Int8G<32>, P>(a, grid, lds, s);
        if (group == 64) return launch_qmv_t<Int8G<64>, P>(a, grid, lds, s);
        if (group == 128) return launch_qmv_t<Int8G<128>, P>(a, grid, lds, s);
        if (group == 256) return launch_qmv_t<Int8G<256>, P>(a, grid, lds, s);
        break;
    case KH_INT4:
        if (group == 32) return launch_qmv_t<Int4G<32>, P>(a, grid, lds, s);
        if (group == 64) return launch_qmv_t<Int4G<64>, P>(a, grid, lds, s);
        if (group == 128) return launch_qmv_t<Int4G<128>, P>(a, grid, lds, s);
        if (group == 256) return launch_qmv_t<Int4G<256>, P>(a, grid, lds, s);
        break;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qmv(uint32_t fmt, uint32_t group, int planes, const QmvArgs &a, dim3 grid,
                      size_t lds, hipStream_t s) {
    return planes == 1 ? launch_qmv_p<1>(fmt, group, a, grid, lds, s)
                       : launch_qmv_p<3>(fmt, group, a, grid, lds, s);
}

hipError_t launch_prep(const PrepArgs &a, hipStream_t s) {
    uint64_t total = a.rows * a.k / PREP_E;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(prep_x_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_fill(uint32_t *p, uint64_t words, hipStream_t s) {
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s, p, words);
    return hipGetLastError();
}

hipError_t launch_fill_bytes(uint8_t *p, uint64_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0, s, p, bytes);
    return hipGetLastError();
}

hipError_t launch_generic(const GenericArgs &a, hipStream_t s) {
    if (a.n == 0 || (a.experts && a.rows == 0)) return hipSuccess;
    const unsigned routes = a.experts ? (unsigned)std::min<uint64_t>(a.rows, 65535) : 1u;
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((unsigned)((a.n + 3) / 4), routes), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_dequantize(const DequantArgs &a, hipStream_t s) {
    uint64_t total = a.count * a.k;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace kh
