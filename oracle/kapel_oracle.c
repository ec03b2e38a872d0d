/*
 * kapel_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU algorithm for the product by
 * quantized weights (smallbard/kapel, read as text; its Rust sources cannot be
 * built here).  It is the checker of the HIP library: only tests/, the smoke
 * check and bench.py's cpu_baseline leg may load it.  Nothing of the product
 * path calls it.
 *
 * Every function names the reference file:line it restates.  Paths are under
 * crates/ of the reference.
 *
 * Build: make -C oracle  (gcc, -ffp-contract=off: the reference's Rust never
 * fuses a multiply and an add unless it calls mul_add, and the restatement
 * must round where it rounds).
 *
 * Pins (what checks each part; the tests live in tests/test_oracle.py):
 *   ko_f16_decode / ko_f16_encode / ko_half_f32 : all 65,536 patterns against
 *       numpy's float16, the published extremes (kapel-core/src/float.rs tests).
 *   ko_dequantize  : golden blocks decoded by GGML-order transcriptions
 *       (kapel-ref/src/golden.rs), hand cases (dtype.rs tests).
 *   ko_quantize    : closed-form rules and the error bounds of dtype.rs tests
 *       (:948-1027), int4 squared-error bound, and an independent
 *       implementation (the product library's host quantizer) byte for byte.
 *   ko_decode_f32  : within 1e-6 relative of ko_dequantize (quantized.rs:1097).
 *   ko_product_f32 : within 1e-4 (1 + |e|) of the f64 product (quantized.rs:1150).
 *   ko_quantize_x  : closed form checked against numpy (round half to even).
 *   ko_block_dots  : brute-force i32 dots from numpy on the same codes.
 *   ko_product_bytes: within 1e-5 sum|x w| + 1e-6 of the exact product of the
 *       quantized activations (bytes.rs:720-774).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

/* Format codes: those of kapel-cuda-abi/src/lib.rs:167-194, plus Q2_K = 13,
 * Q3_K = 14 (the reference's ABI has no code for them). */
enum {
    KO_INT8 = 0, KO_INT4 = 1, KO_Q8_0 = 2, KO_Q4_0 = 3, KO_Q4_1 = 4,
    KO_Q5_0 = 5, KO_Q5_1 = 6, KO_Q4K = 7, KO_Q5K = 8, KO_Q6K = 9,
    KO_Q2K = 13, KO_Q3K = 14
};

/* ---------------------------------------------------------------------- */
/* Geometry: kapel-core/src/dtype.rs:140-187                                */
/* ---------------------------------------------------------------------- */

int ko_block_len(int fmt, int group) {
    switch (fmt) {
    case KO_INT8: case KO_INT4: return group;
    case KO_Q8_0: case KO_Q4_0: case KO_Q4_1: case KO_Q5_0: case KO_Q5_1: return 32;
    case KO_Q2K: case KO_Q3K: case KO_Q4K: case KO_Q5K: case KO_Q6K: return 256;
    default: return 0;
    }
}

int ko_block_bytes(int fmt, int group) {
    switch (fmt) {
    case KO_INT8: return 4 + group;
    case KO_INT4: return 4 + group / 2;
    case KO_Q8_0: return 34;
    case KO_Q4_0: return 18;
    case KO_Q4_1: return 20;
    case KO_Q5_0: return 22;
    case KO_Q5_1: return 24;
    case KO_Q2K: return 84;
    case KO_Q3K: return 110;
    case KO_Q4K: return 144;
    case KO_Q5K: return 176;
    case KO_Q6K: return 210;
    default: return 0;
    }
}

/* ---------------------------------------------------------------------- */
/* f16: kapel-core/src/float.rs:82-145 (exact decode, round-to-nearest-even  */
/* encode), and the branch-free f32 decode of kapel-cpu/src/quantized.rs:  */
/* 386-396.                                                                 */
/* ---------------------------------------------------------------------- */

static double pow2(int e) { return ldexp(1.0, e); }

double ko_f16_decode(uint32_t bits) {
    double sign = (bits & 0x8000) ? -1.0 : 1.0;
    uint32_t exponent = (bits >> 10) & 0x1f, mantissa = bits & 0x3ff;
    if (exponent == 0x1f) return mantissa == 0 ? sign * INFINITY : NAN;
    if (exponent == 0) return sign * (double)mantissa * pow2(1 - 15 - 10);
    return sign * (double)(0x400 | mantissa) * pow2((int)exponent - 15 - 10);
}

uint32_t ko_f16_encode(double x) {
    if (isnan(x)) return 0x7e00;
    uint32_t sign = signbit(x) ? 0x8000 : 0;
    double a = fabs(x);
    if (isinf(a)) return sign | 0x7c00;
    if (a == 0.0) return sign;
    int e2;
    frexp(a, &e2);            /* a = f * 2^e2, f in [0.5, 1) */
    int exponent = e2 - 1;    /* 2^exponent <= a < 2^(exponent+1) */
    if (exponent < -14) {
        double units = nearbyint(a * pow2(10 + 14)); /* ties to even */
        return sign | (uint32_t)units;
    }
    uint32_t significand = (uint32_t)nearbyint(a * pow2(10 - exponent));
    if (significand == (1u << 11)) { significand >>= 1; exponent += 1; }
    uint32_t field = (uint32_t)(exponent + 15);
    uint32_t bits = (field << 10) | (significand & 0x3ff);
    if (field > 0x1f || bits > 0x7bff) return sign | 0x7c00;
    return sign | bits;
}

static inline float f32_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* quantized.rs:386-396 */
float ko_half_f32(uint32_t bits) {
    uint32_t magnitude = bits & 0x7fff;
    float value;
    if (magnitude >= 0x7c00)
        value = f32_of(0x7f800000u | (magnitude & 0x3ff) << 13);
    else
        value = f32_of(magnitude << 13) * f32_of(0x77800000u);
    return f32_of(bits_of(value) | (bits & 0x8000) << 16);
}

static inline double half64(const uint8_t *b, int at) {
    return ko_f16_decode((uint32_t)b[at] | (uint32_t)b[at + 1] << 8);
}
static inline float half32(const uint8_t *b, int at) {
    return ko_half_f32((uint32_t)b[at] | (uint32_t)b[at + 1] << 8);
}
static inline float single32(const uint8_t *b) { float f; memcpy(&f, b, 4); return f; }

/* ---------------------------------------------------------------------- */
/* The reference dequantization in f64: kapel-core/src/dtype.rs:342-520     */
/* ---------------------------------------------------------------------- */

/* dtype.rs:847-858 */
static void k_scales64(const uint8_t *p, double scale[8], double minimum[8]) {
    const uint8_t *d = p, *m = p + 4, *md = p + 8;
    for (int i = 0; i < 4; i++) {
        scale[i] = d[i] & 0x3f;
        minimum[i] = m[i] & 0x3f;
        scale[4 + i] = (md[i] & 0x0f) | ((d[i] >> 2) & 0x30);
        minimum[4 + i] = (md[i] >> 4) | ((m[i] >> 2) & 0x30);
    }
}

/* Decodes `blocks` blocks into out (block_len each).  Returns 0, or -1 for
 * an unknown format. */
int ko_dequantize(int fmt, int group, const uint8_t *bytes, int64_t blocks, double *out) {
    int len = ko_block_len(fmt, group), size = ko_block_bytes(fmt, group);
    if (len <= 0 || size <= 0) return -1;
    for (int64_t bi = 0; bi < blocks; bi++) {
        const uint8_t *block = bytes + bi * size;
        double *y = out + bi * len;
        switch (fmt) {
        case KO_INT8: {                                   /* :364-367 */
            double scale = single32(block);
            for (int i = 0; i < len; i++) y[i] = scale * (double)(int8_t)block[4 + i];
        } break;
        case KO_INT4: {                                   /* :368-374 */
            double scale = single32(block);
            for (int i = 0; i < len / 2; i++) {
                uint8_t byte = block[4 + i];
                y[2 * i] = scale * ((double)(byte & 0x0f) - 8.0);
                y[2 * i + 1] = scale * ((double)(byte >> 4) - 8.0);
            }
        } break;
        case KO_Q8_0: {                                   /* :375-378 */
            double scale = half64(block, 0);
            for (int i = 0; i < 32; i++) y[i] = scale * (double)(int8_t)block[2 + i];
        } break;
        case KO_Q4_0: case KO_Q4_1: {                     /* :379-391 */
            double scale = half64(block, 0);
            double minimum = fmt == KO_Q4_1 ? half64(block, 2) : 0.0;
            const uint8_t *codes = block + (fmt == KO_Q4_1 ? 4 : 2);
            for (int j = 0; j < 16; j++) {
                double lo = codes[j] & 0x0f, hi = codes[j] >> 4;
                y[j] = fmt == KO_Q4_1 ? scale * lo + minimum : scale * (lo - 8.0);
                y[j + 16] = fmt == KO_Q4_1 ? scale * hi + minimum : scale * (hi - 8.0);
            }
        } break;
        case KO_Q5_0: case KO_Q5_1: {                     /* :392-411 */
            double scale = half64(block, 0);
            double minimum = fmt == KO_Q5_1 ? half64(block, 2) : 0.0;
            const uint8_t *rest = block + (fmt == KO_Q5_1 ? 4 : 2);
            uint32_t high = (uint32_t)rest[0] | (uint32_t)rest[1] << 8 |
                            (uint32_t)rest[2] << 16 | (uint32_t)rest[3] << 24;
            const uint8_t *codes = rest + 4;
            for (int j = 0; j < 32; j++) {
                uint8_t low = j < 16 ? (codes[j] & 0x0f) : (codes[j - 16] >> 4);
                double q = (double)(low | (((high >> j) & 1) << 4));
                y[j] = fmt == KO_Q5_1 ? scale * q + minimum : scale * (q - 16.0);
            }
        } break;
        case KO_Q2K: {                                    /* :413-422 */
            const uint8_t *scales = block, *codes = block + 16;
            double d = half64(block, 80), dmin = half64(block, 82);
            for (int e = 0; e < 256; e++) {
                int h = e / 128, s = e % 128 / 32, l = e % 32;
                double q = (codes[h * 32 + l] >> (2 * s)) & 3;
                uint8_t k = scales[e / 16];
                y[e] = d * (double)(k & 0x0f) * q - dmin * (double)(k >> 4);
            }
        } break;
        case KO_Q3K: {                                    /* :423-440 */
            const uint8_t *mask = block, *codes = block + 32, *packed = block + 96;
            double d = half64(block, 108);
            for (int e = 0; e < 256; e++) {
                int i = e / 16;
                int low6 = (packed[i % 8] >> (4 * (i / 8))) & 0x0f;
                int high6 = (packed[8 + i % 4] >> (2 * (i / 4))) & 0x03;
                double scale = (double)((int)(int8_t)(uint8_t)(low6 | (high6 << 4)) - 32);
                int h = e / 128, s = e % 128 / 32, l = e % 32;
                int low = (codes[h * 32 + l] >> (2 * s)) & 3;
                int high = ((mask[e % 32] >> (e / 32)) & 1) ^ 1;
                y[e] = d * scale * (double)(low - 4 * high);
            }
        } break;
        case KO_Q4K: case KO_Q5K: {                       /* :441-457 */
            double d = half64(block, 0), dmin = half64(block, 2);
            double scale[8], minimum[8];
            k_scales64(block + 4, scale, minimum);
            const uint8_t *high = fmt == KO_Q5K ? block + 16 : NULL;
            const uint8_t *codes = fmt == KO_Q5K ? block + 48 : block + 16;
            for (int e = 0; e < 256; e++) {
                int c = e / 64, t = e % 64 / 32, l = e % 32;
                int q = (codes[c * 32 + l] >> (4 * t)) & 0x0f;
                if (high) q |= ((high[l] >> (e / 32)) & 1) << 4;
                int k = e / 32;
                y[e] = d * scale[k] * (double)q - dmin * minimum[k];
            }
        } break;
        case KO_Q6K: {                                    /* :458-469 */
            const uint8_t *low = block, *high = block + 128, *scales = block + 192;
            double d = half64(block, 208);
            for (int f = 0; f < 256; f++) {
                int h = f / 128, t = f % 128 / 64, m = f % 64;
                int ql = (low[h * 64 + m] >> (4 * t)) & 0x0f;
                int s = f % 128 / 32, l = f % 32;
                int qh = (high[h * 32 + l] >> (2 * s)) & 0x03;
                int q = (ql | (qh << 4)) - 32;
                y[f] = d * (double)(int8_t)scales[f / 16] * (double)q;
            }
        } break;
        default: return -1;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------------- */
/* The reference quantizers: kapel-core/src/dtype.rs:565-841                */
/* ---------------------------------------------------------------------- */

/* Rust's f32/f64 `round`: half away from zero = C round/roundf. */

/* dtype.rs:789-841: int4 scale search; codes 0..15 into `codes`. */
static float int4_codes(const float *block, int len, uint8_t *codes) {
    float m = 0.0f;
    for (int i = 0; i < len; i++) if (fabsf(block[i]) > fabsf(m)) m = block[i];
    float best_scale = 0.0f;
    double best_error = INFINITY;
    for (int i = 0; i < len; i++) codes[i] = 8;
    if (m == 0.0f) return 0.0f;
    uint8_t *trial = malloc(len), *refit = malloc(len);
    for (int step = 0; step <= 20; step++) {
        double levels = -8.0 + 15.0 * (double)step / 20.0;
        if (fabs(levels) < 6.5) continue;
        double scale = (double)m / levels;
        for (int i = 0; i < len; i++) {
            double r = round((double)block[i] / scale);
            r = r < -8.0 ? -8.0 : (r > 7.0 ? 7.0 : r);
            trial[i] = (uint8_t)(r + 8.0);
        }
        double num = 0.0, den = 0.0;
        for (int i = 0; i < len; i++) {
            double c = (double)trial[i] - 8.0;
            num = num + (double)block[i] * c;
            den = den + c * c;
        }
        double fit = num / den;
        /* A scale that is not finite and non-zero as f32 is skipped below:
         * its codes are never read. */
        for (int i = 0; i < len; i++) {
            double r = isfinite(fit) && fit != 0.0 ? round((double)block[i] / fit) : 0.0;
            r = r < -8.0 ? -8.0 : (r > 7.0 ? 7.0 : r);
            refit[i] = (uint8_t)(r + 8.0);
        }
        for (int pass = 0; pass < 2; pass++) {
            float s = pass == 0 ? (float)scale : (float)fit;
            const uint8_t *c = pass == 0 ? trial : refit;
            if (!(isfinite(s) && s != 0.0f)) continue;
            double e = 0.0;
            for (int i = 0; i < len; i++) {
                double d = (double)block[i] - (double)s * ((double)c[i] - 8.0);
                e = e + d * d;
            }
            if (e < best_error) {
                best_error = e;
                best_scale = s;
                memcpy(codes, c, len);
            }
        }
    }
    free(trial);
    free(refit);
    return best_scale;
}

static uint8_t clamp_i8_code(float r) {
    if (isnan(r)) r = 0.0f;
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return (uint8_t)(int8_t)r;
}

/* Quantizes `count` values (whole blocks) of `fmt` into out.  Only the
 * formats the reference writes (dtype.rs:546-556): int8, int4, Q8_0, Q4_0,
 * Q4_1.  Returns the bytes written, or -1. */
int64_t ko_quantize(int fmt, int group, const float *values, int64_t count, uint8_t *out) {
    int len = ko_block_len(fmt, group), size = ko_block_bytes(fmt, group);
    if (len <= 0 || count % len) return -1;
    if (!(fmt == KO_INT8 || fmt == KO_INT4 || fmt == KO_Q8_0 || fmt == KO_Q4_0 || fmt == KO_Q4_1))
        return -1;
    uint8_t *codes = malloc(len);
    for (int64_t b = 0; b < count / len; b++) {
        const float *x = values + b * len;
        uint8_t *o = out + b * size;
        double largest = 0.0;                          /* dtype.rs:584 */
        for (int i = 0; i < len; i++) largest = fmax(largest, fabs((double)x[i]));
        switch (fmt) {
        case KO_INT8: {                                /* :588-596, :641-643 */
            double step = (double)(float)(largest / 127.0);
            double inverse = step != 0.0 ? 1.0 / step : 0.0;
            float s = (float)step;
            memcpy(o, &s, 4);
            for (int i = 0; i < len; i++) {
                double r = round((double)x[i] * inverse);
                r = r < -127.0 ? -127.0 : (r > 127.0 ? 127.0 : r);
                o[4 + i] = (uint8_t)(int8_t)r;
            }
        } break;
        case KO_INT4: {                                /* :597-605, :704-706 */
            float s = int4_codes(x, len, codes);
            memcpy(o, &s, 4);
            for (int i = 0; i < len / 2; i++) o[4 + i] = codes[2 * i] | (codes[2 * i + 1] << 4);
        } break;
        case KO_Q8_0: {                                /* :607-615 */
            float d = (float)largest / 127.0f;
            float inverse = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t h = ko_f16_encode((double)d);
            o[0] = h & 0xff; o[1] = h >> 8;
            for (int i = 0; i < 32; i++) o[2 + i] = clamp_i8_code(roundf(x[i] * inverse));
        } break;
        case KO_Q4_0: {                                /* :616-627, :652 */
            float m = 0.0f;
            for (int i = 0; i < 32; i++) if (fabsf(x[i]) > fabsf(m)) m = x[i];
            float d = m / -8.0f;
            float inverse = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t h = ko_f16_encode((double)d);
            o[0] = h & 0xff; o[1] = h >> 8;
            for (int i = 0; i < 32; i++) {
                float t = x[i] * inverse;
                float r = floorf(t + 8.5f);
                r = r < 0.0f ? 0.0f : (r > 15.0f ? 15.0f : r);
                codes[i] = (uint8_t)r;
            }
            for (int j = 0; j < 16; j++) o[2 + j] = codes[j] | (codes[j + 16] << 4);
        } break;
        case KO_Q4_1: {                                /* :628-639, :653-655 */
            float low = INFINITY, high = -INFINITY;
            for (int i = 0; i < 32; i++) { low = fminf(low, x[i]); high = fmaxf(high, x[i]); }
            float d = (high - low) / 15.0f;
            float inverse = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t hd = ko_f16_encode((double)d), hm = ko_f16_encode((double)low);
            o[0] = hd & 0xff; o[1] = hd >> 8; o[2] = hm & 0xff; o[3] = hm >> 8;
            for (int i = 0; i < 32; i++) {
                float t = (x[i] - low) * inverse;
                float r = floorf(t + 0.5f);
                r = r < 0.0f ? 0.0f : (r > 15.0f ? 15.0f : r);
                codes[i] = (uint8_t)r;
            }
            for (int j = 0; j < 16; j++) o[4 + j] = codes[j] | (codes[j + 16] << 4);
        } break;
        }
    }
    free(codes);
    return count / len * size;
}

/* ---------------------------------------------------------------------- */
/* f32 block decoders: kapel-cpu/src/quantized.rs:403-682 (portable).       */
/* Products, not fused, in f32, as written there.                          */
/* ---------------------------------------------------------------------- */

/* quantized.rs:603-616 */
static void k_scales32(const uint8_t *block, float scale[8], float minimum[8]) {
    float d = half32(block, 0), dmin = half32(block, 2);
    const uint8_t *sc = block + 4, *mn = block + 8, *md = block + 12;
    for (int i = 0; i < 4; i++) {
        scale[i] = d * (float)(sc[i] & 0x3f);
        minimum[i] = dmin * (float)(mn[i] & 0x3f);
        scale[4 + i] = d * (float)((md[i] & 0x0f) | ((sc[i] >> 2) & 0x30));
        minimum[4 + i] = dmin * (float)((md[i] >> 4) | ((mn[i] >> 2) & 0x30));
    }
}

int ko_decode_f32(int fmt, int group, const uint8_t *block, float *out) {
    switch (fmt) {
    case KO_INT8: {                                       /* :403-409 */
        float scale = single32(block);
        for (int i = 0; i < group; i++) out[i] = scale * (float)(int8_t)block[4 + i];
    } break;
    case KO_INT4: {                                       /* :411-418 */
        float scale = single32(block);
        for (int i = 0; i < group / 2; i++) {
            out[2 * i] = scale * ((float)(block[4 + i] & 0x0f) - 8.0f);
            out[2 * i + 1] = scale * ((float)(block[4 + i] >> 4) - 8.0f);
        }
    } break;
    case KO_Q8_0: {                                       /* :492-499 */
        float scale = half32(block, 0);
        for (int i = 0; i < 32; i++) out[i] = scale * (float)(int8_t)block[2 + i];
    } break;
    case KO_Q4_0: {                                       /* :511-520 */
        float scale = half32(block, 0);
        for (int j = 0; j < 16; j++) {
            out[j] = scale * ((float)(block[2 + j] & 0x0f) - 8.0f);
            out[j + 16] = scale * ((float)(block[2 + j] >> 4) - 8.0f);
        }
    } break;
    case KO_Q4_1: {                                       /* :501-509, :522-531 */
        float scale = half32(block, 0), minimum = half32(block, 2);
        for (int j = 0; j < 16; j++) {
            out[j] = scale * (float)(block[4 + j] & 0x0f) + minimum;
            out[j + 16] = scale * (float)(block[4 + j] >> 4) + minimum;
        }
    } break;
    case KO_Q5_0: case KO_Q5_1: {                         /* :533-565 */
        int five1 = fmt == KO_Q5_1;
        float scale = half32(block, 0), minimum = five1 ? half32(block, 2) : 0.0f;
        const uint8_t *hb = block + (five1 ? 4 : 2), *codes = hb + 4;
        uint32_t high = (uint32_t)hb[0] | (uint32_t)hb[1] << 8 | (uint32_t)hb[2] << 16 |
                        (uint32_t)hb[3] << 24;
        for (int j = 0; j < 32; j++) {
            uint8_t q = j < 16 ? (codes[j] & 0x0f) : (codes[j - 16] >> 4);
            q |= ((high >> j) & 1) << 4;
            out[j] = five1 ? scale * (float)q + minimum : scale * ((float)q - 16.0f);
        }
    } break;
    case KO_Q2K: {                                        /* :567-583 */
        const uint8_t *scales = block, *codes = block + 16;
        float d = half32(block, 80), dmin = half32(block, 82);
        for (int h = 0; h < 2; h++)
            for (int s = 0; s < 4; s++)
                for (int half = 0; half < 2; half++) {
                    uint8_t k = scales[h * 8 + s * 2 + half];
                    float scale = d * (float)(k & 0x0f), minimum = dmin * (float)(k >> 4);
                    int at = h * 128 + s * 32 + half * 16;
                    const uint8_t *c = codes + h * 32 + half * 16;
                    for (int i = 0; i < 16; i++)
                        out[at + i] = scale * (float)((c[i] >> (2 * s)) & 3) - minimum;
                }
    } break;
    case KO_Q3K: {                                        /* :585-600 */
        const uint8_t *mask = block, *codes = block + 32, *packed = block + 96;
        float d = half32(block, 108);
        for (int i = 0; i < 16; i++) {
            int low6 = (packed[i % 8] >> (4 * (i / 8))) & 0x0f;
            int high6 = (packed[8 + i % 4] >> (2 * (i / 4))) & 0x03;
            float scale = d * (float)((int)(int8_t)(uint8_t)(low6 | (high6 << 4)) - 32);
            int h = i / 8, s = i % 8 / 2, part = i % 2;
            for (int l = part * 16; l < part * 16 + 16; l++) {
                int low = (codes[h * 32 + l] >> (2 * s)) & 3;
                int high = ((mask[l] >> (h * 4 + s)) & 1) ^ 1;
                out[16 * i + l - part * 16] = scale * (float)(low - 4 * high);
            }
        }
    } break;
    case KO_Q4K: {                                        /* :618-636 */
        float scale[8], minimum[8];
        k_scales32(block, scale, minimum);
        const uint8_t *codes = block + 16;
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                uint8_t byte = codes[c * 32 + l];
                out[c * 64 + l] = scale[2 * c] * (float)(byte & 0x0f) - minimum[2 * c];
                out[c * 64 + 32 + l] = scale[2 * c + 1] * (float)(byte >> 4) - minimum[2 * c + 1];
            }
    } break;
    case KO_Q5K: {                                        /* :638-659 */
        float scale[8], minimum[8];
        k_scales32(block, scale, minimum);
        const uint8_t *high = block + 16, *codes = block + 48;
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                uint8_t byte = codes[c * 32 + l], h = high[l];
                uint8_t q0 = (byte & 0x0f) | (((h >> (2 * c)) & 1) << 4);
                uint8_t q1 = (byte >> 4) | (((h >> (2 * c + 1)) & 1) << 4);
                out[c * 64 + l] = scale[2 * c] * (float)q0 - minimum[2 * c];
                out[c * 64 + 32 + l] = scale[2 * c + 1] * (float)q1 - minimum[2 * c + 1];
            }
    } break;
    case KO_Q6K: {                                        /* :661-682 */
        const uint8_t *low = block, *high = block + 128, *scales = block + 192;
        float d = half32(block, 208);
        for (int h = 0; h < 2; h++)
            for (int s = 0; s < 4; s++) {
                int at = h * 128 + s * 32;
                float scale0 = d * (float)(int8_t)scales[at / 16];
                float scale1 = d * (float)(int8_t)scales[at / 16 + 1];
                for (int l = 0; l < 32; l++) {
                    int ql = (low[h * 64 + (s % 2) * 32 + l] >> (4 * (s / 2))) & 0x0f;
                    int qh = (high[h * 32 + l] >> (2 * s)) & 0x03;
                    float q = (float)(ql | (qh << 4)) - 32.0f;
                    out[at + l] = (l < 16 ? scale0 : scale1) * q;
                }
            }
    } break;
    default: return -1;
    }
    return 0;
}

/* ---------------------------------------------------------------------- */
/* Product with f32 activations: quantized.rs:87-175 (tasks, product),     */
/* :261-318 (products, reduce).  FMA as the reference's `fma::<true>`.     */
/* ---------------------------------------------------------------------- */

#define LANES 16
#define MIN_TASK_ROWS 8
#define TASKS_PER_THREAD 4
#define TASK_BYTES (128 << 10)

typedef struct {
    int fmt, group;
    const uint8_t *bytes;
    int64_t n;
} ko_weights;

typedef struct { int matrix; int64_t first, count, column; } ko_task;

/* quantized.rs:87-108 */
static ko_task *make_tasks(int threads, const ko_weights *w, int count, int64_t k, int64_t *ntasks) {
    int64_t total = 0;
    for (int i = 0; i < count; i++) {
        int len = ko_block_len(w[i].fmt, w[i].group), size = ko_block_bytes(w[i].fmt, w[i].group);
        total += w[i].n * (k / len) * size;
    }
    int64_t target = (total + threads * TASKS_PER_THREAD - 1) / (threads * TASKS_PER_THREAD);
    if (target < 1) target = 1;
    if (target > TASK_BYTES) target = TASK_BYTES;
    int64_t cap = 0;
    for (int i = 0; i < count; i++) cap += w[i].n + 1;
    ko_task *tasks = malloc(sizeof(ko_task) * (cap + 1));
    int64_t nt = 0, column = 0;
    for (int i = 0; i < count; i++) {
        int len = ko_block_len(w[i].fmt, w[i].group), size = ko_block_bytes(w[i].fmt, w[i].group);
        int64_t row_bytes = (k / len) * size;
        if (row_bytes < 1) row_bytes = 1;
        int64_t chunk = (target + row_bytes - 1) / row_bytes;
        if (chunk < MIN_TASK_ROWS) chunk = MIN_TASK_ROWS;
        for (int64_t first = 0; first < w[i].n; first += chunk) {
            tasks[nt].matrix = i;
            tasks[nt].first = first;
            tasks[nt].count = chunk < w[i].n - first ? chunk : w[i].n - first;
            tasks[nt].column = column + first;
            nt++;
        }
        column += w[i].n;
    }
    *ntasks = nt;
    return tasks;
}

/* quantized.rs:309-318 */
static float reduce16(float *sums) {
    for (int width = LANES; width > 1;) {
        width /= 2;
        for (int i = 0; i < width; i++) sums[i] += sums[i + width];
    }
    return sums[0];
}

/* quantized.rs:261-305: out[r*count + j] for R rows of x, one task's rows. */
static void products(int fmt, int group, const uint8_t *w, int64_t k, const float *x, int R,
                     int64_t count, float *out, float *block) {
    int len = ko_block_len(fmt, group), bytes = ko_block_bytes(fmt, group);
    int64_t row_bytes = k / len * bytes;
    float acc[8][2][LANES];
    for (int64_t j = 0; j < count; j++) {
        memset(acc, 0, sizeof(acc));
        const uint8_t *row = w + j * row_bytes;
        for (int64_t b = 0; b < k / len; b++) {
            ko_decode_f32(fmt, group, row + b * bytes, block);
            int pairs = len / (2 * LANES), rest = len % (2 * LANES);
            for (int r = 0; r < R; r++) {
                const float *xr = x + r * k + b * len;
                float *even = acc[r][0], *odd = acc[r][1];
                for (int p = 0; p < pairs; p++) {
                    const float *wp = block + p * 2 * LANES, *xp = xr + p * 2 * LANES;
                    for (int i = 0; i < LANES; i++) {
                        even[i] = fmaf(wp[i], xp[i], even[i]);
                        odd[i] = fmaf(wp[LANES + i], xp[LANES + i], odd[i]);
                    }
                }
                const float *wt = block + pairs * 2 * LANES, *xt = xr + pairs * 2 * LANES;
                for (int i = 0; i < rest; i++) even[i % LANES] = fmaf(wt[i], xt[i], even[i % LANES]);
            }
        }
        for (int r = 0; r < R; r++) {
            float sums[LANES];
            for (int i = 0; i < LANES; i++) sums[i] = acc[r][0][i] + acc[r][1][i];
            out[r * count + j] = reduce16(sums);
        }
    }
}

typedef struct {
    const ko_weights *w;
    const ko_task *tasks;
    int64_t ntasks, k, rows, width;
    const float *x;
    float *out;
    int bytes_mode;
    /* byte mode inputs */
    const int8_t *q;
    const float *scale;
    const float *sums32;
    int32_t *dots;          /* optional side output [rows, width, k / 16] */
    int64_t next;
    pthread_mutex_t lock;
} ko_job;

static void product_task(ko_job *job, const ko_task *t);
static void bytes_task(ko_job *job, const ko_task *t);

static void *worker(void *arg) {
    ko_job *job = arg;
    for (;;) {
        pthread_mutex_lock(&job->lock);
        int64_t i = job->next++;
        pthread_mutex_unlock(&job->lock);
        if (i >= job->ntasks) return NULL;
        if (job->bytes_mode) bytes_task(job, &job->tasks[i]);
        else product_task(job, &job->tasks[i]);
    }
}

static void run_job(ko_job *job, int threads) {
    pthread_mutex_init(&job->lock, NULL);
    job->next = 0;
    if (threads <= 1) {
        worker(job);
    } else {
        pthread_t *ids = malloc(sizeof(pthread_t) * threads);
        for (int i = 0; i < threads; i++) pthread_create(&ids[i], NULL, worker, job);
        for (int i = 0; i < threads; i++) pthread_join(ids[i], NULL);
        free(ids);
    }
    pthread_mutex_destroy(&job->lock);
}

/* quantized.rs:151-174: the task's part, ROWS = 8 rows of x at a time in
 * groups of 8, 4, 2, 1 (quantized.rs:180-213). */
static void product_task(ko_job *job, const ko_task *t) {
    const ko_weights *w = &job->w[t->matrix];
    int len = ko_block_len(w->fmt, w->group), size = ko_block_bytes(w->fmt, w->group);
    int64_t k = job->k, row_bytes = k / len * size;
    const uint8_t *bytes = w->bytes + t->first * row_bytes;
    float *part = malloc(sizeof(float) * (size_t)(job->rows * t->count + 1));
    float *block = malloc(sizeof(float) * (size_t)len);
    for (int64_t first = 0; first < job->rows;) {
        int64_t left = job->rows - first;
        int R = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        products(w->fmt, w->group, bytes, k, job->x + first * k, R, t->count,
                 part + first * t->count, block);
        first += R;
    }
    for (int64_t r = 0; r < job->rows; r++)
        memcpy(job->out + r * job->width + t->column, part + r * t->count,
               sizeof(float) * (size_t)t->count);
    free(block);
    free(part);
}

/* out [rows, sum n] = x [rows, k] . [w_1; w_2; ...]^T.  Returns 0 or -1. */
int ko_product_f32(int count, const int *fmts, const int *groups, const uint8_t *const *ptrs,
                   const int64_t *ns, int64_t k, const float *x, int64_t rows, float *out,
                   int threads) {
    ko_weights w[64];
    if (count > 64) return -1;
    int64_t width = 0;
    for (int i = 0; i < count; i++) {
        w[i].fmt = fmts[i]; w[i].group = groups[i]; w[i].bytes = ptrs[i]; w[i].n = ns[i];
        int len = ko_block_len(fmts[i], groups[i]);
        if (len <= 0 || k % len) return -1;
        width += ns[i];
    }
    if (width == 0 || rows == 0) return 0;
    if (k == 0) { memset(out, 0, sizeof(float) * (size_t)(rows * width)); return 0; }
    int64_t nt;
    ko_task *tasks = make_tasks(threads < 1 ? 1 : threads, w, count, k, &nt);
    ko_job job = {.w = w, .tasks = tasks, .ntasks = nt, .k = k, .rows = rows, .width = width,
                  .x = x, .out = out, .bytes_mode = 0};
    run_job(&job, threads);
    free(tasks);
    return 0;
}

/* ---------------------------------------------------------------------- */
/* Byte activations: kapel-cpu/src/bytes.rs                                 */
/* ---------------------------------------------------------------------- */

#define BLOCK 32
#define BROWS 4

/* bytes.rs:51-77: the layout of a format in byte mode, or 0. */
int ko_bytes_layout(int fmt, int group, int *len, int *size, int *grp, int *minimum) {
    int g = group;
    switch (fmt) {
    case KO_Q8_0: *len = 32; *size = 34; *grp = 32; *minimum = 0; return 1;
    case KO_Q4_0: *len = 32; *size = 18; *grp = 32; *minimum = 1; return 1;
    case KO_Q4K: *len = 256; *size = 144; *grp = 32; *minimum = 1; return 1;
    case KO_Q5K: *len = 256; *size = 176; *grp = 32; *minimum = 1; return 1;
    case KO_Q6K: *len = 256; *size = 210; *grp = 16; *minimum = 0; return 1;
    case KO_INT8:
        if (g != 32 && g != 64 && g != 128) return 0;
        *len = g; *size = 4 + g; *grp = g; *minimum = 0; return 1;
    case KO_INT4:
        if (g != 32 && g != 64 && g != 128) return 0;
        *len = g; *size = 4 + g / 2; *grp = g; *minimum = 1; return 1;
    default: return 0;
    }
}

/* bytes.rs:144-158: q [rows*k] i8, scale [rows*k/32], and, as the pieces
 * of bytes.rs:117-131, sums32 [rows*k/32] = scale * (sum of q, as i32, as f32). */
void ko_quantize_x(const float *x, int64_t rows, int64_t k, int8_t *q, float *scale,
                   float *sums32) {
    int64_t blocks = rows * k / BLOCK;
    for (int64_t b = 0; b < blocks; b++) {
        const float *v = x + b * BLOCK;
        float max = 0.0f;
        for (int i = 0; i < BLOCK; i++) max = fmaxf(max, fabsf(v[i]));
        scale[b] = max / 127.0f;
        float inverse = max > 0.0f ? 127.0f / max : 0.0f;
        int32_t total = 0;
        for (int i = 0; i < BLOCK; i++) {
            float r = nearbyintf(v[i] * inverse); /* round half to even */
            if (isnan(r)) r = 0.0f;               /* Rust's `as i8` of NaN */
            r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
            q[b * BLOCK + i] = (int8_t)r;
            total += (int8_t)r;
        }
        if (sums32) sums32[b] = scale[b] * (float)total;
    }
}

/* bytes.rs:258-353: codes, scale[16], minimum[16] of one block. */
typedef struct { float scale[16], minimum[16]; int16_t codes[256]; } ko_decoded;

static void decode_bytes(int fmt, int group, const uint8_t *block, ko_decoded *d) {
    memset(d, 0, sizeof(*d));
    switch (fmt) {
    case KO_Q8_0:
        d->scale[0] = half32(block, 0);
        for (int i = 0; i < 32; i++) d->codes[i] = (int8_t)block[2 + i];
        break;
    case KO_Q4_0:
        d->scale[0] = half32(block, 0);
        d->minimum[0] = 8.0f * d->scale[0];
        for (int j = 0; j < 16; j++) {
            d->codes[j] = block[2 + j] & 0x0f;
            d->codes[j + 16] = block[2 + j] >> 4;
        }
        break;
    case KO_Q4K: case KO_Q5K: {
        k_scales32(block, d->scale, d->minimum);
        int five = fmt == KO_Q5K;
        const uint8_t *codes = five ? block + 48 : block + 16;
        for (int e = 0; e < 256; e++) {
            int c = e / 64, t = e % 64 / 32, l = e % 32;
            int q = (codes[c * 32 + l] >> (4 * t)) & 0x0f;
            if (five) q |= ((block[16 + l] >> (e / 32)) & 1) << 4;
            d->codes[e] = (int16_t)q;
        }
    } break;
    case KO_Q6K: {
        float dd = half32(block, 208);
        for (int i = 0; i < 16; i++) d->scale[i] = dd * (float)(int8_t)block[192 + i];
        for (int f = 0; f < 256; f++) {
            int h = f / 128, t = f % 128 / 64, m = f % 64;
            int ql = (block[h * 64 + m] >> (4 * t)) & 0x0f;
            int s = f % 128 / 32, l = f % 32;
            int qh = (block[128 + h * 32 + l] >> (2 * s)) & 0x03;
            d->codes[f] = (int16_t)((ql | (qh << 4)) - 32);
        }
    } break;
    case KO_INT8:
        d->scale[0] = single32(block);
        for (int i = 0; i < group; i++) d->codes[i] = (int8_t)block[4 + i];
        break;
    case KO_INT4:
        d->scale[0] = single32(block);
        d->minimum[0] = 8.0f * d->scale[0];
        for (int i = 0; i < group / 2; i++) {
            d->codes[2 * i] = block[4 + i] & 0x0f;
            d->codes[2 * i + 1] = block[4 + i] >> 4;
        }
        break;
    }
}

/* The group sums of bytes.rs:117-131 for group g from the per-32 pieces:
 * groups of 16 lie within one block and take that block's whole-half sum
 * (computed here from q); larger groups add their pieces in order. */
static float group_sum(const ko_job *job, int64_t r, int64_t start, int g) {
    int width = g < BLOCK ? g : BLOCK;
    float sum = 0.0f;
    for (int64_t at = start; at < start + g; at += width) {
        const int8_t *piece = job->q + r * job->k + at;
        int32_t total = 0;
        for (int i = 0; i < width; i++) total += piece[i];
        sum = sum + job->scale[(r * job->k + at) / BLOCK] * (float)total;
    }
    return sum;
}

/* bytes.rs:200-241 with portable (:356-394). */
static void bytes_task(ko_job *job, const ko_task *t) {
    const ko_weights *w = &job->w[t->matrix];
    int len, size, grp, minimum;
    ko_bytes_layout(w->fmt, w->group, &len, &size, &grp, &minimum);
    int64_t k = job->k, blocks = k / len, row_bytes = blocks * size;
    const uint8_t *bytes = w->bytes + t->first * row_bytes;
    int gw = grp < BLOCK ? grp : BLOCK;
    ko_decoded d;
    for (int64_t j = 0; j < t->count; j++) {
        const uint8_t *row = bytes + j * row_bytes;
        for (int64_t r0 = 0; r0 < job->rows; r0 += BROWS) {
            int taken = job->rows - r0 < BROWS ? (int)(job->rows - r0) : BROWS;
            float acc[BROWS] = {0}, low[BROWS] = {0};
            for (int64_t b = 0; b < blocks; b++) {
                decode_bytes(w->fmt, w->group, row + b * size, &d);
                for (int rr = 0; rr < taken; rr++) {
                    int64_t r = r0 + rr;
                    const int8_t *q = job->q + r * k;
                    const float *sc = job->scale + r * (k / BLOCK);
                    for (int c = 0; c < len / BLOCK; c++) {
                        int64_t at = b * len + c * BLOCK;
                        float s = sc[at / BLOCK];
                        for (int half = 0; half < BLOCK / gw; half++) {
                            int start = c * BLOCK + half * gw;
                            int g = start / grp;
                            int32_t dot = 0;
                            for (int i = 0; i < gw; i++)
                                dot += (int32_t)d.codes[start + i] * (int32_t)q[b * len + start + i];
                            if (job->dots) {
                                int64_t col = t->column + j;
                                int64_t slot = (b * len + start) / 16;
                                job->dots[(r * job->width + col) * (k / 16) + slot] = dot;
                            }
                            acc[rr] += d.scale[g] * s * (float)dot;
                        }
                    }
                    if (minimum)
                        for (int g = 0; g < len / grp; g++)
                            low[rr] += d.minimum[g] * group_sum(job, r, b * len + g * grp, grp);
                }
            }
            for (int rr = 0; rr < taken; rr++)
                job->out[(r0 + rr) * job->width + t->column + j] = acc[rr] - low[rr];
        }
    }
}

/* Byte-activation product (bytes.rs:168-242).  q/scale from ko_quantize_x.
 * dots (optional): [rows, width, k/16] i32, each block dot at the slot of
 * its first element / 16 (a dot of 32 fills the even slot only).
 * Returns 0, or -1 if a format is not read with byte activations. */
int ko_product_bytes(int count, const int *fmts, const int *groups, const uint8_t *const *ptrs,
                     const int64_t *ns, int64_t k, const int8_t *q, const float *scale,
                     int64_t rows, float *out, int32_t *dots, int threads) {
    ko_weights w[64];
    if (count > 64) return -1;
    int64_t width = 0;
    for (int i = 0; i < count; i++) {
        int len, size, grp, minimum;
        if (!ko_bytes_layout(fmts[i], groups[i], &len, &size, &grp, &minimum)) return -1;
        if (k % len) return -1;
        w[i].fmt = fmts[i]; w[i].group = groups[i]; w[i].bytes = ptrs[i]; w[i].n = ns[i];
        width += ns[i];
    }
    if (width == 0 || rows == 0) return 0;
    if (k == 0) { memset(out, 0, sizeof(float) * (size_t)(rows * width)); return 0; }
    int64_t nt;
    ko_task *tasks = make_tasks(threads < 1 ? 1 : threads, w, count, k, &nt);
    ko_job job = {.w = w, .tasks = tasks, .ntasks = nt, .k = k, .rows = rows, .width = width,
                  .out = out, .bytes_mode = 1, .q = q, .scale = scale, .dots = dots};
    run_job(&job, threads);
    free(tasks);
    return 0;
}

/* ---------------------------------------------------------------------- */
/* f64 reference product: kapel-ref/src/matmul.rs:96-117                  */
/* ---------------------------------------------------------------------- */

int ko_product_f64(int count, const int *fmts, const int *groups, const uint8_t *const *ptrs,
                   const int64_t *ns, int64_t k, const double *x, int64_t rows, double *out) {
    int64_t width = 0;
    for (int i = 0; i < count; i++) width += ns[i];
    double *w = malloc(sizeof(double) * (size_t)(k > 0 ? k : 1));
    int64_t col = 0;
    for (int i = 0; i < count; i++) {
        int len = ko_block_len(fmts[i], groups[i]), size = ko_block_bytes(fmts[i], groups[i]);
        if (len <= 0 || k % len) { free(w); return -1; }
        int64_t row_bytes = k / len * size;
        for (int64_t j = 0; j < ns[i]; j++, col++) {
            if (k > 0) ko_dequantize(fmts[i], groups[i], ptrs[i] + j * row_bytes, k / len, w);
            for (int64_t r = 0; r < rows; r++) {
                double sum = 0.0;
                for (int64_t e = 0; e < k; e++) sum = sum + x[r * k + e] * w[e];
                out[r * width + col] = sum;
            }
        }
    }
    free(w);
    return 0;
}
