// Host quantization at load time: the bytes the device kernels read.
//
// int8, int4, Q8_0, Q4_0 and Q4_1 follow the reference's quantizers
// (kapel-core/src/dtype.rs:565-841): the same scale rules, the same f32/f64
// arithmetic and roundings, so that a model quantized here holds the bytes
// Kapel writes.  Q5_0, Q5_1 and the K formats (Q2_K ... Q6_K) are not written
// by the reference (dtype.rs:546-556; they come from GGUF files there): their
// encoders here are this library's own round-to-nearest ones, valid blocks of
// the GGUF layouts that kapel-core/src/dtype.rs:392-469 decodes.
//
// Built with -ffp-contract=off: no multiply-add is fused unless written so.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/kapel_hip.h"

namespace {

// IEEE binary16 encoding, round to nearest even (kapel-core/src/float.rs:111).
uint16_t f16_bits(double x) {
    if (std::isnan(x)) return 0x7e00;
    uint16_t sign = std::signbit(x) ? 0x8000 : 0;
    double a = std::fabs(x);
    if (std::isinf(a)) return sign | 0x7c00;
    if (a == 0.0) return sign;
    int e2 = 0;
    std::frexp(a, &e2);
    int exponent = e2 - 1;
    if (exponent < -14) return sign | (uint16_t)std::nearbyint(std::ldexp(a, 24));
    uint32_t significand = (uint32_t)std::nearbyint(std::ldexp(a, 10 - exponent));
    if (significand == 2048u) {
        significand = 1024u;
        exponent += 1;
    }
    int field = exponent + 15;
    if (field >= 31) return sign | 0x7c00;
    return sign | (uint16_t)((field << 10) | (significand & 0x3ff));
}

double f16_value(uint16_t bits) {
    int exponent = (bits >> 10) & 0x1f, mantissa = bits & 0x3ff;
    double sign = (bits & 0x8000) ? -1.0 : 1.0;
    if (exponent == 0x1f) return mantissa ? NAN : sign * INFINITY;
    if (exponent == 0) return sign * std::ldexp((double)mantissa, -24);
    return sign * std::ldexp((double)(1024 + mantissa), exponent - 25);
}

void put16(uint8_t *at, uint16_t v) {
    at[0] = (uint8_t)(v & 0xff);
    at[1] = (uint8_t)(v >> 8);
}

float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
double clampd(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }

// The value of largest magnitude, with its sign, the first of ties
// (dtype.rs:618-620).
float signed_extreme(const float *x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++)
        if (std::fabs(x[i]) > std::fabs(m)) m = x[i];
    return m;
}

// ---------------------------------------------------------------- reference
// Kapel int8 (dtype.rs:588-596, :641-643): f64 scale amax / 127 rounded to f32;
// codes round-half-away(x / scale) in f64.
void encode_int8(const float *x, int g, uint8_t *out) {
    double amax = 0.0;
    for (int i = 0; i < g; i++) amax = std::fmax(amax, std::fabs((double)x[i]));
    float step32 = (float)(amax / 127.0);
    double step = step32, inv = step != 0.0 ? 1.0 / step : 0.0;
    std::memcpy(out, &step32, 4);
    for (int i = 0; i < g; i++) {
        double r = clampd(std::round((double)x[i] * inv), -127.0, 127.0);
        out[4 + i] = (uint8_t)(int8_t)r;
    }
}

// Kapel int4 (dtype.rs:789-841): among the scales that put the extreme at
// level -8 .. 7 by twentieths, and the least-squares refits of their codes,
// the one of least squared error (the first of equals).
void encode_int4(const float *x, int g, uint8_t *out) {
    std::vector<uint8_t> best(g, 8), trial(g), fit_codes(g);
    float best_scale = 0.0f;
    double best_err = INFINITY;
    float m = signed_extreme(x, g);
    auto codes_for = [&](double scale, std::vector<uint8_t> &c) {
        for (int i = 0; i < g; i++) {
            double r = std::isfinite(scale) && scale != 0.0 ? std::round((double)x[i] / scale) : 0.0;
            c[i] = (uint8_t)(clampd(r, -8.0, 7.0) + 8.0);
        }
    };
    auto error_of = [&](float scale, const std::vector<uint8_t> &c) {
        double e = 0.0;
        for (int i = 0; i < g; i++) {
            double d = (double)x[i] - (double)scale * ((double)c[i] - 8.0);
            e = e + d * d;
        }
        return e;
    };
    if (m != 0.0f) {
        for (int step = 0; step <= 20; step++) {
            double levels = -8.0 + 15.0 * (double)step / 20.0;
            if (std::fabs(levels) < 6.5) continue;
            double scale = (double)m / levels;
            codes_for(scale, trial);
            double num = 0.0, den = 0.0;
            for (int i = 0; i < g; i++) {
                double c = (double)trial[i] - 8.0;
                num = num + (double)x[i] * c;
                den = den + c * c;
            }
            double fit = num / den;
            codes_for(fit, fit_codes);
            const double cand[2] = {scale, fit};
            const std::vector<uint8_t> *cc[2] = {&trial, &fit_codes};
            for (int p = 0; p < 2; p++) {
                float s = (float)cand[p];
                if (!(std::isfinite(s) && s != 0.0f)) continue;
                double e = error_of(s, *cc[p]);
                if (e < best_err) {
                    best_err = e;
                    best_scale = s;
                    best = *cc[p];
                }
            }
        }
    }
    std::memcpy(out, &best_scale, 4);
    for (int i = 0; i < g / 2; i++) out[4 + i] = (uint8_t)(best[2 * i] | (best[2 * i + 1] << 4));
}

// GGUF Q8_0 (dtype.rs:607-615): f32 d = amax / 127, codes round(x * (1/d)).
void encode_q8_0(const float *x, uint8_t *out) {
    double amax = 0.0;
    for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs((double)x[i]));
    float d = (float)amax / 127.0f;
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, f16_bits(d));
    for (int i = 0; i < 32; i++) {
        float r = std::round(x[i] * inv);
        if (std::isnan(r)) r = 0.0f;
        out[2 + i] = (uint8_t)(int8_t)clampf(r, -127.0f, 127.0f);
    }
}

// GGUF Q4_0 (dtype.rs:616-627, :652): d = extreme / -8 (f32), codes
// floor(x * (1/d) + 8.5) in 0..15, the inverse of d before its rounding.
void encode_q4_0(const float *x, uint8_t *out) {
    float d = signed_extreme(x, 32) / -8.0f;
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, f16_bits(d));
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        float t = x[i] * inv;
        float r = std::floor(t + 8.5f);
        if (std::isnan(r)) r = 0.0f;
        q[i] = (uint8_t)clampf(r, 0.0f, 15.0f);
    }
    for (int j = 0; j < 16; j++) out[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

// GGUF Q4_1 (dtype.rs:628-639, :653-655): from the minimum in 15 steps.
void encode_q4_1(const float *x, uint8_t *out) {
    float lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < 32; i++) {
        lo = std::fmin(lo, x[i]);
        hi = std::fmax(hi, x[i]);
    }
    float d = (hi - lo) / 15.0f;
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, f16_bits(d));
    put16(out + 2, f16_bits(lo));
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        float t = (x[i] - lo) * inv;
        float r = std::floor(t + 0.5f);
        if (std::isnan(r)) r = 0.0f;
        q[i] = (uint8_t)clampf(r, 0.0f, 15.0f);
    }
    for (int j = 0; j < 16; j++) out[4 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

// ---------------------------------------------------------------- this library's
// Q5_0: as Q4_0 with 32 levels (d = extreme / -16); Q5_1: as Q4_1 with 31 steps.
void encode_q5(const float *x, uint8_t *out, bool with_min) {
    uint8_t q[32];
    float d, lo = 0.0f;
    if (with_min) {
        float hi = -INFINITY;
        lo = INFINITY;
        for (int i = 0; i < 32; i++) {
            lo = std::fmin(lo, x[i]);
            hi = std::fmax(hi, x[i]);
        }
        d = (hi - lo) / 31.0f;
    } else {
        d = signed_extreme(x, 32) / -16.0f;
    }
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) {
        float r = with_min ? std::floor((x[i] - lo) * inv + 0.5f) : std::floor(x[i] * inv + 16.5f);
        if (std::isnan(r)) r = 0.0f;
        q[i] = (uint8_t)clampf(r, 0.0f, 31.0f);
    }
    put16(out, f16_bits(d));
    uint8_t *rest = out + 2;
    if (with_min) {
        put16(out + 2, f16_bits(lo));
        rest = out + 4;
    }
    uint32_t high = 0;
    for (int j = 0; j < 32; j++) high |= (uint32_t)((q[j] >> 4) & 1) << j;
    std::memcpy(rest, &high, 4);
    for (int j = 0; j < 16; j++) rest[4 + j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

// A sub-scale of `bits` bits for `value` relative to the block's `step`.
int sub_scale(double value, double step, int top) {
    if (step == 0.0) return 0;
    return (int)clampd(std::nearbyint(value / step), 0.0, (double)top);
}

// Q4_K / Q5_K: per sub-block of 32, the range [min(0, lo), hi] in 2^b - 1
// steps; 6-bit scales of d, 6-bit minimums of dmin.
void encode_q45_k(const float *x, uint8_t *out, bool five) {
    const int levels = five ? 31 : 15;
    double scale[8], minimum[8], smax = 0.0, mmax = 0.0;
    for (int j = 0; j < 8; j++) {
        double lo = 0.0, hi = 0.0;
        for (int i = 0; i < 32; i++) {
            lo = std::fmin(lo, (double)x[32 * j + i]);
            hi = std::fmax(hi, (double)x[32 * j + i]);
        }
        scale[j] = (hi - lo) / levels;
        minimum[j] = -lo;
        smax = std::fmax(smax, scale[j]);
        mmax = std::fmax(mmax, minimum[j]);
    }
    uint16_t dbits = f16_bits(smax / 63.0), mbits = f16_bits(mmax / 63.0);
    double d = f16_value(dbits), dmin = f16_value(mbits);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = sub_scale(scale[j], d, 63);
        mn[j] = sub_scale(minimum[j], dmin, 63);
    }
    put16(out, dbits);
    put16(out + 2, mbits);
    uint8_t *packed = out + 4;
    for (int j = 0; j < 4; j++) {
        packed[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        packed[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        packed[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        double s = d * sc[j], m = dmin * mn[j];
        for (int i = 0; i < 32; i++) {
            double r = s != 0.0 ? std::nearbyint(((double)x[32 * j + i] + m) / s) : 0.0;
            q[32 * j + i] = (uint8_t)clampd(r, 0.0, (double)levels);
        }
    }
    uint8_t *high = five ? out + 16 : nullptr;
    uint8_t *codes = five ? out + 48 : out + 16;
    if (high) std::memset(high, 0, 32);
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            uint8_t a = q[64 * c + l], b = q[64 * c + 32 + l];
            codes[32 * c + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
            if (high) high[l] |= (uint8_t)(((a >> 4) << (2 * c)) | ((b >> 4) << (2 * c + 1)));
        }
}

// Q6_K: per group of 16, scale amax / 32 (codes -32..31), signed 8-bit
// sub-scales of d = the largest / 127.
void encode_q6_k(const float *x, uint8_t *out) {
    double scale[16], smax = 0.0;
    for (int g = 0; g < 16; g++) {
        double amax = 0.0;
        for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs((double)x[16 * g + i]));
        scale[g] = amax / 32.0;
        smax = std::fmax(smax, scale[g]);
    }
    uint16_t dbits = f16_bits(smax / 127.0);
    double d = f16_value(dbits);
    int8_t sc[16];
    int q[256];
    for (int g = 0; g < 16; g++) {
        sc[g] = (int8_t)sub_scale(scale[g], d, 127);
        double s = d * sc[g];
        for (int i = 0; i < 16; i++) {
            double r = s != 0.0 ? std::nearbyint((double)x[16 * g + i] / s) : 0.0;
            q[16 * g + i] = (int)clampd(r, -32.0, 31.0) + 32;
        }
    }
    uint8_t *ql = out, *qh = out + 128, *scales = out + 192;
    std::memset(out, 0, 192);
    for (int f = 0; f < 256; f++) {
        int h = f / 128, t = f % 128 / 64, m = f % 64, s = f % 128 / 32, l = f % 32;
        ql[h * 64 + m] |= (uint8_t)((q[f] & 15) << (4 * t));
        qh[h * 32 + l] |= (uint8_t)(((q[f] >> 4) & 3) << (2 * s));
    }
    for (int g = 0; g < 16; g++) scales[g] = (uint8_t)sc[g];
    put16(out + 208, dbits);
}

// Q2_K: per group of 16, the range [min(0, lo), hi] in 3 steps; 4-bit scales
// of d and 4-bit minimums of dmin.
void encode_q2_k(const float *x, uint8_t *out) {
    double scale[16], minimum[16], smax = 0.0, mmax = 0.0;
    for (int g = 0; g < 16; g++) {
        double lo = 0.0, hi = 0.0;
        for (int i = 0; i < 16; i++) {
            lo = std::fmin(lo, (double)x[16 * g + i]);
            hi = std::fmax(hi, (double)x[16 * g + i]);
        }
        scale[g] = (hi - lo) / 3.0;
        minimum[g] = -lo;
        smax = std::fmax(smax, scale[g]);
        mmax = std::fmax(mmax, minimum[g]);
    }
    uint16_t dbits = f16_bits(smax / 15.0), mbits = f16_bits(mmax / 15.0);
    double d = f16_value(dbits), dmin = f16_value(mbits);
    uint8_t *scales = out, *qs = out + 16;
    std::memset(qs, 0, 64);
    for (int g = 0; g < 16; g++) {
        int sc = sub_scale(scale[g], d, 15), mn = sub_scale(minimum[g], dmin, 15);
        scales[g] = (uint8_t)(sc | (mn << 4));
        double s = d * sc, m = dmin * mn;
        for (int i = 0; i < 16; i++) {
            int e = 16 * g + i;
            double r = s != 0.0 ? std::nearbyint(((double)x[e] + m) / s) : 0.0;
            int q = (int)clampd(r, 0.0, 3.0);
            int h = e / 128, sh = e % 128 / 32, l = e % 32;
            qs[h * 32 + l] |= (uint8_t)(q << (2 * sh));
        }
    }
    put16(out + 80, dbits);
    put16(out + 82, mbits);
}

// Q3_K: per group of 16, scale amax / 4 (codes -4..3), signed 6-bit
// sub-scales of d = the largest / 31.
void encode_q3_k(const float *x, uint8_t *out) {
    double scale[16], smax = 0.0;
    for (int g = 0; g < 16; g++) {
        double amax = 0.0;
        for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs((double)x[16 * g + i]));
        scale[g] = amax / 4.0;
        smax = std::fmax(smax, scale[g]);
    }
    uint16_t dbits = f16_bits(smax / 31.0);
    double d = f16_value(dbits);
    uint8_t *mask = out, *qs = out + 32, *packed = out + 96;
    std::memset(out, 0, 108);
    for (int g = 0; g < 16; g++) {
        int sc = sub_scale(scale[g], d, 31);
        int v = sc + 32;  // stored with an offset of 32
        packed[g % 8] |= (uint8_t)((v & 15) << (4 * (g / 8)));
        packed[8 + g % 4] |= (uint8_t)(((v >> 4) & 3) << (2 * (g / 4)));
        double s = d * sc;
        for (int i = 0; i < 16; i++) {
            int e = 16 * g + i;
            double r = s != 0.0 ? std::nearbyint((double)x[e] / s) : 0.0;
            int u = (int)clampd(r, -4.0, 3.0) + 4;
            int h = e / 128, sh = e % 128 / 32, l = e % 32;
            qs[h * 32 + l] |= (uint8_t)((u & 3) << (2 * sh));
            mask[l] |= (uint8_t)(((u >> 2) & 1) << (e / 32));
        }
    }
    put16(out + 108, dbits);
}

}  // namespace

extern "C" int64_t kh_quantize_host(uint32_t format, uint32_t group, const float *values,
                                     uint64_t count, uint8_t *out, int threads) {
    uint32_t len = kh_block_len(format, group), size = kh_block_bytes(format, group);
    if (len == 0 || size == 0) return -KH_ERR_DTYPE;
    // The non-linear formats have no encoder (dtype.rs:547-556 writes none).
    if (format == KH_IQ4_NL || format == KH_IQ4_XS || format == KH_IQ3_S) return -KH_ERR_DTYPE;
    if (count % len) return -KH_ERR_MISALIGNED;
    if (!values || !out) return count == 0 ? 0 : -KH_ERR_NULL;
    uint64_t blocks = count / len;
    auto one = [&](uint64_t b) {
        const float *x = values + b * len;
        uint8_t *o = out + b * size;
        switch (format) {
        case KH_INT8: encode_int8(x, (int)group, o); break;
        case KH_INT4: encode_int4(x, (int)group, o); break;
        case KH_Q8_0: encode_q8_0(x, o); break;
        case KH_Q4_0: encode_q4_0(x, o); break;
        case KH_Q4_1: encode_q4_1(x, o); break;
        case KH_Q5_0: encode_q5(x, o, false); break;
        case KH_Q5_1: encode_q5(x, o, true); break;
        case KH_Q4K: encode_q45_k(x, o, false); break;
        case KH_Q5K: encode_q45_k(x, o, true); break;
        case KH_Q6K: encode_q6_k(x, o); break;
        case KH_Q2K: encode_q2_k(x, o); break;
        case KH_Q3K: encode_q3_k(x, o); break;
        }
    };
    int t = threads < 1 ? 1 : threads;
    if (t == 1 || blocks < 1024) {
        for (uint64_t b = 0; b < blocks; b++) one(b);
    } else {
        std::vector<std::thread> pool;
        for (int i = 0; i < t; i++)
            pool.emplace_back([&, i] {
                for (uint64_t b = (uint64_t)i * blocks / t; b < (uint64_t)(i + 1) * blocks / t; b++)
                    one(b);
            });
        for (auto &th : pool) th.join();
    }
    return (int64_t)(blocks * size);
}
