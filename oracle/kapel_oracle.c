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
#include <immintrin.h>

/* Format codes: those of kapel-cuda-abi/src/lib.rs:167-194, plus Q2_K = 13,
 * Q3_K = 14 (the reference's ABI has no code for them). */
enum {
    KO_INT8 = 0, KO_INT4 = 1, KO_Q8_0 = 2, KO_Q4_0 = 3, KO_Q4_1 = 4,
    KO_Q5_0 = 5, KO_Q5_1 = 6, KO_Q4K = 7, KO_Q5K = 8, KO_Q6K = 9,
    KO_IQ4NL = 10, KO_IQ4XS = 11, KO_IQ3S = 12,
    KO_Q2K = 13, KO_Q3K = 14
};

/* The tables of IQ4_NL / IQ4_XS / IQ3_S (kapel-core/src/iq.rs:7-78): format
 * constants, checked against tests/golden/iq_tables.json. */
static const int8_t KO_IQ4NL_VALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
static const uint32_t KO_IQ3S_GRID[512] = {
    0x01010101u, 0x01010103u, 0x01010105u, 0x0101010bu, 0x0101010fu, 0x01010301u, 0x01010303u, 0x01010305u,
    0x01010309u, 0x0101030du, 0x01010501u, 0x01010503u, 0x0101050bu, 0x01010707u, 0x01010901u, 0x01010905u,
    0x0101090bu, 0x0101090fu, 0x01010b03u, 0x01010b07u, 0x01010d01u, 0x01010d05u, 0x01010f03u, 0x01010f09u,
    0x01010f0fu, 0x01030101u, 0x01030103u, 0x01030105u, 0x01030109u, 0x01030301u, 0x01030303u, 0x0103030bu,
    0x01030501u, 0x01030507u, 0x0103050fu, 0x01030703u, 0x0103070bu, 0x01030909u, 0x01030d03u, 0x01030d0bu,
    0x01030f05u, 0x01050101u, 0x01050103u, 0x0105010bu, 0x0105010fu, 0x01050301u, 0x01050307u, 0x0105030du,
    0x01050503u, 0x0105050bu, 0x01050701u, 0x01050709u, 0x01050905u, 0x0105090bu, 0x0105090fu, 0x01050b03u,
    0x01050b07u, 0x01050f01u, 0x01050f07u, 0x01070107u, 0x01070303u, 0x0107030bu, 0x01070501u, 0x01070505u,
    0x01070703u, 0x01070707u, 0x0107070du, 0x01070909u, 0x01070b01u, 0x01070b05u, 0x01070d0fu, 0x01070f03u,
    0x01070f0bu, 0x01090101u, 0x01090307u, 0x0109030fu, 0x01090503u, 0x01090509u, 0x01090705u, 0x01090901u,
    0x01090907u, 0x01090b03u, 0x01090f01u, 0x010b0105u, 0x010b0109u, 0x010b0501u, 0x010b0505u, 0x010b050du,
    0x010b0707u, 0x010b0903u, 0x010b090bu, 0x010b090fu, 0x010b0d0du, 0x010b0f07u, 0x010d010du, 0x010d0303u,
    0x010d0307u, 0x010d0703u, 0x010d0b05u, 0x010d0f03u, 0x010f0101u, 0x010f0105u, 0x010f0109u, 0x010f0501u,
    0x010f0505u, 0x010f050du, 0x010f0707u, 0x010f0b01u, 0x010f0b09u, 0x03010101u, 0x03010103u, 0x03010105u,
    0x03010109u, 0x03010301u, 0x03010303u, 0x03010307u, 0x0301030bu, 0x0301030fu, 0x03010501u, 0x03010505u,
    0x03010703u, 0x03010709u, 0x0301070du, 0x03010b09u, 0x03010b0du, 0x03010d03u, 0x03010f05u, 0x03030101u,
    0x03030103u, 0x03030107u, 0x0303010du, 0x03030301u, 0x03030309u, 0x03030503u, 0x03030701u, 0x03030707u,
    0x03030903u, 0x03030b01u, 0x03030b05u, 0x03030f01u, 0x03030f0du, 0x03050101u, 0x03050305u, 0x0305030bu,
    0x0305030fu, 0x03050501u, 0x03050509u, 0x03050705u, 0x03050901u, 0x03050907u, 0x03050b0bu, 0x03050d01u,
    0x03050f05u, 0x03070103u, 0x03070109u, 0x0307010fu, 0x03070301u, 0x03070307u, 0x03070503u, 0x0307050fu,
    0x03070701u, 0x03070709u, 0x03070903u, 0x03070d05u, 0x03070f01u, 0x03090107u, 0x0309010bu, 0x03090305u,
    0x03090309u, 0x03090703u, 0x03090707u, 0x03090905u, 0x0309090du, 0x03090b01u, 0x03090b09u, 0x030b0103u,
    0x030b0301u, 0x030b0307u, 0x030b0503u, 0x030b0701u, 0x030b0705u, 0x030b0b03u, 0x030d0501u, 0x030d0509u,
    0x030d050fu, 0x030d0909u, 0x030d090du, 0x030f0103u, 0x030f0107u, 0x030f0301u, 0x030f0305u, 0x030f0503u,
    0x030f070bu, 0x030f0903u, 0x030f0d05u, 0x030f0f01u, 0x05010101u, 0x05010103u, 0x05010107u, 0x0501010bu,
    0x0501010fu, 0x05010301u, 0x05010305u, 0x05010309u, 0x0501030du, 0x05010503u, 0x05010507u, 0x0501050fu,
    0x05010701u, 0x05010705u, 0x05010903u, 0x05010907u, 0x0501090bu, 0x05010b01u, 0x05010b05u, 0x05010d0fu,
    0x05010f01u, 0x05010f07u, 0x05010f0bu, 0x05030101u, 0x05030105u, 0x05030301u, 0x05030307u, 0x0503030fu,
    0x05030505u, 0x0503050bu, 0x05030703u, 0x05030709u, 0x05030905u, 0x05030b03u, 0x05050103u, 0x05050109u,
    0x0505010fu, 0x05050503u, 0x05050507u, 0x05050701u, 0x0505070fu, 0x05050903u, 0x05050b07u, 0x05050b0fu,
    0x05050f03u, 0x05050f09u, 0x05070101u, 0x05070105u, 0x0507010bu, 0x05070303u, 0x05070505u, 0x05070509u,
    0x05070703u, 0x05070707u, 0x05070905u, 0x05070b01u, 0x05070d0du, 0x05090103u, 0x0509010fu, 0x05090501u,
    0x05090507u, 0x05090705u, 0x0509070bu, 0x05090903u, 0x05090f05u, 0x05090f0bu, 0x050b0109u, 0x050b0303u,
    0x050b0505u, 0x050b070fu, 0x050b0901u, 0x050b0b07u, 0x050b0f01u, 0x050d0101u, 0x050d0105u, 0x050d010fu,
    0x050d0503u, 0x050d0b0bu, 0x050d0d03u, 0x050f010bu, 0x050f0303u, 0x050f050du, 0x050f0701u, 0x050f0907u,
    0x050f0b01u, 0x07010105u, 0x07010303u, 0x07010307u, 0x0701030bu, 0x0701030fu, 0x07010505u, 0x07010703u,
    0x07010707u, 0x0701070bu, 0x07010905u, 0x07010909u, 0x0701090fu, 0x07010b03u, 0x07010d07u, 0x07010f03u,
    0x07030103u, 0x07030107u, 0x0703010bu, 0x07030309u, 0x07030503u, 0x07030507u, 0x07030901u, 0x07030d01u,
    0x07030f05u, 0x07030f0du, 0x07050101u, 0x07050305u, 0x07050501u, 0x07050705u, 0x07050709u, 0x07050b01u,
    0x07070103u, 0x07070301u, 0x07070309u, 0x07070503u, 0x07070507u, 0x0707050fu, 0x07070701u, 0x07070903u,
    0x07070907u, 0x0707090fu, 0x07070b0bu, 0x07070f07u, 0x07090107u, 0x07090303u, 0x0709030du, 0x07090505u,
    0x07090703u, 0x07090b05u, 0x07090d01u, 0x07090d09u, 0x070b0103u, 0x070b0301u, 0x070b0305u, 0x070b050bu,
    0x070b0705u, 0x070b0909u, 0x070b0b0du, 0x070b0f07u, 0x070d030du, 0x070d0903u, 0x070f0103u, 0x070f0107u,
    0x070f0501u, 0x070f0505u, 0x070f070bu, 0x09010101u, 0x09010109u, 0x09010305u, 0x09010501u, 0x09010509u,
    0x0901050fu, 0x09010705u, 0x09010903u, 0x09010b01u, 0x09010f01u, 0x09030105u, 0x0903010fu, 0x09030303u,
    0x09030307u, 0x09030505u, 0x09030701u, 0x0903070bu, 0x09030907u, 0x09030b03u, 0x09030b0bu, 0x09050103u,
    0x09050107u, 0x09050301u, 0x0905030bu, 0x09050503u, 0x09050707u, 0x09050901u, 0x09050b0fu, 0x09050d05u,
    0x09050f01u, 0x09070109u, 0x09070303u, 0x09070307u, 0x09070501u, 0x09070505u, 0x09070703u, 0x0907070bu,
    0x09090101u, 0x09090105u, 0x09090509u, 0x0909070fu, 0x09090901u, 0x09090f03u, 0x090b010bu, 0x090b010fu,
    0x090b0503u, 0x090b0d05u, 0x090d0307u, 0x090d0709u, 0x090d0d01u, 0x090f0301u, 0x090f030bu, 0x090f0701u,
    0x090f0907u, 0x090f0b03u, 0x0b010105u, 0x0b010301u, 0x0b010309u, 0x0b010505u, 0x0b010901u, 0x0b010909u,
    0x0b01090fu, 0x0b010b05u, 0x0b010d0du, 0x0b010f09u, 0x0b030103u, 0x0b030107u, 0x0b03010bu, 0x0b030305u,
    0x0b030503u, 0x0b030705u, 0x0b030f05u, 0x0b050101u, 0x0b050303u, 0x0b050507u, 0x0b050701u, 0x0b05070du,
    0x0b050b07u, 0x0b070105u, 0x0b07010fu, 0x0b070301u, 0x0b07050fu, 0x0b070909u, 0x0b070b03u, 0x0b070d0bu,
    0x0b070f07u, 0x0b090103u, 0x0b090109u, 0x0b090501u, 0x0b090705u, 0x0b09090du, 0x0b0b0305u, 0x0b0b050du,
    0x0b0b0b03u, 0x0b0b0b07u, 0x0b0d0905u, 0x0b0f0105u, 0x0b0f0109u, 0x0b0f0505u, 0x0d010303u, 0x0d010307u,
    0x0d01030bu, 0x0d010703u, 0x0d010707u, 0x0d010d01u, 0x0d030101u, 0x0d030501u, 0x0d03050fu, 0x0d030d09u,
    0x0d050305u, 0x0d050709u, 0x0d050905u, 0x0d050b0bu, 0x0d050d05u, 0x0d050f01u, 0x0d070101u, 0x0d070309u,
    0x0d070503u, 0x0d070901u, 0x0d09050bu, 0x0d090907u, 0x0d090d05u, 0x0d0b0101u, 0x0d0b0107u, 0x0d0b0709u,
    0x0d0b0d01u, 0x0d0d010bu, 0x0d0d0901u, 0x0d0f0303u, 0x0d0f0307u, 0x0f010101u, 0x0f010109u, 0x0f01010fu,
    0x0f010501u, 0x0f010505u, 0x0f01070du, 0x0f010901u, 0x0f010b09u, 0x0f010d05u, 0x0f030105u, 0x0f030303u,
    0x0f030509u, 0x0f030907u, 0x0f03090bu, 0x0f050103u, 0x0f050109u, 0x0f050301u, 0x0f05030du, 0x0f050503u,
    0x0f050701u, 0x0f050b03u, 0x0f070105u, 0x0f070705u, 0x0f07070bu, 0x0f070b07u, 0x0f090103u, 0x0f09010bu,
    0x0f090307u, 0x0f090501u, 0x0f090b01u, 0x0f0b0505u, 0x0f0b0905u, 0x0f0d0105u, 0x0f0d0703u, 0x0f0f0101u,
};

/* The tables as the tests read them: which 0 is IQ4_NL's values, 1 the
 * IQ3_S grid; -1 past the end. */
int64_t ko_iq_table(int which, int index) {
    if (which == 0 && index >= 0 && index < 16) return KO_IQ4NL_VALUES[index];
    if (which == 1 && index >= 0 && index < 512) return KO_IQ3S_GRID[index];
    return -1;
}

/* ---------------------------------------------------------------------- */
/* Geometry: kapel-core/src/dtype.rs:140-187                                */
/* ---------------------------------------------------------------------- */

int ko_block_len(int fmt, int group) {
    switch (fmt) {
    case KO_INT8: case KO_INT4: return group;
    case KO_Q8_0: case KO_Q4_0: case KO_Q4_1: case KO_Q5_0: case KO_Q5_1: case KO_IQ4NL: return 32;
    case KO_Q2K: case KO_Q3K: case KO_Q4K: case KO_Q5K: case KO_Q6K: case KO_IQ4XS: case KO_IQ3S:
        return 256;
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
    case KO_IQ4NL: return 18;
    case KO_IQ4XS: return 136;
    case KO_IQ3S: return 110;
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
        case KO_IQ4NL: {                                  /* :470-477 */
            double d = half64(block, 0);
            for (int e = 0; e < 32; e++) {
                uint8_t byte = block[2 + e % 16];
                y[e] = d * (double)KO_IQ4NL_VALUES[e < 16 ? byte & 0x0f : byte >> 4];
            }
        } break;
        case KO_IQ4XS: {                                  /* :478-493 */
            double d = half64(block, 0);
            uint32_t high = (uint32_t)block[2] | (uint32_t)block[3] << 8;
            for (int e = 0; e < 256; e++) {
                int g = e / 32;
                int s = ((block[4 + g / 2] >> (4 * (g % 2))) & 0x0f) | (int)((high >> (2 * g)) & 3) << 4;
                uint8_t byte = block[8 + 16 * g + e % 16];
                y[e] = d * (double)(s - 32) * (double)KO_IQ4NL_VALUES[e % 32 < 16 ? byte & 0x0f : byte >> 4];
            }
        } break;
        case KO_IQ3S: {                                   /* :494-516 */
            double d = half64(block, 0);
            const uint8_t *codes = block + 2, *high = block + 66, *signs = block + 74,
                          *scales = block + 106;
            for (int e = 0; e < 256; e++) {
                int g = e / 32, l = e % 32 / 8, j = e % 8;
                double db = d * (double)(1 + 2 * ((scales[g / 2] >> (4 * (g % 2))) & 0x0f));
                int index = codes[8 * g + 2 * l + j / 4] | (((int)high[g] << (8 - 2 * l - j / 4)) & 256);
                double v = db * (double)((KO_IQ3S_GRID[index] >> (8 * (j % 4))) & 0xff);
                y[e] = (signs[4 * g + l] >> j) & 1 ? -v : v;
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
    case KO_IQ4NL: {                                      /* :420-433 */
        float scale = half32(block, 0);
        for (int j = 0; j < 16; j++) {
            out[j] = scale * (float)KO_IQ4NL_VALUES[block[2 + j] & 0x0f];
            out[j + 16] = scale * (float)KO_IQ4NL_VALUES[block[2 + j] >> 4];
        }
    } break;
    case KO_IQ4XS: {                                      /* :435-452 */
        float d = half32(block, 0);
        uint32_t high = (uint32_t)block[2] | (uint32_t)block[3] << 8;
        for (int g = 0; g < 8; g++) {
            int s = ((block[4 + g / 2] >> (4 * (g % 2))) & 0x0f) | (int)((high >> (2 * g)) & 3) << 4;
            float scale = d * (float)(s - 32);
            const uint8_t *codes = block + 8 + 16 * g;
            for (int j = 0; j < 16; j++) {
                out[32 * g + j] = scale * (float)KO_IQ4NL_VALUES[codes[j] & 0x0f];
                out[32 * g + 16 + j] = scale * (float)KO_IQ4NL_VALUES[codes[j] >> 4];
            }
        }
    } break;
    case KO_IQ3S: {                                       /* :454-485 */
        float d = half32(block, 0);
        const uint8_t *codes = block + 2, *high = block + 66, *signs = block + 74,
                      *scales = block + 106;
        for (int g = 0; g < 8; g++) {
            float db = d * (float)(1 + 2 * ((scales[g / 2] >> (4 * (g % 2))) & 0x0f));
            for (int l = 0; l < 4; l++)
                for (int half = 0; half < 2; half++) {
                    int index = codes[8 * g + 2 * l + half] | (((int)high[g] << (8 - 2 * l - half)) & 256);
                    uint32_t grid = KO_IQ3S_GRID[index];
                    for (int j = 0; j < 4; j++) {
                        int bit = 4 * half + j;
                        float m = db * (float)((grid >> (8 * j)) & 0xff);
                        out[32 * g + 8 * l + bit] = (signs[4 * g + l] >> bit) & 1 ? -m : m;
                    }
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
    int wide;               /* the AVX-512 (f32) / AVX-512 VNNI (bytes) kernels */
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
static void wide_task(ko_job *job, const ko_task *t);
static void vnni_task(ko_job *job, const ko_task *t);

static void *worker(void *arg) {
    ko_job *job = arg;
    for (;;) {
        pthread_mutex_lock(&job->lock);
        int64_t i = job->next++;
        pthread_mutex_unlock(&job->lock);
        if (i >= job->ntasks) return NULL;
        if (job->bytes_mode) (job->wide ? vnni_task : bytes_task)(job, &job->tasks[i]);
        else (job->wide ? wide_task : product_task)(job, &job->tasks[i]);
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

/* ---------------------------------------------------------------------- */
/* The AVX-512 kernels kapel-cpu runs on a processor that has them: the    */
/* timed CPU baseline.  f32 activations: quantized.rs:699-1021 (`wide`),   */
/* rows by 8, 4, 2, 1 (:711-731); bytes: bytes.rs:395-652 (`vnni`), views  */
/* of up to 4 rows (bytes.rs:38, :411-418).  Formats Q4_0, Q8_0, Q4_K and  */
/* Q6_K (the benchmark's); the tasks and the thread split are those of the */
/* portable products above.                                                 */
/* ---------------------------------------------------------------------- */

#define WIDE __attribute__((target("avx512f,avx512bw,avx512dq,avx512vl,avx2,fma")))
#define VNNI __attribute__((target("avx512f,avx512bw,avx512dq,avx512vl,avx512vnni,avx2,fma")))
#define INLINE static inline __attribute__((always_inline))

/* An f16 scale as f32 (exact), by F16C: no call in the loops. */
WIDE INLINE float w_half(const uint8_t *b, int at) {
    uint16_t h;
    memcpy(&h, b + at, 2);
    return _cvtsh_ss(h);
}

/* Bit 0: AVX-512 F/BW/DQ/VL; bit 1: also VNNI (isa.rs:20-35, bytes.rs:89). */
int ko_wide_available(void) {
    __builtin_cpu_init();
    int wide = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
               __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl") &&
               __builtin_cpu_supports("fma");
    return wide ? 1 | (__builtin_cpu_supports("avx512vnni") ? 2 : 0) : 0;
}

static int wide_format(int fmt) {
    return fmt == KO_Q4_0 || fmt == KO_Q8_0 || fmt == KO_Q4K || fmt == KO_Q6K;
}

/* quantized.rs:980-1011 */
WIDE INLINE __m128i w_bytes(const uint8_t *b) { return _mm_loadu_si128((const __m128i *)b); }
WIDE INLINE __m128i w_take(__m128i v, int shift, char mask) {
    return _mm_and_si128(_mm_srl_epi16(v, _mm_cvtsi64_si128(shift)), _mm_set1_epi8(mask));
}
WIDE INLINE __m512 w_unsigned(__m128i v) { return _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(v)); }
WIDE INLINE __m512 w_signed(__m128i v) { return _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(v)); }

/* Codes 16 s ... 16 s + 15 of a block as floats (quantized.rs:779-899). */
WIDE INLINE __m512 w_codes(int fmt, const uint8_t *b, int s) {
    switch (fmt) {
    case KO_Q8_0: return w_signed(w_bytes(b + 2 + 16 * s));
    case KO_Q4_0: return w_signed(_mm_sub_epi8(w_take(w_bytes(b + 2), 4 * s, 0x0f), _mm_set1_epi8(8)));
    case KO_Q4K: {
        int c = s / 4, high = s % 4 / 2, part = s % 2;
        return w_unsigned(w_take(w_bytes(b + 16 + c * 32 + part * 16), 4 * high, 0x0f));
    }
    default: { /* Q6_K */
        int h = s / 8, shift = s % 8 / 2, part = s % 2;
        __m128i ql = w_take(w_bytes(b + h * 64 + (shift % 2) * 32 + part * 16), 4 * (shift / 2), 0x0f);
        __m128i qh = w_take(w_bytes(b + 128 + h * 32 + part * 16), 2 * shift, 3);
        __m128i q = _mm_or_si128(ql, _mm_slli_epi16(qh, 4));
        return w_signed(_mm_sub_epi8(q, _mm_set1_epi8(32)));
    }
    }
}

/* k_scales32 (quantized.rs:603-617) with the scales converted inline. */
WIDE INLINE void w_k_scales(const uint8_t *block, float *scale, float *minimum) {
    float d = w_half(block, 0), dmin = w_half(block, 2);
    const uint8_t *sc = block + 4, *mn = block + 8, *md = block + 12;
    for (int i = 0; i < 4; i++) {
        scale[i] = d * (float)(sc[i] & 0x3f);
        minimum[i] = dmin * (float)(mn[i] & 0x3f);
        scale[4 + i] = d * (float)((md[i] & 0x0f) | ((sc[i] >> 2) & 0x30));
        minimum[4 + i] = dmin * (float)((md[i] >> 4) | ((mn[i] >> 2) & 0x30));
    }
}

/* The scales (and minimums) of a block's groups. */
WIDE INLINE void w_scales(int fmt, const uint8_t *b, float *scale, float *minimum) {
    switch (fmt) {
    case KO_Q8_0: case KO_Q4_0: scale[0] = w_half(b, 0); minimum[0] = 0.0f; break;
    case KO_Q4K: w_k_scales(b, scale, minimum); break;
    default: {
        __m512 d = _mm512_set1_ps(w_half(b, 208));
        _mm512_storeu_ps(scale, _mm512_mul_ps(w_signed(w_bytes(b + 192)), d));
    }
    }
}

/* quantized.rs:914-975: out[r * count + j] = x[r] . w[j] for R rows. */
WIDE INLINE void w_fused(int fmt, int R, const uint8_t *w, int64_t k, const float *x, int64_t count,
                         float *out) {
    const int LEN = fmt == KO_Q4K || fmt == KO_Q6K ? 256 : 32;
    const int BYTES = fmt == KO_Q8_0 ? 34 : fmt == KO_Q4_0 ? 18 : fmt == KO_Q4K ? 144 : 210;
    const int GROUP = fmt == KO_Q6K ? 16 : 32;
    const int MIN = fmt == KO_Q4K;
    const int64_t blocks = k / LEN, groups = k / GROUP;
    float *sums = NULL;
    if (MIN) {
        sums = malloc(sizeof(float) * (size_t)(R * groups));
        for (int r = 0; r < R; r++)
            for (int64_t g = 0; g < groups; g++) {
                float lanes[LANES] = {0};
                const float *v = x + r * k + g * GROUP;
                for (int i = 0; i < GROUP; i++) lanes[i % LANES] += v[i];
                sums[r * groups + g] = reduce16(lanes);
            }
    }
    float scale[16], minimum[16];
    for (int64_t j = 0; j < count; j++) {
        const uint8_t *row = w + j * blocks * BYTES;
        __m512 acc[8];
        float low[8];
        for (int r = 0; r < R; r++) { acc[r] = _mm512_setzero_ps(); low[r] = 0.0f; }
        for (int64_t b = 0; b < blocks; b++) {
            const uint8_t *block = row + b * BYTES;
            w_scales(fmt, block, scale, minimum);
#pragma GCC unroll 16
            for (int g = 0; g < LEN / GROUP; g++) {
                __m512 t[8];
                for (int r = 0; r < R; r++) t[r] = _mm512_setzero_ps();
#pragma GCC unroll 2
                for (int s = 0; s < GROUP / 16; s++) {
                    __m512 q = w_codes(fmt, block, g * GROUP / 16 + s);
                    for (int r = 0; r < R; r++) {
                        __m512 v = _mm512_loadu_ps(x + r * k + b * LEN + g * GROUP + s * 16);
                        t[r] = _mm512_fmadd_ps(q, v, t[r]);
                    }
                }
                __m512 sc = _mm512_set1_ps(scale[g]);
                for (int r = 0; r < R; r++) acc[r] = _mm512_fmadd_ps(t[r], sc, acc[r]);
                if (MIN)
                    for (int r = 0; r < R; r++) low[r] += minimum[g] * sums[r * groups + b * (LEN / GROUP) + g];
            }
        }
        for (int r = 0; r < R; r++) out[r * count + j] = _mm512_reduce_add_ps(acc[r]) - low[r];
    }
    free(sums);
}

/* One instance per format and row count, as the reference's generics. */
#define W_INST(F, R) \
    WIDE static void w_##F##_##R(const uint8_t *w, int64_t k, const float *x, int64_t n, float *o) { \
        w_fused(KO_##F, R, w, k, x, n, o); \
    }
#define W_ROWS(F) W_INST(F, 1) W_INST(F, 2) W_INST(F, 4) W_INST(F, 8)
W_ROWS(Q8_0) W_ROWS(Q4_0) W_ROWS(Q4K) W_ROWS(Q6K)

WIDE static void w_rows(int fmt, const uint8_t *w, int64_t k, const float *x, int R, int64_t count,
                        float *out) {
#define W_PICK(F) \
    (R == 8 ? w_##F##_8 : R == 4 ? w_##F##_4 : R == 2 ? w_##F##_2 : w_##F##_1)
    void (*f)(const uint8_t *, int64_t, const float *, int64_t, float *) =
        fmt == KO_Q8_0 ? W_PICK(Q8_0) : fmt == KO_Q4_0 ? W_PICK(Q4_0) : fmt == KO_Q4K ? W_PICK(Q4K) : W_PICK(Q6K);
    f(w, k, x, count, out);
#undef W_PICK
}

/* quantized.rs:151-174 with wide::rows (:711-731). */
static void wide_task(ko_job *job, const ko_task *t) {
    const ko_weights *w = &job->w[t->matrix];
    int len = ko_block_len(w->fmt, w->group), size = ko_block_bytes(w->fmt, w->group);
    int64_t k = job->k, row_bytes = k / len * size;
    const uint8_t *bytes = w->bytes + t->first * row_bytes;
    float *part = malloc(sizeof(float) * (size_t)(job->rows * t->count + 1));
    for (int64_t first = 0; first < job->rows;) {
        int64_t left = job->rows - first;
        int R = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        w_rows(w->fmt, bytes, k, job->x + first * k, R, t->count, part + first * t->count);
        first += R;
    }
    for (int64_t r = 0; r < job->rows; r++)
        memcpy(job->out + r * job->width + t->column, part + r * t->count,
               sizeof(float) * (size_t)t->count);
    free(part);
}

/* ko_product_f32 with the AVX-512 kernels.  -2: no AVX-512 here or a format
 * they do not take. */
int ko_wide_product_f32(int count, const int *fmts, const int *groups, const uint8_t *const *ptrs,
                        const int64_t *ns, int64_t k, const float *x, int64_t rows, float *out,
                        int threads) {
    ko_weights w[64];
    if (count > 64) return -1;
    if (!(ko_wide_available() & 1)) return -2;
    int64_t width = 0;
    for (int i = 0; i < count; i++) {
        if (!wide_format(fmts[i])) return -2;
        w[i].fmt = fmts[i]; w[i].group = groups[i]; w[i].bytes = ptrs[i]; w[i].n = ns[i];
        if (k % ko_block_len(fmts[i], groups[i])) return -1;
        width += ns[i];
    }
    if (width == 0 || rows == 0) return 0;
    if (k == 0) { memset(out, 0, sizeof(float) * (size_t)(rows * width)); return 0; }
    int64_t nt;
    ko_task *tasks = make_tasks(threads < 1 ? 1 : threads, w, count, k, &nt);
    ko_job job = {.w = w, .tasks = tasks, .ntasks = nt, .k = k, .rows = rows, .width = width,
                  .x = x, .out = out, .bytes_mode = 0, .wide = 1};
    run_job(&job, threads);
    free(tasks);
    return 0;
}

/* bytes.rs:420-452 */
VNNI INLINE __m256i v_load32(const void *b) { return _mm256_loadu_si256((const __m256i *)b); }
VNNI INLINE __m128i v_load16(const void *b) { return _mm_loadu_si128((const __m128i *)b); }
VNNI INLINE __m256i v_take(__m256i v, int shift, char mask) {
    return _mm256_and_si256(_mm256_srl_epi16(v, _mm_cvtsi64_si128(shift)), _mm256_set1_epi8(mask));
}
VNNI INLINE __m128i v_take16(__m128i v, int shift, char mask) {
    return _mm_and_si128(_mm_srl_epi16(v, _mm_cvtsi64_si128(shift)), _mm_set1_epi8(mask));
}
/* bytes.rs:641-648: the sum of eight lanes, pairwise. */
VNNI INLINE float v_reduce(__m256 v) {
    __m128 quad = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    __m128 pair = _mm_add_ps(quad, _mm_movehl_ps(quad, quad));
    return _mm_cvtss_f32(_mm_add_ss(pair, _mm_movehdup_ps(pair)));
}

/* Codes 32 c ... 32 c + 31 of a block as bytes (bytes.rs:488-537). */
VNNI INLINE __m256i v_codes(int fmt, const uint8_t *b, int c) {
    switch (fmt) {
    case KO_Q8_0: return v_load32(b + 2);
    case KO_Q4_0: {
        __m128i v = v_load16(b + 2);
        return _mm256_set_m128i(v_take16(v, 4, 0x0f), v_take16(v, 0, 0x0f));
    }
    case KO_Q4K: return v_take(v_load32(b + 16 + c / 2 * 32), 4 * (c % 2), 0x0f);
    default: { /* Q6_K */
        int h = c / 4, s = c % 4;
        __m256i ql = v_take(v_load32(b + h * 64 + (s % 2) * 32), 4 * (s / 2), 0x0f);
        __m256i qh = v_take(v_load32(b + 128 + h * 32), 2 * s, 3);
        return _mm256_sub_epi8(_mm256_or_si256(ql, _mm256_slli_epi16(qh, 4)), _mm256_set1_epi8(32));
    }
    }
}

VNNI INLINE void v_scales(int fmt, const uint8_t *b, float *scale, float *minimum) {
    switch (fmt) {
    case KO_Q8_0: scale[0] = w_half(b, 0); minimum[0] = 0.0f; break;
    case KO_Q4_0: scale[0] = w_half(b, 0); minimum[0] = 8.0f * scale[0]; break;
    case KO_Q4K: w_k_scales(b, scale, minimum); break;
    default: {
        __m512 s = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(v_load16(b + 192)));
        _mm512_storeu_ps(scale, _mm512_mul_ps(s, _mm512_set1_ps(w_half(b, 208))));
    }
    }
}

/* bytes.rs:557-638: R rows of byte activations (q, scale, sums32 of the
 * job, rows r0 ...), signed codes by vpdpbusd with the signs moved to the
 * activations. */
VNNI INLINE void v_fused(int fmt, int R, const uint8_t *w, const ko_job *job, int64_t r0, int64_t count,
                         float *out) {
    const int LEN = fmt == KO_Q4K || fmt == KO_Q6K ? 256 : 32;
    const int BYTES = fmt == KO_Q8_0 ? 34 : fmt == KO_Q4_0 ? 18 : fmt == KO_Q4K ? 144 : 210;
    const int GROUP = fmt == KO_Q6K ? 16 : 32;
    const int SIGNED = fmt == KO_Q8_0 || fmt == KO_Q6K, MIN = fmt == KO_Q4_0 || fmt == KO_Q4K;
    const int64_t k = job->k, blocks = k / LEN;
    float scale[16], minimum[16];
    for (int64_t j = 0; j < count; j++) {
        const uint8_t *row = w + j * blocks * BYTES;
        __m256 acc[4], lows[4];
        float low[4];
        for (int r = 0; r < R; r++) { acc[r] = lows[r] = _mm256_setzero_ps(); low[r] = 0.0f; }
        for (int64_t b = 0; b < blocks; b++) {
            const uint8_t *block = row + b * BYTES;
            v_scales(fmt, block, scale, minimum);
#pragma GCC unroll 8
            for (int c = 0; c < LEN / BLOCK; c++) {
                __m256 factor = GROUP >= BLOCK ? _mm256_set1_ps(scale[c * BLOCK / GROUP])
                                               : _mm256_set_m128(_mm_set1_ps(scale[2 * c + 1]),
                                                                 _mm_set1_ps(scale[2 * c]));
                __m256i u = v_codes(fmt, block, c), sign = _mm256_setzero_si256();
                if (SIGNED) { sign = u; u = _mm256_abs_epi8(u); }
                for (int r = 0; r < R; r++) {
                    int64_t at = b * LEN + c * BLOCK, row_at = (r0 + r) * k;
                    __m256i xq = v_load32(job->q + row_at + at);
                    if (SIGNED) xq = _mm256_sign_epi8(xq, sign);
                    __m256i dot = _mm256_dpbusd_epi32(_mm256_setzero_si256(), u, xq);
                    __m256 f = _mm256_mul_ps(factor, _mm256_set1_ps(job->scale[(row_at + at) / BLOCK]));
                    acc[r] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(dot), f, acc[r]);
                }
            }
            if (MIN && LEN / GROUP == 8) {
                __m256 m = _mm256_loadu_ps(minimum);
                for (int r = 0; r < R; r++)
                    lows[r] = _mm256_fmadd_ps(m, _mm256_loadu_ps(job->sums32 + ((r0 + r) * k) / BLOCK + b * 8),
                                              lows[r]);
            } else if (MIN) {
                for (int r = 0; r < R; r++)
                    for (int g = 0; g < LEN / GROUP; g++)
                        low[r] += minimum[g] * job->sums32[((r0 + r) * k) / BLOCK + b * (LEN / GROUP) + g];
            }
        }
        for (int r = 0; r < R; r++) out[r * count + j] = v_reduce(acc[r]) - (low[r] + v_reduce(lows[r]));
    }
}

#define V_INST(F, R) \
    VNNI static void v_##F##_##R(const uint8_t *w, const ko_job *j, int64_t r0, int64_t n, float *o) { \
        v_fused(KO_##F, R, w, j, r0, n, o); \
    }
#define V_ROWS(F) V_INST(F, 1) V_INST(F, 2) V_INST(F, 3) V_INST(F, 4)
V_ROWS(Q8_0) V_ROWS(Q4_0) V_ROWS(Q4K) V_ROWS(Q6K)

/* bytes.rs:200-241 with vnni::rows (:411-418). */
static void vnni_task(ko_job *job, const ko_task *t) {
    const ko_weights *w = &job->w[t->matrix];
    int len = ko_block_len(w->fmt, w->group), size = ko_block_bytes(w->fmt, w->group);
    int64_t k = job->k, row_bytes = k / len * size;
    const uint8_t *bytes = w->bytes + t->first * row_bytes;
    float *part = malloc(sizeof(float) * (size_t)(job->rows * t->count + 1));
#define V_PICK(F) \
    (R == 4 ? v_##F##_4 : R == 3 ? v_##F##_3 : R == 2 ? v_##F##_2 : v_##F##_1)
    for (int64_t r0 = 0; r0 < job->rows; r0 += BROWS) {
        int R = job->rows - r0 < BROWS ? (int)(job->rows - r0) : BROWS;
        void (*f)(const uint8_t *, const ko_job *, int64_t, int64_t, float *) =
            w->fmt == KO_Q8_0 ? V_PICK(Q8_0) : w->fmt == KO_Q4_0 ? V_PICK(Q4_0)
                              : w->fmt == KO_Q4K ? V_PICK(Q4K) : V_PICK(Q6K);
        f(bytes, job, r0, t->count, part + r0 * t->count);
    }
#undef V_PICK
    for (int64_t r = 0; r < job->rows; r++)
        memcpy(job->out + r * job->width + t->column, part + r * t->count,
               sizeof(float) * (size_t)t->count);
    free(part);
}

/* ko_product_bytes with the VNNI kernels; sums32 as ko_quantize_x writes
 * them.  -2: no AVX-512 VNNI here or a format they do not take. */
int ko_vnni_product_bytes(int count, const int *fmts, const int *groups, const uint8_t *const *ptrs,
                          const int64_t *ns, int64_t k, const int8_t *q, const float *scale,
                          const float *sums32, int64_t rows, float *out, int threads) {
    ko_weights w[64];
    if (count > 64) return -1;
    if (!(ko_wide_available() & 2)) return -2;
    int64_t width = 0;
    for (int i = 0; i < count; i++) {
        if (!wide_format(fmts[i])) return -2;
        if (k % ko_block_len(fmts[i], groups[i])) return -1;
        w[i].fmt = fmts[i]; w[i].group = groups[i]; w[i].bytes = ptrs[i]; w[i].n = ns[i];
        width += ns[i];
    }
    if (width == 0 || rows == 0) return 0;
    if (k == 0) { memset(out, 0, sizeof(float) * (size_t)(rows * width)); return 0; }
    int64_t nt;
    ko_task *tasks = make_tasks(threads < 1 ? 1 : threads, w, count, k, &nt);
    ko_job job = {.w = w, .tasks = tasks, .ntasks = nt, .k = k, .rows = rows, .width = width,
                  .out = out, .bytes_mode = 1, .wide = 1, .q = q, .scale = scale, .sums32 = sums32};
    run_job(&job, threads);
    free(tasks);
    return 0;
}
