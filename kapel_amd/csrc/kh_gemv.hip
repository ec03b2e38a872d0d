// The small-M product's entry points: shapes of its launches and the kernel
// of each format.  The kernels themselves are in kh_gemv.h, instantiated by
// format family in kh_gemv_k.hip, kh_gemv_b.hip, kh_gemv_i.hip and kh_gemv_q.hip.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kh_internal.h"

namespace kh {

hipError_t gemv_kquants(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s);
hipError_t gemv_blocks(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s);
hipError_t gemv_groups(uint32_t fmt, uint32_t group, int planes, const GemvArgs &a, hipStream_t s);
hipError_t gemv_iq(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s);

int gemv_max_waves(int planes, int rows) {
    return planes == 3 && rows == 1 ? 16 : 8;
}

int gemv_unit(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K: case KH_IQ4_XS: case KH_IQ3_S:
        return 256;
    case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0: case KH_IQ4_NL: return 128;
    case KH_INT8: case KH_INT4:
        return (group == 32 || group == 64 || group == 128 || group == 256) ? 128 : 0;
    default: return 0;
    }
}

size_t gemv_lds(int rows, int planes, int chunk, int unit, int waves) {
    size_t span = (size_t)chunk * unit;
    return 16 + (size_t)rows * planes * span + span + (size_t)rows * (span / 32) * 16 +
           (size_t)waves * 16 * rows * 4;
}

size_t gemv2_lds(int rows, int planes, int units, int unit, int tiles, int kw, int tb) {
    size_t span = (size_t)units * unit;
    size_t head = 16 + (size_t)rows * planes * span + span + (size_t)rows * (span / 32) * 16 +
                  (size_t)kw * tiles * 16 * rows * 4;
    return (head + 15) / 16 * 16 + (size_t)kw * tb * 1024;
}

size_t gemv4_lds(int rows, int planes, int units, int unit, int tiles, int ks, int tb) {
    size_t span = (size_t)units * unit;
    size_t head = 16 + (size_t)rows * planes * span + span + (size_t)rows * (span / 32) * 16 +
                  (size_t)tiles * ks * 16 * rows * 4;
    return (head + 15) / 16 * 16 + (size_t)tiles * ks * tb * 1024;
}

hipError_t launch_gemv(uint32_t fmt, uint32_t group, int planes, const GemvArgs &a, hipStream_t s) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K:
        return gemv_kquants(fmt, planes, a, s);
    case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0:
        return gemv_blocks(fmt, planes, a, s);
    case KH_INT8: case KH_INT4:
        return gemv_groups(fmt, group, planes, a, s);
    case KH_IQ4_NL: case KH_IQ4_XS: case KH_IQ3_S:
        return gemv_iq(fmt, planes, a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
