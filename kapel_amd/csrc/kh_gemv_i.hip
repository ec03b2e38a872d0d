// Instances of the small-M product (kh_gemv.h): Kapel's int8 and int4 groups of 32 to 256.
#include "kh_gemv.h"

namespace kh {
using namespace lanes;

hipError_t gemv_groups(uint32_t fmt, uint32_t group, int planes, const GemvArgs &a, hipStream_t s) {
    if (planes == 1) {
        if (fmt == KH_INT8) {
            if (group == 32) return launch_f<Int8G<32>, 1>(a, s);
            if (group == 64) return launch_f<Int8G<64>, 1>(a, s);
            if (group == 128) return launch_f<Int8G<128>, 1>(a, s);
        } else if (fmt == KH_INT4) {
            if (group == 32) return launch_f<Int4G<32>, 1>(a, s);
            if (group == 64) return launch_f<Int4G<64>, 1>(a, s);
            if (group == 128) return launch_f<Int4G<128>, 1>(a, s);
        }
        return hipErrorInvalidValue;
    }
    if (fmt == KH_INT8) {
        if (group == 32) return launch_f<Int8G<32>, 3>(a, s);
        if (group == 64) return launch_f<Int8G<64>, 3>(a, s);
        if (group == 128) return launch_f<Int8G<128>, 3>(a, s);
        if (group == 256) return launch_f<Int8G<256>, 3>(a, s);
    } else if (fmt == KH_INT4) {
        if (group == 32) return launch_f<Int4G<32>, 3>(a, s);
        if (group == 64) return launch_f<Int4G<64>, 3>(a, s);
        if (group == 128) return launch_f<Int4G<128>, 3>(a, s);
        if (group == 256) return launch_f<Int4G<256>, 3>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
