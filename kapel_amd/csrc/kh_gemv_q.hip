// Instances of the small-M product (kh_gemv.h): the non-linear formats
// IQ4_NL, IQ4_XS and IQ3_S, f32 activations only.
#include "kh_gemv.h"

namespace kh {
using namespace lanes;

hipError_t gemv_iq(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s) {
    if (planes != 3) return hipErrorInvalidValue;
    switch (fmt) {
    case KH_IQ4_NL: return launch_f<IQ4NL, 3>(a, s);
    case KH_IQ4_XS: return launch_f<IQ4XS, 3>(a, s);
    case KH_IQ3_S: return launch_f<IQ3S, 3>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
