// Instances of the small-M product (kh_gemv.h): the 32-element blocks, Q4_0 to Q8_0.
#include "kh_gemv.h"

namespace kh {
using namespace lanes;

hipError_t gemv_blocks(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s) {
    if (planes == 1) {
        switch (fmt) {
        case KH_Q4_0: return launch_f<Q4_0, 1>(a, s);
        case KH_Q8_0: return launch_f<Q8_0, 1>(a, s);
        }
        return hipErrorInvalidValue;
    }
    switch (fmt) {
    case KH_Q4_0: return launch_f<Q4_0, 3>(a, s);
    case KH_Q4_1: return launch_f<Q4_1, 3>(a, s);
    case KH_Q5_0: return launch_f<Q5_0, 3>(a, s);
    case KH_Q5_1: return launch_f<Q5_1, 3>(a, s);
    case KH_Q8_0: return launch_f<Q8_0, 3>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
