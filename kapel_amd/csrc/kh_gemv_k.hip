// Instances of the small-M product (kh_gemv.h): the 256-element super-blocks, Q2_K to Q6_K.
#include "kh_gemv.h"

namespace kh {
using namespace lanes;

hipError_t gemv_kquants(uint32_t fmt, int planes, const GemvArgs &a, hipStream_t s) {
    if (planes == 1) {
        switch (fmt) {
        case KH_Q4K: return launch_f<Q4K, 1>(a, s);
        case KH_Q5K: return launch_f<Q5K, 1>(a, s);
        case KH_Q6K: return launch_f<Q6K, 1>(a, s);
        }
        return hipErrorInvalidValue;
    }
    switch (fmt) {
    case KH_Q4K: return launch_f<Q4K, 3>(a, s);
    case KH_Q5K: return launch_f<Q5K, 3>(a, s);
    case KH_Q6K: return launch_f<Q6K, 3>(a, s);
    case KH_Q2K: return launch_f<Q2K, 3>(a, s);
    case KH_Q3K: return launch_f<Q3K, 3>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
