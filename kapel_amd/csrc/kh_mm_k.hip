// Instances of the many-row product (kh_mm.h): the 256-element super-blocks, Q2_K to Q6_K.
#include "kh_mm.h"

namespace kh {

hipError_t mm_kquants(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q4K: return mm::launch_f<mm::Q4K>(a, planes, s, cols);
    case KH_Q5K: return mm::launch_f<mm::Q5K>(a, planes, s, cols);
    case KH_Q6K: return mm::launch_f<mm::Q6K>(a, planes, s, cols);
    case KH_Q2K: return mm::launch_f<mm::Q2K>(a, planes, s, cols);
    case KH_Q3K: return mm::launch_f<mm::Q3K>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
