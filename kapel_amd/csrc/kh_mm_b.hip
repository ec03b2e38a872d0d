// Instances of the many-row product (kh_mm.h): the 32-element blocks, Q4_0 to Q8_0.
#include "kh_mm.h"

namespace kh {

hipError_t mm_blocks(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q8_0: return mm::launch_f<mm::Q8_0>(a, planes, s, cols);
    case KH_Q4_0: return mm::launch_f<mm::Q4_0>(a, planes, s, cols);
    case KH_Q4_1: return mm::launch_f<mm::Q4_1>(a, planes, s, cols);
    case KH_Q5_0: return mm::launch_f<mm::Q5x<false>>(a, planes, s, cols);
    case KH_Q5_1: return mm::launch_f<mm::Q5x<true>>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
