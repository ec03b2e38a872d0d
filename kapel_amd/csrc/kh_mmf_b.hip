// Instances of the float many-row product (kh_mmf.h): the blocks of 32.
#include "kh_mmf.h"

namespace kh {
using namespace mm;

hipError_t mmf_blocks(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q8_0: return mmf::launch_f<Q8_0>(a, planes, s, cols);
    case KH_Q4_0: return mmf::launch_f<Q4_0>(a, planes, s, cols);
    case KH_Q4_1: return mmf::launch_f<Q4_1>(a, planes, s, cols);
    case KH_Q5_0: return mmf::launch_f<Q5x<false>>(a, planes, s, cols);
    case KH_Q5_1: return mmf::launch_f<Q5x<true>>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
