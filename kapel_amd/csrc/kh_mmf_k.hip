// Instances of the float many-row product (kh_mmf.h): Q2_K to Q6_K.
#include "kh_mmf.h"

namespace kh {
using namespace mm;

hipError_t mmf_kquants(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q4K: return mmf::launch_f<Q4K>(a, planes, s, cols);
    case KH_Q5K: return mmf::launch_f<Q5K>(a, planes, s, cols);
    case KH_Q6K: return mmf::launch_f<Q6K>(a, planes, s, cols);
    case KH_Q2K: return mmf::launch_f<Q2K>(a, planes, s, cols);
    case KH_Q3K: return mmf::launch_f<Q3K>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
