// Instances of the many-row product (kh_mm.h): the non-linear formats
// IQ4_NL, IQ4_XS and IQ3_S, f32 activations only.
#include "kh_mm.h"

namespace kh {

hipError_t mm_iq(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_IQ4_NL: return mm::launch_f3<mm::IQ4NL>(a, planes, s, cols);
    case KH_IQ4_XS: return mm::launch_f3<mm::IQ4XS>(a, planes, s, cols);
    case KH_IQ3_S: return mm::launch_f3<mm::IQ3S>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
