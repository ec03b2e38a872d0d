// Instances of the float many-row product (kh_mmf.h): the non-linear formats.
#include "kh_mmf.h"

namespace kh {
using namespace mm;

hipError_t mmf_iq(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_IQ4_NL: return mmf::launch_f<IQ4NL>(a, planes, s, cols);
    case KH_IQ4_XS: return mmf::launch_f<IQ4XS>(a, planes, s, cols);
    case KH_IQ3_S: return mmf::launch_f<IQ3S>(a, planes, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
