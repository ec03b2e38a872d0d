// Instances of the float many-row product (kh_mmf.h): Kapel's int8 and int4
// groups.
#include "kh_mmf.h"

namespace kh {
using namespace mm;

hipError_t mmf_groups(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    if (fmt == KH_INT8) {
        switch (group) {
        case 32: return mmf::launch_f<Int8G<32>>(a, planes, s, cols);
        case 64: return mmf::launch_f<Int8G<64>>(a, planes, s, cols);
        case 128: return mmf::launch_f<Int8G<128>>(a, planes, s, cols);
        case 256: return mmf::launch_f<Int8G<256>>(a, planes, s, cols);
        }
    } else if (fmt == KH_INT4) {
        switch (group) {
        case 32: return mmf::launch_f<Int4G<32>>(a, planes, s, cols);
        case 64: return mmf::launch_f<Int4G<64>>(a, planes, s, cols);
        case 128: return mmf::launch_f<Int4G<128>>(a, planes, s, cols);
        case 256: return mmf::launch_f<Int4G<256>>(a, planes, s, cols);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
