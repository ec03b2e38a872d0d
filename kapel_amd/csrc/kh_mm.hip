// The many-row product's entry points: the kernel of each format and the
// reduction of K splits.  The kernels are in kh_mm.h, instantiated by format
// family in kh_mm_k.hip, kh_mm_b.hip, kh_mm_i.hip and kh_mm_q.hip.
#include "kh_mm.h"

namespace kh {
namespace mm {

// The K splits of a launch, added in order (the partial sums of mm_kernel,
// [ks][rows][width]) into the output.
__global__ void mm_reduce_kernel(MmArgs a) {
    const int mat = blockIdx.y;
    const uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (uint64_t)a.rows * a.n[mat]) return;
    const uint64_t m = e / a.n[mat], col = a.col0[mat] + e % a.n[mat];
    float y = a.partials[m * a.width + col];
    for (int z = 1; z < a.ks; z++) y = y + a.partials[((uint64_t)z * a.rows + m) * a.width + col];
    store_out(a.out_kind, a.out, m * a.out_stride + col, y);
}

}  // namespace mm


hipError_t mm_kquants(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mm_blocks(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mm_groups(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mm_iq(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);

int mm_group(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q6K: return 16;
    case KH_Q4K: case KH_Q5K: case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0:
    case KH_IQ4_NL: case KH_IQ4_XS: case KH_IQ3_S:
        return 32;
    case KH_INT8: case KH_INT4:
        return (group == 32 || group == 64 || group == 128 || group == 256) ? 32 : 0;
    default: return 0;
    }
}

namespace {
hipError_t dispatch(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K:
        return mm_kquants(fmt, planes, a, s, cols);
    case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0:
        return mm_blocks(fmt, planes, a, s, cols);
    case KH_INT8: case KH_INT4:
        return mm_groups(fmt, group, planes, a, s, cols);
    case KH_IQ4_NL: case KH_IQ4_XS: case KH_IQ3_S:
        return mm_iq(fmt, planes, a, s, cols);
    }
    return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_mm(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s) {
    return dispatch(fmt, group, planes, a, s, nullptr);
}

void mm_shape(int planes, int rows, int &wm, int &wmg) { mm::shape_of(planes, rows, wm, wmg); }

int mm_cols(uint32_t fmt, uint32_t group, int planes, int rows) {
    MmArgs a{};
    mm::shape_of(planes, rows, a.wm, a.wmg);
    int cols = 0;
    return dispatch(fmt, group, planes, a, nullptr, &cols) == hipSuccess ? cols : 0;
}

int mm_unit(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K: case KH_IQ4_XS: case KH_IQ3_S:
        return 256;
    case KH_INT8: case KH_INT4: return group == 256 ? 256 : 128;
    default: return 128;
    }
}

hipError_t launch_mm_reduce(const MmArgs &a, hipStream_t s) {
    uint64_t most = 0;
    for (int i = 0; i < a.count; i++) most = a.n[i] > most ? a.n[i] : most;
    uint64_t blocks = ((uint64_t)a.rows * most + 255) / 256;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(mm::mm_reduce_kernel, dim3((unsigned)blocks, (unsigned)a.count), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace kh
