// The float many-row product's entry points (kh_mmf.h): the activations as
// bf16 planes, and the kernel of each format (instantiated by format family
// in kh_mmf_k.hip, kh_mmf_b.hip, kh_mmf_i.hip and kh_mmf_q.hip).
#include "kh_mmf.h"

namespace kh {
namespace mmf {

// Eight consecutive elements a thread: k is a multiple of 32, kpad of 64.
// The planes of x, each rounded to nearest even from what the planes before
// it leave (exact: f16 in two planes, f32 in three; a plane after one that
// is not finite is zero).
__global__ __launch_bounds__(256) void prep_bf16_kernel(PrepBf16Args a) {
    const uint64_t e = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (e >= a.rows * a.kpad) return;
    const uint64_t m = e / a.kpad, k0 = e % a.kpad;
    uint32_t pl[3][4] = {};
    // x of any alignment: vector loads when it is 16-byte aligned (every row
    // then is: k is a multiple of 32), element loads otherwise.
    const bool vec = ((uintptr_t)a.x & 15u) == 0;
    if (k0 < a.k && !vec) {
        const uint64_t at = m * a.k + k0;
        for (int i = 0; i < 8; i++) {
            float r;
            if (a.x_kind == KH_F32) r = static_cast<const float *>(a.x)[at + i];
            else if (a.x_kind == KH_BF16) r = __uint_as_float((uint32_t)static_cast<const uint16_t *>(a.x)[at + i] << 16);
            else r = lanes::f16(static_cast<const uint16_t *>(a.x)[at + i]);
            for (int p = 0; p < a.planes; p++) {
                const uint32_t b = to_bf16(r);
                pl[p][i / 2] |= b << (16 * (i % 2));
                const float v = __uint_as_float(b << 16);
                r = isfinite(v) ? r - v : 0.0f;
            }
        }
    } else if (k0 < a.k) {
        const uint64_t at = m * a.k + k0;
        if (a.x_kind == KH_BF16) {
            const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.x) + at);
            pl[0][0] = v.x, pl[0][1] = v.y, pl[0][2] = v.z, pl[0][3] = v.w;
        } else {
            float f[8];
            if (a.x_kind == KH_F32) {
                const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + at);
                const float4 u = p[0], v = p[1];
                f[0] = u.x, f[1] = u.y, f[2] = u.z, f[3] = u.w, f[4] = v.x, f[5] = v.y, f[6] = v.z, f[7] = v.w;
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.x) + at);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
                for (int i = 0; i < 8; i++) f[i] = lanes::f16((w[i / 2] >> (16 * (i % 2))) & 0xffffu);
            }
            for (int i = 0; i < 8; i++) {
                float r = f[i];
                for (int p = 0; p < a.planes; p++) {
                    const uint32_t b = to_bf16(r);
                    pl[p][i / 2] |= b << (16 * (i % 2));
                    const float v = __uint_as_float(b << 16);
                    r = isfinite(v) ? r - v : 0.0f;
                }
            }
        }
    }
    uint16_t *o = a.out + (m * a.planes) * a.kpad + k0;
    for (int p = 0; p < a.planes; p++)
        *reinterpret_cast<uint4 *>(o + p * a.kpad) = uint4{pl[p][0], pl[p][1], pl[p][2], pl[p][3]};
}

}  // namespace mmf

hipError_t launch_prep_bf16(const PrepBf16Args &a, hipStream_t s) {
    const uint64_t threads = a.rows * a.kpad / 8;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(mmf::prep_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t mmf_kquants(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mmf_blocks(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mmf_groups(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t mmf_iq(uint32_t fmt, int planes, const MmArgs &a, hipStream_t s, int *cols);

hipError_t launch_mmf(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols) {
    switch (fmt) {
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K:
        return mmf_kquants(fmt, planes, a, s, cols);
    case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_Q8_0:
        return mmf_blocks(fmt, planes, a, s, cols);
    case KH_INT8: case KH_INT4:
        return mmf_groups(fmt, group, planes, a, s, cols);
    case KH_IQ4_NL: case KH_IQ4_XS: case KH_IQ3_S:
        return mmf_iq(fmt, planes, a, s, cols);
    }
    return hipErrorInvalidValue;
}

}  // namespace kh
