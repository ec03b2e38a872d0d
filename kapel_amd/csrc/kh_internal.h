// Internal arguments of the kernels of libkapel_hip (host and device).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "../../include/kapel_hip.h"

namespace kh {

// Activations already in bytes (kh_block_dots): the small-M product takes
// them as its plane, with scale 1.
constexpr uint32_t KH_I8_INTERNAL = 0x100u;

// Weights per launch of the product (stacked matrices of one format).
constexpr int MAX_WEIGHTS = 8;
// MFMAs per step at most: 8 x 4 slot groups with f32 activations, 8 x 16
// with byte activations (a slot group is one activation row and one group
// of weights of a step).
constexpr int MAX_MFMAS = 8;
// Slot groups of one MFMA: 4 with f32 activations (four rows of A each: the
// three planes and a zero row), 16 with byte activations (one row each).
constexpr int slot_groups_per_mfma(int planes) { return planes == 3 ? 4 : 16; }
// Segments of K at most.
constexpr int MAX_SEGS = 64;
// Counters of the segment split: at the start of every workspace, a region
// no call uses for anything else, so that the zeros each launch leaves behind
// are there for the next call whatever its shapes.
constexpr uint64_t MAX_COUNTERS = 1u << 16;
// LDS of one workgroup of the product at most.
constexpr int MAX_LDS = 64 * 1024;

// A kernel's dynamic LDS limit, raised once per device: std::call_once per
// device ordinal, so that host threads making their first calls at once do
// not race (the attribute is per device).
constexpr int MAX_DEVICES = 64;
struct OncePerDevice {
    std::once_flag flag[MAX_DEVICES];
    hipError_t err[MAX_DEVICES] = {};
};

// The current device's compute units (queried once per device).
inline int cu_count() {
    static OncePerDevice once;
    static int cus[MAX_DEVICES];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return 256;
    std::call_once(once.flag[dev], [&] {
        int n = 0;
        once.err[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        cus[dev] = once.err[dev] == hipSuccess && n > 0 ? n : 256;
    });
    return cus[dev];
}

inline hipError_t set_lds_limit(OncePerDevice &once, const void *kernel, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::call_once(once.flag[dev], [&] {
        // At most what the kernel's static LDS (as rounded up by the
        // compiler) leaves of a CU's 160 KiB.
        hipFuncAttributes at;
        once.err[dev] = hipFuncGetAttributes(&at, kernel);
        if (once.err[dev] != hipSuccess) return;
        once.err[dev] = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            std::min(bytes, 160 * 1024 - (int)at.sharedSizeBytes));
    });
    return once.err[dev];
}

struct PrepArgs {
    uint32_t x_kind;
    const void *x;        // [rows, k] floats, or NULL with q_in
    const int8_t *q_in;   // [rows, k] bytes already quantized (block dots)
    uint64_t rows, k, kpad;
    int planes;           // 1: bytes (CPU rule), 3: f32 activations
    int8_t *planes_out;   // [rows, planes, kpad] or NULL
    float *xscale;        // [rows, k/32] or NULL
    float *xsum32;        // [rows, k/32] or NULL
    float *xsum16;        // [rows, k/16] or NULL
    int32_t *xsumi16;     // [rows, k/16] or NULL
    int8_t *q_out;        // [rows, k] or NULL (kh_quantize_x)
    float *q_scale;       // [rows, k/32] or NULL
    float *q_sums;        // [rows, k/32] or NULL
};

struct QmvArgs {
    // Weights of one format, rows stacked in tiles of 16 (a tile never spans
    // two weights).
    int count;
    const uint8_t *w[MAX_WEIGHTS];
    uint64_t n[MAX_WEIGHTS];
    uint64_t col0[MAX_WEIGHTS];   // first output column of each weight
    int tile0[MAX_WEIGHTS];       // first tile of each weight in this launch
    uint64_t row_bytes;
    int k, steps, seg_steps, segs;
    int rows;                     // activation rows of this launch
    // Prepared activations of these rows.
    const int8_t *planes;
    uint64_t kpad;
    const float *xscale, *xsum32, *xsum16;
    const int32_t *xsumi16;
    // Output [rows, width] with row stride out_stride (elements).
    uint32_t out_kind;
    void *out;
    uint64_t width, out_stride;
    float *partials;              // [segs, rows, pwidth]: pwidth = 16 x tiles
    uint64_t pwidth;
    int *counters;                // [gridDim.x], zero between launches
    // Block dots instead of the product (kh_block_dots).
    int32_t *dots;
    int signed_offset;
};

// The small-M product (kh_gemv.hip): weights of one format in tiles of 16
// rows; a workgroup takes `tiles` tiles with `kw` waves each, the waves of a
// tile splitting K; K is walked in chunks of `chunk` units whose activations
// the workgroup prepares in LDS.
struct GemvArgs {
    int count;
    const uint8_t *w[MAX_WEIGHTS];
    uint32_t wbytes[MAX_WEIGHTS];  // bytes of each matrix (< 2 GiB)
    uint64_t n[MAX_WEIGHTS];
    uint64_t col0[MAX_WEIGHTS];
    int tile0[MAX_WEIGHTS];
    uint64_t row_bytes;
    int k, units, chunk;
    int total_tiles, tiles, tiles_log2, kw;  // tiles: 1, 2 or 4
    int rows;                     // activation rows of a workgroup (of a row chunk)
    int rows_total, mchunks;      // all activation rows, in mchunks chunks of `rows`
    uint32_t x_kind;
    const void *x;                // [rows_total, k], aligned to 4 elements
    uint32_t out_kind;
    void *out;                    // [rows, out_stride]
    uint64_t out_stride;
    int32_t *dots;                // block dots [rows, width, k / 16] instead of out
    uint64_t width;
    // Activations prepared beforehand (prep_x_kernel) for all rows, copied
    // instead of prepared by each workgroup; NULL: prepared in the kernel.
    const int8_t *pplanes;        // [rows_total][P][pkpad]
    uint64_t pkpad;
    const float *pxscale, *pxsum32, *pxsum16;  // [rows_total][k / 32, k / 32, k / 16]
    // The planes' digits: v = a hi + (b << shift) + c (2^16, 8).
    float hi;
    int shift;
    // The kernel with its weights staged in LDS (gemv2_kernel): `npw`
    // preparing waves, `kw` multiplying waves, `tb` copies of 1 KiB a wave.
    int dma, npw, tb;
    // The experts' product (kh_expert_matmul): a chunk of one activation
    // row is a route; its weights are expert experts[route] of the stacked
    // matrix w[0] (wbytes[0] bytes an expert), its input row route (per
    // route) or route / topk.  An expert of n_experts or more: NaN outputs.
    const uint32_t *experts;
    uint32_t n_experts;
    int topk, per_route;
    // Spins of a wave waiting for the activations in LDS before it gives up
    // (its outputs then NaN): 2^24; negative (a test of the path only):
    // give up at once.
    int spin_limit;
    // Non-NULL (the streamed kernel only): nothing is launched; the
    // workgroups of this shape that a CU holds at once are written here (0
    // when the runtime cannot tell).
    int *occupancy;
#ifdef KH_TRACE
    int *trace;
#endif
};

// The many-row product (kh_mm.h): weights of one format in column groups of
// 256 (or 128) rows; a workgroup takes one group, wmg x wm x 32 activation
// rows and one of `ks` splits of K (`ups` units each).
struct MmArgs {
    int count;
    const uint8_t *w[MAX_WEIGHTS];
    uint32_t wbytes[MAX_WEIGHTS];  // bytes of each matrix (< 2 GiB)
    uint64_t n[MAX_WEIGHTS];
    uint64_t col0[MAX_WEIGHTS];
    int ng0[MAX_WEIGHTS];          // first column group of each weight
    uint64_t row_bytes;
    int k, units, ups, ks, ngroups, mtiles;
    int wm, wmg;                   // row tiles of 32 a wave, groups of waves a workgroup
    int rows;                      // activation rows of this launch
    // Prepared activations of these rows (prep_x_kernel).
    const int8_t *planes;          // [rows][P][kpad]
    uint32_t planes_bytes;         // < 2 GiB
    uint64_t kpad;
    const float *xscale;           // [rows][k / 32]
    const float *xsum;             // [rows][k / G]: the sums of the format's groups
    float hi;                      // three planes: v = a hi + (b << shift) + c
    int shift;
    uint32_t out_kind;
    void *out;                     // [rows, out_stride]
    uint64_t out_stride, width;
    float *partials;               // [ks][rows][width] when ks > 1
};

struct GenericArgs {
    uint32_t format, group;
    const uint8_t *w;
    uint64_t n, row_bytes, k, rows;
    uint32_t x_kind;
    const void *x;
    uint32_t out_kind;
    void *out;
    uint64_t col0, out_stride;
    // The experts' product, as GemvArgs: `rows` routes; n rows an expert
    // (expert_bytes bytes) of the stacked matrix w.
    const uint32_t *experts;
    uint32_t n_experts;
    int topk, per_route;
    uint64_t expert_bytes;
};

struct DequantArgs {
    uint32_t format, group;
    const uint8_t *w;
    uint64_t n, row_bytes, k, first, count;
    const uint32_t *indices;
    uint32_t out_kind;
    void *out;
};

hipError_t launch_prep(const PrepArgs &a, hipStream_t s);

// Activations as bf16 planes for the float many-row product (mmf_kernel):
// [rows][planes][kpad] bf16: 1 plane (bf16 rows), 2 (f16) or 3 (f32).
struct PrepBf16Args {
    uint32_t x_kind;
    const void *x;        // [rows, k]
    uint64_t rows, k, kpad;
    int planes;
    uint16_t *out;
};
hipError_t launch_prep_bf16(const PrepBf16Args &a, hipStream_t s);
// The float many-row product (bf16 planes in MmArgs::planes): one launch, or
// with cols the weight rows of one of its column groups.
hipError_t launch_mmf(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s, int *cols);
hipError_t launch_fill(uint32_t *p, uint64_t words, hipStream_t s);
hipError_t launch_fill_bytes(uint8_t *p, uint64_t bytes, hipStream_t s);
hipError_t launch_qmv(uint32_t fmt, uint32_t group, int planes, const QmvArgs &a, dim3 grid,
                      size_t lds, hipStream_t s);
// Units of the small-M product for a format (0: not read by it).
int gemv_unit(uint32_t fmt, uint32_t group);
// Waves of one of its workgroups at most.
int gemv_max_waves(int planes, int rows);
// Bytes of LDS of one of its workgroups.
size_t gemv_lds(int rows, int planes, int chunk, int unit, int waves);
hipError_t launch_gemv(uint32_t fmt, uint32_t group, int planes, const GemvArgs &a, hipStream_t s);
// LDS bytes of a workgroup of the decode kernel staged in LDS.
size_t gemv2_lds(int rows, int planes, int units, int unit, int tiles, int kw, int tb);
size_t gemv4_lds(int rows, int planes, int units, int unit, int tiles, int ks, int tb);
// The many-row product: the size of a format's scale groups (32 or 16; 0:
// not read by it).
int mm_group(uint32_t fmt, uint32_t group);
// Elements of K a unit of it takes, and the weight rows of its column
// groups (for `wm` row tiles of 32).
int mm_unit(uint32_t fmt, uint32_t group);
int mm_cols(uint32_t fmt, uint32_t group, int planes, int rows);
// Row tiles of a wave and groups of waves of a workgroup for `rows` rows.
void mm_shape(int planes, int rows, int &wm, int &wmg);
hipError_t launch_mm(uint32_t fmt, uint32_t group, int planes, const MmArgs &a, hipStream_t s);
hipError_t launch_mm_reduce(const MmArgs &a, hipStream_t s);
hipError_t launch_generic(const GenericArgs &a, hipStream_t s);
hipError_t launch_dequantize(const DequantArgs &a, hipStream_t s);

}  // namespace kh
