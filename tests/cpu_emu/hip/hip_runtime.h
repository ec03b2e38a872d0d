// CPU emulation of the HIP device features libkapel_hip's kernels use, for a
// host build of the unchanged kernel sources (test infrastructure only).
//
// A launch runs its workgroups one after the other; each workgroup is
// blockDim.x host threads (one per lane), with a barrier for __syncthreads
// and one per wave of 64 for the wave-wide operations (__shfl_xor and the
// MFMA), which exchange their operands through per-wave slots.  Built with
// AddressSanitizer, every global and LDS access of the kernels is bounds
// checked on the host.
#pragma once
#include <barrier>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__
#define __align__(n) __attribute__((aligned(n)))
#define __HIP_MEMORY_SCOPE_AGENT 0
#define __HIP_MEMORY_SCOPE_WORKGROUP 1

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorInvalidDevice = 101 };
typedef struct ihipStream_t *hipStream_t;
struct int2 {
    int x, y;
};
struct uint2 {
    unsigned x, y;
};
struct float4 {
    float x, y, z, w;
};
struct uint4 {
    unsigned x, y, z, w;
};

namespace emu {

constexpr size_t LDS_BYTES = 160 * 1024;

struct Lane {
    dim3 tid, bid;
};
inline thread_local Lane self;
inline dim3 block_dim;
inline dim3 grid_dim;

struct Block {
    std::barrier<> *all = nullptr;
    std::barrier<> *wave[16] = {};
    uint64_t slots[16][64][4];  // per wave, per lane: up to 32 bytes
    unsigned threads = 0;
};
inline Block block;

inline int lane_id() { return (int)(self.tid.x & 63); }
inline int wave_id() { return (int)(self.tid.x >> 6); }
inline void wave_sync() { block.wave[wave_id()]->arrive_and_wait(); }

template <class T>
T shfl_xor(T v, int mask, int width = 64) {
    static_assert(sizeof(T) <= 8, "shuffled values fit a slot");
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &v, sizeof(T));
    wave_sync();
    int src = l ^ mask;
    if ((src / width) != (l / width)) src = l;
    T out;
    std::memcpy(&out, &block.slots[w][src][0], sizeof(T));
    wave_sync();
    return out;
}

typedef int v4i __attribute__((ext_vector_type(4)));

// v_mfma_i32_16x16x64_i8: D[i][j] = C[i][j] + sum_k A[i][k] B[k][j], i, j <
// 16, k < 64.  Lane l supplies A[l % 16][16 (l / 16) + b] and
// B[16 (l / 16) + b][l % 16] as bytes b = 0..15 of its 16-byte operand, and
// receives D[4 (l / 16) + v][l % 16], v = 0..3.
inline v4i mfma_i8(v4i a, v4i b, v4i c, int, int, int) {
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &a, 16);
    std::memcpy(&block.slots[w][l][2], &b, 16);
    wave_sync();
    v4i d = c;
    int j = l % 16;
    for (int v = 0; v < 4; v++) {
        int i = 4 * (l / 16) + v;
        int sum = 0;
        for (int k = 0; k < 64; k++) {
            int g = k / 16, byte = k % 16;
            const int8_t *ai = reinterpret_cast<const int8_t *>(&block.slots[w][16 * g + i][0]);
            const int8_t *bj = reinterpret_cast<const int8_t *>(&block.slots[w][16 * g + j][2]);
            sum += (int)ai[byte] * (int)bj[byte];
        }
        d[v] += sum;
    }
    wave_sync();
    return d;
}

typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// The 32 x 32 MFMAs: lane l supplies row l % 32 of A and column l % 32 of B
// for the k-slice l / 32 (B bytes, or one f32, per lane), and receives
// D[8 (v / 4) + 4 (l / 32) + v % 4][l % 32], v = 0..15.
inline int row32(int l, int v) { return 8 * (v / 4) + 4 * (l / 32) + v % 4; }

template <int B>
inline v16i mfma32_i8(const void *a, const void *b, v16i c) {
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], a, B);
    std::memcpy(&block.slots[w][l][2], b, B);
    wave_sync();
    v16i d = c;
    int j = l % 32;
    for (int v = 0; v < 16; v++) {
        int i = row32(l, v), sum = 0;
        for (int half = 0; half < 2; half++) {
            const int8_t *ai = reinterpret_cast<const int8_t *>(&block.slots[w][32 * half + i][0]);
            const int8_t *bj = reinterpret_cast<const int8_t *>(&block.slots[w][32 * half + j][2]);
            for (int k = 0; k < B; k++) sum += (int)ai[k] * (int)bj[k];
        }
        d[v] += sum;
    }
    wave_sync();
    return d;
}
inline v16i mfma32_i8x32(v4i a, v4i b, v16i c, int, int, int) { return mfma32_i8<16>(&a, &b, c); }

// v_mfma_f32_32x32x16_bf16: 8 bf16 a lane, as the i8 MFMAs; the 16 exact
// products summed in f64, rounded once, then added to C.
inline v16f mfma32_bf16(v4i a, v4i b, v16f c) {
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &a, 16);
    std::memcpy(&block.slots[w][l][2], &b, 16);
    wave_sync();
    v16f d = c;
    int j = l % 32;
    for (int v = 0; v < 16; v++) {
        int i = row32(l, v);
        double sum = 0;
        for (int half = 0; half < 2; half++) {
            const uint16_t *ai = reinterpret_cast<const uint16_t *>(&block.slots[w][32 * half + i][0]);
            const uint16_t *bj = reinterpret_cast<const uint16_t *>(&block.slots[w][32 * half + j][2]);
            for (int k = 0; k < 8; k++) {
                uint32_t x = (uint32_t)ai[k] << 16, y = (uint32_t)bj[k] << 16;
                float fx, fy;
                std::memcpy(&fx, &x, 4);
                std::memcpy(&fy, &y, 4);
                sum += (double)fx * (double)fy;
            }
        }
        d[v] = c[v] + (float)sum;
    }
    wave_sync();
    return d;
}
inline v16i mfma32_i8x16(long a, long b, v16i c, int, int, int) { return mfma32_i8<8>(&a, &b, c); }

inline v16f mfma32_f32x2(float a, float b, v16f c, int, int, int) {
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &a, 4);
    std::memcpy(&block.slots[w][l][2], &b, 4);
    wave_sync();
    v16f d = c;
    int j = l % 32;
    for (int v = 0; v < 16; v++) {
        int i = row32(l, v);
        // The hardware's sum of the two products: emulated as f64 products
        // summed then rounded once, then added to C (both products here are
        // exact in f32 whenever one k-slot is zero).
        float sum = 0.0f;
        for (int half = 0; half < 2; half++) {
            float ai, bj;
            std::memcpy(&ai, &block.slots[w][32 * half + i][0], 4);
            std::memcpy(&bj, &block.slots[w][32 * half + j][2], 4);
            sum += ai * bj;
        }
        d[v] += sum;
    }
    wave_sync();
    return d;
}

// v_perm_b32: byte s of the result is byte sel[s] of {hi:lo} (0..3 of lo,
// 4..7 of hi); selectors above 7 are not used by the kernels.
inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    uint64_t both = ((uint64_t)hi << 32) | lo;
    uint32_t out = 0;
    for (int s = 0; s < 4; s++) {
        uint32_t k = (sel >> (8 * s)) & 0xff;
        if (k == 12) continue;  // the constant 0x00
        if (k > 7) std::abort();
        out |= (uint32_t)((both >> (8 * k)) & 0xff) << (8 * s);
    }
    return out;
}

// v_alignbyte_b32: bits 8 (s % 4) .. 8 (s % 4) + 31 of {hi:lo}.
inline uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t s) {
    uint64_t both = ((uint64_t)hi << 32) | lo;
    return (uint32_t)(both >> (8 * (s & 3)));
}

// v_mov_b32_dpp with a quad permutation (ctrl < 0x100): lane 4i + j takes
// lane 4i + ctrl[2j + 1 : 2j].
inline int mov_dpp(int v, int ctrl, int, int, bool) {
    if (ctrl >= 0x100) std::abort();
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &v, 4);
    wave_sync();
    int src = (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);
    int out;
    std::memcpy(&out, &block.slots[w][src][0], 4);
    wave_sync();
    return out;
}

// ds_swizzle_b32 in bit mode (offset < 0x8000): within each 32 lanes, lane l
// takes lane ((l & and) | or) ^ xor.
inline int ds_swizzle(int v, int offset) {
    if (offset & 0x8000) std::abort();
    int w = wave_id(), l = lane_id();
    std::memcpy(&block.slots[w][l][0], &v, 4);
    wave_sync();
    int am = offset & 0x1f, om = (offset >> 5) & 0x1f, xm = (offset >> 10) & 0x1f;
    int src = (l & 32) | ((((l & 31) & am) | om) ^ xm);
    int out;
    std::memcpy(&out, &block.slots[w][src][0], 4);
    wave_sync();
    return out;
}

// Buffer resources and raw buffer loads: a dword whose offset is not
// wholly inside num_records bytes reads as zero.
struct BufferRsrc {
    const uint8_t *base;
    uint32_t num;
};
inline BufferRsrc make_rsrc(void *p, short, int num, int) { return BufferRsrc{(const uint8_t *)p, (uint32_t)num}; }
inline uint32_t buf_dword(const BufferRsrc &r, int off) {
    uint32_t o = (uint32_t)off, v = 0;
    if ((uint64_t)o + 4 <= r.num) std::memcpy(&v, r.base + o, 4);
    return v;
}
template <int N>
struct BufVec {
    typedef unsigned int type __attribute__((ext_vector_type(N)));
};
template <int N>
inline typename BufVec<N>::type buf_load(const BufferRsrc &r, int off) {
    typename BufVec<N>::type out;
    for (int i = 0; i < N; i++) out[i] = buf_dword(r, off + 4 * i);
    return out;
}

// buffer_load_* ... lds: `size` bytes of each lane at offset off, to lds +
// size * lane (dwords past num_records read as zero).
inline void lds_load(const BufferRsrc &r, void *lds, int size, uint32_t off) {
    uint8_t *dst = static_cast<uint8_t *>(lds) + size * lane_id();
    for (int i = 0; i < size / 4; i++) {
        uint32_t v = buf_dword(r, (int)(off + 4 * i));
        std::memcpy(dst + 4 * i, &v, 4);
    }
}

inline int frexp_exp(float v) {
    int e = 0;
    if (std::isfinite(v)) std::frexp(v, &e);
    return e;
}

template <class T>
T atomic_load(const T *p) {
    T v;
    __atomic_load(p, &v, __ATOMIC_SEQ_CST);
    return v;
}

template <class K, class... A>
void launch(K kernel, dim3 grid, dim3 threads, size_t lds, A... args);

}  // namespace emu

namespace kh {
alignas(16) inline uint8_t lds[emu::LDS_BYTES];
namespace mm {
alignas(16) inline uint8_t lds[emu::LDS_BYTES];
}
namespace mmf {
alignas(16) inline uint8_t lds[emu::LDS_BYTES];
}
}

#define threadIdx (emu::self.tid)
#define blockIdx (emu::self.bid)
#define blockDim (emu::block_dim)
#define gridDim (emu::grid_dim)
#define __syncthreads() (emu::block.all->arrive_and_wait())
#define __threadfence() __atomic_thread_fence(__ATOMIC_SEQ_CST)
#define __shfl_xor(v, m, ...) emu::shfl_xor((v), (m) __VA_OPT__(, ) __VA_ARGS__)
#define __builtin_amdgcn_mfma_i32_16x16x64_i8(...) emu::mfma_i8(__VA_ARGS__)
#define __builtin_amdgcn_mfma_i32_32x32x32_i8(...) emu::mfma32_i8x32(__VA_ARGS__)
#define __builtin_amdgcn_mfma_i32_32x32x16_i8(...) emu::mfma32_i8x16(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f32_32x32x2f32(...) emu::mfma32_f32x2(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) \
    emu::mfma32_bf16(__builtin_bit_cast(emu::v4i, (a)), __builtin_bit_cast(emu::v4i, (b)), (c))
#define __builtin_amdgcn_sched_barrier(m) ((void)0)
#define KH_PIN(x) ((void)0)
#define KH_EMU_LDS 1
#define KH_LDS_READ128(dst, ptr) memcpy(&(dst), (const void *)(ptr), 16)
#define KH_LDS_LOAD(rsrc, lds, size, voff) emu::lds_load((rsrc), (void *)(lds), (size), (uint32_t)(voff))
#define __builtin_amdgcn_s_waitcnt(n) ((void)0)
#define __builtin_amdgcn_s_barrier() (emu::block.all->arrive_and_wait())
#define __builtin_amdgcn_perm(hi, lo, s) emu::perm((hi), (lo), (s))
#define __builtin_amdgcn_alignbyte(hi, lo, s) emu::alignbyte((hi), (lo), (s))
#define __builtin_amdgcn_mov_dpp(v, c, r, b, z) emu::mov_dpp((v), (c), (r), (b), (z))
#define __builtin_amdgcn_ds_swizzle(v, o) emu::ds_swizzle((v), (o))
#define __builtin_amdgcn_frexp_expf(v) emu::frexp_exp(v)
#define __builtin_amdgcn_s_sleep(n) std::this_thread::yield()
typedef emu::BufferRsrc __amdgpu_buffer_rsrc_t;
#define __builtin_amdgcn_make_buffer_rsrc(p, s, n, f) emu::make_rsrc((p), (s), (n), (f))
#define __builtin_amdgcn_raw_buffer_load_b32(r, o, so, a) emu::buf_dword((r), (o) + (so))
#define __builtin_amdgcn_raw_buffer_load_b64(r, o, so, a) emu::buf_load<2>((r), (o) + (so))
#define __builtin_amdgcn_raw_buffer_load_b96(r, o, so, a) emu::buf_load<3>((r), (o) + (so))
#define __builtin_amdgcn_raw_buffer_load_b128(r, o, so, a) emu::buf_load<4>((r), (o) + (so))
#define __builtin_amdgcn_readfirstlane(v) (v)
#define __builtin_amdgcn_wave_barrier() emu::wave_sync()
#define __hip_atomic_fetch_add(p, v, order, scope) __atomic_fetch_add((p), (v), __ATOMIC_SEQ_CST)
#define __hip_atomic_load(p, order, scope) emu::atomic_load(p)
#define __hip_atomic_store(p, v, order, scope) __atomic_store_n((p), (v), __ATOMIC_SEQ_CST)
#define hipLaunchKernelGGL(kernel, grid, threads, lds, stream, ...) \
    emu::launch(kernel, dim3(grid), dim3(threads), (size_t)(lds), __VA_ARGS__)

inline hipError_t hipGetLastError() { return hipSuccess; }
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
#define HIP_SYMBOL(X) X
template <class T>
inline hipError_t hipGetSymbolAddress(void **p, T &symbol) {
    *p = (void *)&symbol;
    return hipSuccess;
}
inline hipError_t hipGetDevice(int *dev) {
    *dev = 0;
    return hipSuccess;
}
// A small device: few compute units, so that the emulated launches that
// size their grids by them walk several tiles a workgroup.
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
inline hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t, int) {
    *v = 2;
    return hipSuccess;
}
struct hipFuncAttributes {
    size_t sharedSizeBytes;
};
// Static LDS is counted in the emulator's dynamic pool.
inline hipError_t hipFuncGetAttributes(hipFuncAttributes *at, const void *) {
    at->sharedSizeBytes = 0;
    return hipSuccess;
}
// Workgroups a CU holds: by LDS and by 32 waves a CU (registers are not
// modelled).
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int *n, const void *, int threads, size_t lds) {
    const int by_waves = 32 / ((threads + 63) / 64);
    const int by_lds = lds ? (int)(emu::LDS_BYTES / lds) : by_waves;
    *n = by_waves < by_lds ? by_waves : by_lds;
    return hipSuccess;
}
inline hipError_t hipFuncSetAttribute(const void *, hipFuncAttribute, int bytes) {
    return bytes <= (int)emu::LDS_BYTES ? hipSuccess : hipErrorInvalidValue;
}
enum hipMemcpyKind { hipMemcpyDeviceToDevice = 3 };
inline hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind, hipStream_t) {
    std::memcpy(dst, src, n);
    return hipSuccess;
}

inline float __uint_as_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint32_t __float_as_uint(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline uint32_t max(uint32_t a, uint32_t b) { return a > b ? a : b; }
inline int64_t min(int64_t a, int64_t b) { return a < b ? a : b; }
using std::isfinite;

namespace emu {

// Lane threads, created once and reused by every launch.
struct Pool {
    std::vector<std::thread> workers;
    std::mutex m;
    std::condition_variable wake, idle;
    uint64_t generation = 0;
    unsigned active = 0, finished = 0;
    std::function<void(unsigned)> job;

    void ensure(unsigned n) {
        while (workers.size() < n) {
            unsigned t = (unsigned)workers.size();
            workers.emplace_back([this, t] {
                uint64_t seen = 0;
                for (;;) {
                    std::function<void(unsigned)> fn;
                    {
                        std::unique_lock<std::mutex> lock(m);
                        wake.wait(lock, [&] { return generation != seen; });
                        seen = generation;
                        if (t >= active) continue;
                        fn = job;
                    }
                    fn(t);
                    std::lock_guard<std::mutex> lock(m);
                    if (++finished == active) idle.notify_all();
                }
            });
            workers.back().detach();
        }
    }

    void run(unsigned n, std::function<void(unsigned)> fn) {
        ensure(n);
        std::unique_lock<std::mutex> lock(m);
        job = std::move(fn);
        active = n;
        finished = 0;
        generation++;
        wake.notify_all();
        idle.wait(lock, [&] { return finished == active; });
    }
};
// Never destroyed: its detached lanes wait on it until the process ends.
inline Pool &pool = *new Pool;

inline void fresh_block(unsigned threads, size_t lds) {
    // Uninitialised LDS reads show as garbage, not as zeros.
    std::memset(kh::lds, 0xA5, lds + 16);
    delete block.all;
    block.all = new std::barrier<>((ptrdiff_t)threads);
    for (unsigned w = 0; w < 16; w++) {
        delete block.wave[w];
        block.wave[w] = w < threads / 64 ? new std::barrier<>(64) : nullptr;
    }
    block.threads = threads;
}

template <class K, class... A>
void launch(K kernel, dim3 grid, dim3 threads, size_t lds, A... args) {
    if (lds + 16 > LDS_BYTES || threads.x % 64 || threads.x > 1024 || threads.y != 1 || threads.z != 1) {
        std::fprintf(stderr, "emu: launch shape not emulated (lds %zu, threads %u)\n", lds, threads.x);
        std::abort();
    }
    const unsigned total = grid.x * grid.y * grid.z;
    if (total == 0) return;
    fresh_block(threads.x, lds);
    block_dim = threads;
    grid_dim = grid;
    // Between workgroups, the last lane to arrive makes the next one's barriers.
    std::barrier<std::function<void()>> next((ptrdiff_t)threads.x,
                                             std::function<void()>([&] { fresh_block(threads.x, lds); }));
    pool.run(threads.x, [&](unsigned t) {
        self.tid = dim3(t, 0, 0);
        for (unsigned b = 0; b < total; b++) {
            self.bid = dim3(b % grid.x, (b / grid.x) % grid.y, b / (grid.x * grid.y));
            kernel(args...);
            // A lane that ends leaves the barriers it no longer waits at.
            block.wave[t / 64]->arrive_and_drop();
            block.all->arrive_and_drop();
            next.arrive_and_wait();
        }
    });
}
}  // namespace emu
