// The decode product (one row of f32 activations, or up to four of bytes),
// streamed: every multiplying wave owns whole weight rows.
//
// A workgroup takes `tiles` tiles of 16 weight rows, each split over `ks`
// waves by contiguous ranges of units of K, plus `npw` preparing waves.  A
// multiplying wave streams its 16 row segments unit after unit into a ring of
// LDS of its own with direct-to-LDS copies (16 bytes a lane, 1 KiB a copy;
// per unit the rows' chunks [row][CW] one after the other, CW the 16-byte
// chunks of a row's unit: odd for most formats, so that the 16 rows of a
// read fall on different banks; Q6_K's 14 and Q2_K's 6 leave two rows a
// bank, under 1 % of the table's time), keeping up to 56 copies in
// flight, and multiplies each unit as soon as its own copies have landed
// (`s_waitcnt vmcnt(n)` with n its later copies): the copies of later units
// are in flight meanwhile.  The preparing waves load and prepare the
// activations while the first copies fly (they issue no copies, so waiting
// for the activations never waits for weights).
//
// LDS written by the copies is read by inline assembly (each read waits for
// its own results): the compiler, which cannot tell the copies' LDS from
// what it reads, would otherwise wait for every copy in flight before the
// first read.
//
// The multiplication is the lane-group MFMA scheme of the lane readers
// (kh_lanes.h).  A wave's sums: its lane groups added in a fixed tree; with
// ks = 1 the wave writes its rows' outputs itself, with ks > 1 the sums of a
// tile's waves go through LDS and the preparing waves add them in wave
// order.  Reductions follow the shapes only: results do not depend on timing.
#pragma once

namespace kh {

namespace lanes {

#ifdef KH_EMU_LDS
// The host emulation: LDS addresses are pointers, reads are copies.
using lds_ptr = uintptr_t;
template <int N>
__device__ __forceinline__ void lds_rd(uint32_t (&v)[N], lds_ptr a) {
    memcpy(v, reinterpret_cast<const void *>(a), 4 * N);
}
#else
using lds_ptr = uint32_t;
// LDS reads by inline assembly: N dwords at a byte address, waited for.
template <int N>
__device__ __forceinline__ void lds_rd(uint32_t (&v)[N], lds_ptr a);
template <>
__device__ __forceinline__ void lds_rd<1>(uint32_t (&v)[1], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v[0]) : "v"(a) : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<2>(uint32_t (&v)[2], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:4\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]) : "v"(a) : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<3>(uint32_t (&v)[3], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %3\n\tds_read_b32 %1, %3 offset:4\n\tds_read_b32 %2, %3 offset:8\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]) : "v"(a) : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<4>(uint32_t (&v)[4], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %4\n\tds_read_b32 %1, %4 offset:4\n\tds_read_b32 %2, %4 offset:8\n\t"
                 "ds_read_b32 %3, %4 offset:12\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]) : "v"(a) : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<5>(uint32_t (&v)[5], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %5\n\tds_read_b32 %1, %5 offset:4\n\tds_read_b32 %2, %5 offset:8\n\t"
                 "ds_read_b32 %3, %5 offset:12\n\tds_read_b32 %4, %5 offset:16\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]) : "v"(a) : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<6>(uint32_t (&v)[6], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %6\n\tds_read_b32 %1, %6 offset:4\n\tds_read_b32 %2, %6 offset:8\n\t"
                 "ds_read_b32 %3, %6 offset:12\n\tds_read_b32 %4, %6 offset:16\n\t"
                 "ds_read_b32 %5, %6 offset:20\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
                 : "v"(a)
                 : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<8>(uint32_t (&v)[8], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:4\n\tds_read_b32 %2, %8 offset:8\n\t"
                 "ds_read_b32 %3, %8 offset:12\n\tds_read_b32 %4, %8 offset:16\n\t"
                 "ds_read_b32 %5, %8 offset:20\n\tds_read_b32 %6, %8 offset:24\n\t"
                 "ds_read_b32 %7, %8 offset:28\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7])
                 : "v"(a)
                 : "memory");
}
template <>
__device__ __forceinline__ void lds_rd<9>(uint32_t (&v)[9], lds_ptr a) {
    asm volatile("ds_read_b32 %0, %9\n\tds_read_b32 %1, %9 offset:4\n\tds_read_b32 %2, %9 offset:8\n\t"
                 "ds_read_b32 %3, %9 offset:12\n\tds_read_b32 %4, %9 offset:16\n\t"
                 "ds_read_b32 %5, %9 offset:20\n\tds_read_b32 %6, %9 offset:24\n\t"
                 "ds_read_b32 %7, %9 offset:28\n\tds_read_b32 %8, %9 offset:32\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8])
                 : "v"(a)
                 : "memory");
}

#endif

// The lane readers' reads from a wave's LDS ring by inline assembly.
struct AsmLdsSrc {
    lds_ptr base;  // LDS byte address
};

template <int N>
__device__ __forceinline__ void ldb(uint32_t (&v)[N], const AsmLdsSrc &s, uint32_t off) {
    lds_rd<N>(v, s.base + off);
}

template <int R>
__device__ __forceinline__ void run(uint32_t (&w)[(R + 3) / 4], const AsmLdsSrc &src, uint32_t off) {
    static_assert(R % 2 == 0, "even runs only");
    constexpr int D = (R + 5) / 4, W = (R + 3) / 4;
    const uint32_t s = off & 2u;
    uint32_t v[D + 1];
    lds_rd<D>(*reinterpret_cast<uint32_t(*)[D]>(v), src.base + (off - s));
    v[D] = 0u;
#pragma unroll
    for (int i = 0; i < W; i++) w[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], s);
}

}  // namespace lanes

#ifdef KH_EMU_LDS
__device__ __forceinline__ lanes::lds_ptr lds_addr(const void *p) { return (uintptr_t)p; }
#else
__device__ __forceinline__ lanes::lds_ptr lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}
#endif

// One unit's LDS reads for one row of activations, issued together and
// waited for once: the lane's weight bytes (every read at an address aligned
// to its size), the A operands of the unit's steps (`pa`, steps at the
// reader's xpos offsets) and the activation info of its groups (`ia`).  Q4_K
// and Q6_K have them in one instruction sequence; the other readers read
// their weights through AsmLdsSrc (a wait a field).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

template <class F>
struct FastUnit {
    static constexpr bool ON = false;
    static constexpr int NI = 1;
    __device__ static int info_of(int) { return 0; }
};
template <>
struct FastUnit<lanes::Q4K> {
    static constexpr bool ON = true;
    static constexpr int NI = 2;  // info reads: the unit's two groups of 32 of this lane group
    // Group gi's info entry.
    __device__ static int info_of(int gi) { return gi; }
    __device__ static void reads(lanes::Q4K::Regs &r, v4i (&av)[4], float4 (&inf)[NI], lanes::lds_ptr wa, int g,
                                 lanes::lds_ptr pa, lanes::lds_ptr ia) {
        u32x4_t h, q0, q1, p0, p1, p2, p3, i0, i1;
        const lanes::lds_ptr qa = wa + 16 + 32 * g;
#ifdef KH_EMU_LDS
        memcpy(&h, (const void *)wa, 16), memcpy(&q0, (const void *)qa, 16), memcpy(&q1, (const void *)(qa + 16), 16);
        memcpy(&p0, (const void *)pa, 16), memcpy(&p1, (const void *)(pa + 16), 16);
        memcpy(&p2, (const void *)(pa + 32), 16), memcpy(&p3, (const void *)(pa + 48), 16);
        memcpy(&i0, (const void *)ia, 16), memcpy(&i1, (const void *)(ia + 16), 16);
#else
        asm volatile(
            "ds_read_b128 %0, %9\n\tds_read_b128 %1, %10\n\tds_read_b128 %2, %10 offset:16\n\t"
            "ds_read_b128 %3, %11\n\tds_read_b128 %4, %11 offset:16\n\tds_read_b128 %5, %11 offset:32\n\t"
            "ds_read_b128 %6, %11 offset:48\n\tds_read_b128 %7, %12\n\tds_read_b128 %8, %12 offset:16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(h), "=&v"(q0), "=&v"(q1), "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3), "=&v"(i0), "=&v"(i1)
            : "v"(wa), "v"(qa), "v"(pa), "v"(ia)
            : "memory");
#endif
        r.h[0] = h.x, r.h[1] = h.y, r.h[2] = h.z, r.h[3] = h.w;
        r.q[0] = q0.x, r.q[1] = q0.y, r.q[2] = q0.z, r.q[3] = q0.w;
        r.q[4] = q1.x, r.q[5] = q1.y, r.q[6] = q1.z, r.q[7] = q1.w;
        av[0] = (v4i)p0, av[1] = (v4i)p1, av[2] = (v4i)p2, av[3] = (v4i)p3;
        inf[0] = float4{__uint_as_float(i0.x), __uint_as_float(i0.y), __uint_as_float(i0.z), __uint_as_float(i0.w)};
        inf[1] = float4{__uint_as_float(i1.x), __uint_as_float(i1.y), __uint_as_float(i1.z), __uint_as_float(i1.w)};
    }
};
template <>
struct FastUnit<lanes::Q6K> {
    static constexpr bool ON = true;
    static constexpr int NI = 2;  // groups of 16 at steps 0, 1 share block 0 of 32; 2, 3 block 2
    __device__ static int info_of(int gi) { return gi >> 1; }
    // A unit starts 0 or 2 bytes past a 16-byte boundary (blocks of 210
    // bytes): every field is read from the aligned address below it, one
    // dword more, and shifted into place with v_alignbyte.
    __device__ static void reads(lanes::Q6K::Regs &r, v4i (&av)[4], float4 (&inf)[NI], lanes::lds_ptr wa, int g,
                                 lanes::lds_ptr pa, lanes::lds_ptr ia) {
        u32x4_t l0, l1, l2, h0, h1, h2, p0, p1, p2, p3, i0, i1;
        u32x2_t s01;
        unsigned s2, dd;
        const uint32_t sh = (uint32_t)wa & 3u;
        const lanes::lds_ptr w0 = wa - sh;  // 16-byte aligned
        const int hh = g >> 1, qq = g & 1;
        const lanes::lds_ptr la = w0 + 64 * hh + 32 * qq, ha = w0 + 128 + 32 * hh, sa = w0 + 192 + 8 * hh;
#ifdef KH_EMU_LDS
        memcpy(&l0, (const void *)la, 16), memcpy(&l1, (const void *)(la + 16), 16), memcpy(&l2, (const void *)(la + 32), 16);
        memcpy(&h0, (const void *)ha, 16), memcpy(&h1, (const void *)(ha + 16), 16), memcpy(&h2, (const void *)(ha + 32), 16);
        memcpy(&s01, (const void *)sa, 8), memcpy(&s2, (const void *)(sa + 8), 4), memcpy(&dd, (const void *)(w0 + 208), 4);
        memcpy(&p0, (const void *)pa, 16), memcpy(&p1, (const void *)(pa + 16), 16);
        memcpy(&p2, (const void *)(pa + 64), 16), memcpy(&p3, (const void *)(pa + 80), 16);
        memcpy(&i0, (const void *)ia, 16), memcpy(&i1, (const void *)(ia + 32), 16);
#else
        asm volatile(
            "ds_read_b128 %0, %15\n\tds_read_b128 %1, %15 offset:16\n\tds_read_b128 %2, %15 offset:32\n\t"
            "ds_read_b128 %3, %16\n\tds_read_b128 %4, %16 offset:16\n\tds_read_b128 %5, %16 offset:32\n\t"
            "ds_read_b64 %6, %17\n\tds_read_b32 %7, %17 offset:8\n\tds_read_b32 %8, %18 offset:208\n\t"
            "ds_read_b128 %9, %19\n\tds_read_b128 %10, %19 offset:16\n\tds_read_b128 %11, %19 offset:64\n\t"
            "ds_read_b128 %12, %19 offset:80\n\tds_read_b128 %13, %20\n\tds_read_b128 %14, %20 offset:32\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(l0), "=&v"(l1), "=&v"(l2), "=&v"(h0), "=&v"(h1), "=&v"(h2), "=&v"(s01), "=&v"(s2), "=&v"(dd),
              "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3), "=&v"(i0), "=&v"(i1)
            : "v"(la), "v"(ha), "v"(sa), "v"(w0), "v"(pa), "v"(ia)
            : "memory");
#endif
        const uint32_t l[12] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w, l2.x, l2.y, l2.z, l2.w};
        const uint32_t h[12] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w, h2.x, h2.y, h2.z, h2.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            r.ql[i] = __builtin_amdgcn_alignbyte(l[i + 1], l[i], sh);
            r.qh[i] = __builtin_amdgcn_alignbyte(h[i + 1], h[i], sh);
        }
        r.sc[0] = __builtin_amdgcn_alignbyte(s01.y, s01.x, sh);
        r.sc[1] = __builtin_amdgcn_alignbyte(s2, s01.y, sh);
        r.d = (dd >> (8 * sh)) & 0xffffu;
        av[0] = (v4i)p0, av[1] = (v4i)p1, av[2] = (v4i)p2, av[3] = (v4i)p3;
        inf[0] = float4{__uint_as_float(i0.x), __uint_as_float(i0.y), __uint_as_float(i0.z), __uint_as_float(i0.w)};
        inf[1] = float4{__uint_as_float(i1.x), __uint_as_float(i1.y), __uint_as_float(i1.z), __uint_as_float(i1.w)};
    }
};

template <class F, int P, int MT, int XK>
__global__ __launch_bounds__(1024) void gemv4_kernel(GemvArgs a) {
    using UN = Unit<F>;
    constexpr int U = F::U, CW = UN::CW, UC = 16 * CW;  // chunks of a unit
    constexpr int ACC = P == 3 ? MT : 4 * MT;
    constexpr int NG = F::GS == 16 ? F::STEPS : F::STEPS / 2;
    constexpr int INFLIGHT = 56;  // copies a wave keeps in flight (vmcnt <= 63)
    extern __shared__ __align__(16) uint8_t lds[];

    const int t0 = blockIdx.x * a.tiles;
    if (t0 >= a.total_tiles) return;
    grid_fill<F>();
    const int T = min(a.tiles, a.total_tiles - t0);
    const int rows = a.rows, ks = a.kw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n16 = lane & 15;
    const int span = a.units * U;
    const int RC = a.tb * 64;  // chunks of a wave's ring
    KH_T(0);

    // LDS: planes [rows][P][span], zeros [span], info [rows][span / 32],
    // sums [tiles][ks][16][rows], rings [tiles * ks][RC chunks].
    int8_t *planes = reinterpret_cast<int8_t *>(lds + 16);
    int8_t *zeros = planes + (size_t)rows * P * span;
    float4 *info = reinterpret_cast<float4 *>(zeros + span);
    float *sums = reinterpret_cast<float *>(info + (size_t)rows * (span / 32));
    uint8_t *rings = lds + (((uintptr_t)(sums + (size_t)a.tiles * ks * 16 * rows) - (uintptr_t)lds + 15) & ~(uintptr_t)15);

    // The matrix and row of a tile's row.
    auto row_of = [&](int tile, int r, int &mat) {
        mat = 0;
        for (int i = 1; i < a.count; i++)
            if (tile >= a.tile0[i]) mat = i;
        return (int64_t)(tile - a.tile0[mat]) * 16 + r;
    };

    if (wave < a.npw) {
        // ---- the activations, then (with ks > 1) the sums of the tiles
        for (int i = threadIdx.x; i < span / 16; i += 64 * a.npw)
            reinterpret_cast<v4i *>(zeros)[i] = v4i{0, 0, 0, 0};
        const XIn xin{a.x, rows, a.k, a.x_kind};
        const int qpc = rows * span / 4;
        // The first pass's loads go out before any weight copy (a CU's
        // loads return in order): the multiplying waves wait for them here.
        float xv[PASSES][4];
        x_load<XK>(xin, 0, span, 0, threadIdx.x, 64 * a.npw, xv);
        __builtin_amdgcn_s_barrier();
        x_prepare<P, XK>(xin, span, 0, threadIdx.x, 64 * a.npw, xv, planes, info);
        for (int q0 = 64 * a.npw * PASSES; q0 < qpc; q0 += 64 * a.npw * PASSES) {
            x_load<XK>(xin, 0, span, q0, threadIdx.x, 64 * a.npw, xv);
            x_prepare<P, XK>(xin, span, q0, threadIdx.x, 64 * a.npw, xv, planes, info);
        }
        KH_T(1);
        lds_barrier();  // the activations are ready
        KH_T(2);
        if (ks == 1) return;
        lds_barrier();  // the sums are written
        for (int o = threadIdx.x; o < T * 16 * rows; o += 64 * a.npw) {
            const int t = o / (16 * rows), r = (o / rows) % 16, m = o % rows;
            int mat;
            const int64_t n = row_of(t0 + t, r, mat);
            if (n >= (int64_t)a.n[mat]) continue;
            float v = sums[((t * ks + 0) * 16 + r) * rows + m];
            for (int c = 1; c < ks; c++) v = v + sums[((t * ks + c) * 16 + r) * rows + m];
            store_out(a.out_kind, a.out, (uint64_t)m * a.out_stride + a.col0[mat] + (uint64_t)n, v);
        }
        KH_T(5);
        return;
    }

    // ---- a multiplying wave: units [u0, u0 + nu) of K of its tiles.  With
    // ks = 1 and one matrix a wave takes tile t of its workgroup, then the
    // same tile of every gridDim.x-th workgroup after it (ni tiles): its
    // stream of copies runs on from one tile to the next.
    const int cw = wave - a.npw, t = cw / ks, kk = cw % ks;
    const bool live = t < T;
    const int upw = (a.units + ks - 1) / ks;
    const int u0 = kk * upw;
    const int nu = live ? max(0, min(upw, a.units - u0)) : 0;
    const bool walk = ks == 1 && a.count == 1;
    const int stride = walk ? (int)gridDim.x * a.tiles : 0;
    const int first = t0 + t;
    const int ni = !live ? 0 : walk ? (a.total_tiles - first + stride - 1) / stride : 1;
    const int nunits = ni * nu;                 // units of the stream
    const int nc = (nunits * UC + 63) / 64;     // copies of the stream
    uint8_t *ring = rings + (size_t)cw * RC * 16;
    int mat;
    (void)row_of(first, 0, mat);
    const lanes::Src src = lanes::source(a.w[mat], a.wbytes[mat]);
    const int64_t nmat = (int64_t)a.n[mat];
    const int tile_base = a.tile0[mat];

    // Copy c: chunks [64 c, 64 c + 64) of the stream, [unit][row][CW] unit
    // after unit (tile i's units i nu .. i nu + nu - 1).
    auto issue = [&](int c) __attribute__((always_inline)) {
        const int ci = c * 64 + lane;
        const int J = ci / UC, rem = ci - J * UC, r = rem / CW, cc = rem - r * CW;
        const int i = nu ? J / nu : 0, j = J - i * nu;
        const int64_t n = (int64_t)(first + i * stride - tile_base) * 16 + r;
        const bool on = J < nunits && n < nmat;
        const uint32_t at = (uint32_t)n * (uint32_t)a.row_bytes + UN::block(u0 + j) * F::BYTES;
        KH_LDS_LOAD(src.r, ring + (size_t)((c * 64) % RC) * 16, 16, on ? (at & ~3u) + 16u * cc : lanes::NONE);
    };
    // The copies that may be issued before unit J of the stream is
    // multiplied: at most INFLIGHT beyond those of the units before J, none
    // over a unit not yet multiplied.
    auto allowed = [&](int J) {
        const int done = (J * UC) / 64;  // copies wholly of units < J
        return min(nc, min(done + INFLIGHT, (J * UC + RC) / 64));
    };
    __builtin_amdgcn_s_barrier();  // the activations' first loads are out
    int issued = 0;
    // A few copies before the activations' barrier: issuing more would keep
    // this wave from the barrier while the memory pipeline is full.
    for (const int lim = min(allowed(0), a.chunk > 0 ? a.chunk : 8); issued < lim; issued++) issue(issued);
    KH_T(1);
    lds_barrier();  // the activations are ready
    KH_T(2);

    // The A operand of this lane (as in the staged kernel).
    const int ai = lane & 15, aj = ai & 3;
    const bool a_lane = (ai >> 2) == (lane >> 4);
    lanes::lds_ptr a_addr[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        int m = P == 3 ? mi : 4 * mi + aj, p = P == 3 ? aj : 0;
        bool on = a_lane && p < P && m < rows;
        a_addr[mi] = lds_addr(on ? planes + (m * P + p) * span : zeros) + F::xpos(g, 0);
    }
    const lanes::lds_ptr info_addr = lds_addr(info) + (F::xpos(g, 0) / 32) * 16;
    const int blocks32 = a.k / 32;

    float acc[ACC];
#pragma unroll
    for (int i = 0; i < ACC; i++) acc[i] = 0.0f;
    int64_t row0 = (int64_t)(first - tile_base) * 16;
    for (int J = 0, j = 0; J < nunits; J++) {
        for (const int lim = allowed(J); issued < lim; issued++) issue(issued);
        // The last copy of unit J may have been issued just now: every lane
        // issues it before any lane reads unit J (one instruction for the
        // wave on the device; lanes that run apart in a host emulation).
        __builtin_amdgcn_wave_barrier();
        // Unit J's copies are the first ((J + 1) UC + 63) / 64.
        wait_vm_n(min(63, issued - ((J + 1) * UC + 63) / 64));
        if (J == 0) KH_T(3);
        if (J < 12) KH_T(8 + 2 * J);
        const int u = u0 + j;
        const bool ok = U == 256 || 4 * u + g < blocks32;
        const uint32_t at = (uint32_t)(row0 + n16) * (uint32_t)a.row_bytes + UN::block(u) * F::BYTES;
        typename F::Regs R;
        const lanes::lds_ptr wbase = lds_addr(ring) + (lanes::lds_ptr)(((J * UC) % RC) * 16);
        constexpr bool FAST = FastUnit<F>::ON && P == 3;
        v4i avf[F::STEPS];
        float4 inff[FastUnit<F>::NI];
        if constexpr (FAST) {
            FastUnit<F>::reads(R, avf, inff, wbase + (lanes::lds_ptr)(n16 * CW * 16) + (at & 3u), g,
                               a_addr[0] + (lanes::lds_ptr)(u * U),
                               info_addr + (lanes::lds_ptr)(((u * U) / 32) * 16));
        } else {
            F::load(R, lanes::AsmLdsSrc{wbase}, (uint32_t)(n16 * CW * 16) + (at & 3u), UN::local(u), g);
        }
        float sc[NG], mn[NG];
        F::scales(R, g, sc, mn);
        v4i c[MT];
#pragma unroll
        for (int s = 0; s < F::STEPS; s++) {
            v4i bw = F::codes(R, s, g);
            if (U == 128 && !ok) bw = v4i{0, 0, 0, 0};
            if (F::GS == 16 || (s & 1) == 0)
#pragma unroll
                for (int mi = 0; mi < MT; mi++) c[mi] = v4i{0, 0, 0, 0};
            const int xo = u * U + F::xpos(g, s) - F::xpos(g, 0);
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
                v4i av;
                if constexpr (FAST) {
                    av = avf[s];
                } else {
                    uint32_t w4[4];
                    lanes::lds_rd<4>(w4, a_addr[mi] + xo);
                    av = lanes::vec(w4[0], w4[1], w4[2], w4[3]);
                }
                c[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bw, c[mi], 0, 0, 0);
            }
            if (!(F::GS == 16 || (s & 1) == 1)) continue;
            // The group of this step is complete: scale it (nothing past K).
            const int s0 = F::GS == 16 ? s : s - 1, gi = F::GS == 16 ? s : s / 2;
            const int blk = (u * U + F::xpos(g, s0) - F::xpos(g, 0)) / 32;
            const bool second = ((F::xpos(g, s0) / 16) & 1) != 0;
#pragma unroll
            for (int mi = 0; mi < MT; mi++) {
#pragma unroll
                for (int jj = 0; jj < (P == 3 ? 1 : 4); jj++) {
                    int m = P == 3 ? mi : 4 * mi + jj;
                    if (m >= rows) continue;
                    float4 in;
                    if constexpr (FAST) {
                        in = inff[FastUnit<F>::info_of(gi)];
                    } else {
                        uint32_t i4[4];
                        lanes::lds_rd<4>(i4, info_addr + (lanes::lds_ptr)((m * (span / 32) + (ok ? blk : 0)) * 16));
                        in = float4{__uint_as_float(i4[0]), __uint_as_float(i4[1]), __uint_as_float(i4[2]),
                                    __uint_as_float(i4[3])};
                    }
                    float dot;
                    if (P == 3) dot = fmaf((float)c[mi].x, a.hi, (float)((c[mi].y << a.shift) + c[mi].z));
                    else dot = (float)c[mi][jj];
                    float xsum = F::GS == 32 ? in.y : (second ? in.w : in.z);
                    float tt = fmaf(dot, sc[gi] * in.x, acc[m]);
                    tt = fmaf(-mn[gi], xsum, tt);
                    acc[m] = ok ? tt : acc[m];
                }
            }
        }
        if (J < 12) KH_T(9 + 2 * J);
        if (++j < nu || ks > 1) continue;
        // ks = 1: the tile is done.  Its four lane groups of each row in a
        // fixed tree, then its outputs.
        j = 0;
#pragma unroll
        for (int i = 0; i < ACC; i++) {
            float v = acc[i];
            v = v + __shfl_xor(v, 16);
            v = v + __shfl_xor(v, 32);
            const int64_t n = row0 + n16;
            if (g == 0 && i < rows && n < nmat)
                store_out(a.out_kind, a.out, (uint64_t)i * a.out_stride + a.col0[mat] + (uint64_t)n, v);
            acc[i] = 0.0f;
        }
        row0 += (int64_t)stride * 16;
    }
    KH_T(4);
    if (ks == 1) {
        KH_T(5);
        return;
    }
    // The four lane groups of each row in a fixed tree.
#pragma unroll
    for (int i = 0; i < ACC; i++) {
        float v = acc[i];
        v = v + __shfl_xor(v, 16);
        acc[i] = v + __shfl_xor(v, 32);
    }
    wait_vm_n(0);
    if (live && g == 0)
#pragma unroll
        for (int i = 0; i < ACC; i++)
            if (i < rows) sums[((t * ks + kk) * 16 + n16) * rows + i] = acc[i];
    lds_barrier();  // the sums are written
    KH_T(5);
}

}  // namespace kh
