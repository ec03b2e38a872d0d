// The C ABI of libkapel_hip: argument checks, the choice of mode, the
// workspace, and the plan of launches.
//
// Checks follow QuantizedMatmul::infer (kapel-ops/src/matmul.rs:105-150) and
// the launch's refusals (kapel-cuda/src/device.rs:673-718); the choice of
// byte activations follows Run<QuantizedMatmul> for Cpu
// (kapel-cpu/src/matmul.rs:286-301) and bytes::layout (bytes.rs:51-77).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kh_internal.h"

using namespace kh;

namespace {

uint64_t div_up(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
uint64_t align_up(uint64_t a, uint64_t b) { return div_up(a, b) * b; }

// Formats the MFMA product reads; the others take the generic kernel.
bool mfma_format(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q8_0: case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1:
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K:
    case KH_IQ4_NL: case KH_IQ4_XS: case KH_IQ3_S:
        return true;
    case KH_INT8: case KH_INT4:
        return group == 32 || group == 64 || group == 128 || group == 256;
    default:
        return false;
    }
}

// Weights the generic kernel takes: formats without an MFMA reader, and the
// non-linear formats in matrices of 2 GiB or more (read by the small-M and
// many-row kernels only, at 32-bit offsets).
bool generic_weight(const kh_weight &w) {
    if (!mfma_format(w.format, w.group)) return true;
    const bool iq = w.format == KH_IQ4_NL || w.format == KH_IQ4_XS || w.format == KH_IQ3_S;
    return iq && w.bytes >= (1ull << 31);
}

// bytes.rs:51-77: the formats read with activations in bytes.
bool byte_format(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q8_0: case KH_Q4_0: case KH_Q4K: case KH_Q5K: case KH_Q6K:
        return true;
    case KH_INT8: case KH_INT4:
        return group == 32 || group == 64 || group == 128;
    default:
        return false;
    }
}

int groups_per_step(uint32_t fmt) {
    return (fmt == KH_Q6K || fmt == KH_Q2K || fmt == KH_Q3K) ? 4 : 2;
}

// Activation rows one launch takes: the slot groups (row, group) of a step
// fit in MAX_MFMAS MFMAs.
int rows_per_launch(uint32_t fmt, int planes) {
    int slot_groups = MAX_MFMAS * slot_groups_per_mfma(planes);
    return slot_groups / groups_per_step(fmt);
}

bool float_kind(uint32_t kind) { return kind == KH_F32 || kind == KH_BF16 || kind == KH_F16; }
uint64_t kind_bytes(uint32_t kind) { return kind == KH_F32 ? 4 : 2; }

// The split of K into segments for one launch: a function of the shapes only
// (tiles of 16 rows, steps of 64 elements), so the sums are the same on any
// device.  Enough workgroups to give each of the 256 CUs several, segments of
// at least 4 steps, whole super-blocks for the 256-element formats.
struct Split {
    int segs, seg_steps;
    size_t lds;
};

size_t lds_bytes(int rows, int planes, int seg_steps) {
    size_t span = (size_t)seg_steps * 64;
    return 16 + (size_t)rows * planes * (span + 16) + (size_t)rows * (span / 32) * 2 * 4 +
           (size_t)rows * (span / 16) * 4;
}

Split split_k(uint64_t tiles, int steps, int rows, int planes, uint32_t fmt) {
    uint64_t wgs = div_up(tiles, 4);
    int quantum = (steps % 4 == 0) ? 4 : 1;
    int want = (int)std::min<uint64_t>(MAX_SEGS, std::max<uint64_t>(1, div_up(1024, wgs)));
    int seg_steps = (int)align_up(std::max<int>(4, (int)div_up(steps, want)), quantum);
    seg_steps = std::min(seg_steps, (int)align_up(steps, quantum));
    while (seg_steps > quantum && lds_bytes(rows, planes, seg_steps) > (size_t)MAX_LDS)
        seg_steps -= quantum;
    int segs = (int)div_up(steps, seg_steps);
    while (segs > MAX_SEGS) {
        seg_steps += quantum;
        segs = (int)div_up(steps, seg_steps);
    }
    (void)fmt;
    return Split{segs, seg_steps, lds_bytes(rows, planes, seg_steps)};
}

// The small-M product: activation rows of one of its workgroups, and the
// rows it takes in one launch (in chunks of the former).
int gemv_max_rows(int planes) { return planes == 1 ? 16 : 8; }
constexpr uint64_t GEMV_ROWS = 64;
constexpr int GEMV_DIRECT_ROWS = 4;

// Its split, a function of the shapes only: tiles per workgroup (4, 2 or 1:
// as many as still leave a workgroup for each of the 256 CUs), waves per tile
// (up to 16 or 8 waves a workgroup, not more than the units of K) splitting K, and
// chunks of K whose activations fit the preparation (16 per thread) and LDS.
struct GemvSplit {
    int units, chunk, tiles, kw;
};

GemvSplit gemv_split(uint64_t k, int unit, int tiles, int rows, int planes, int mchunks, bool copied) {
    GemvSplit g{};
    g.units = (int)div_up(k, unit);
    g.tiles = 4;
    while (g.tiles > 1 && div_up(tiles, g.tiles) * mchunks < 256) g.tiles /= 2;
    // One tile a workgroup past one round of the CUs but two within it: two
    // (measured: the Llama layer's [q; k; v], 320 tiles, 7.79 -> 7.28 us at
    // M = 1; o, 192 tiles, stays at one).
    if (g.tiles == 1 && (uint64_t)tiles * mchunks > 256 && div_up(tiles, 2) * mchunks <= 256) g.tiles = 2;
    g.kw = std::max(1, std::min(gemv_max_waves(planes, rows) / g.tiles, g.units));
    int threads = 64 * g.tiles * g.kw;
    // Activations copied (prepared beforehand) are not limited by the threads.
    int by_threads = copied ? 1 << 30 : 16 * threads / (rows * unit);
    // LDS: 16 + span (rows planes + 1 + rows / 2) + waves 64 rows <= 64 KiB.
    long room = 65536 - 16 - 64L * g.tiles * g.kw * rows;
    int by_lds = (int)(room / ((long)unit * rows * planes + unit + (long)unit * rows / 2));
    g.chunk = std::max(1, std::min({g.units, by_threads, by_lds}));
    return g;
}

// The many-row product's split, a function of the shapes only: the kernel's
// row tiles (mm_shape), its column groups (mm_cols), and K split into `ks`
// ranges of `ups` units when that shortens the rounds of 256 workgroups (one
// a CU: a workgroup fills its CU's LDS).  Each range keeps at least 512
// elements of K.
struct MmSplit {
    int wm, wmg, cols, mtiles, ngroups, units, ups, ks;
};

// The K split of a many-row launch of m.mtiles x m.ngroups workgroups: the
// time of a split is rounds of 256 workgroups times units each; a split is
// taken when it saves more than 15 % (its partial sums cost a pass of their
// own), each range keeping at least 512 elements of K.
void split_k_of(MmSplit &m, int unit, uint64_t k) {
    m.units = (int)div_up(k, unit);
    const uint64_t base = (uint64_t)m.mtiles * m.ngroups;
    const int most = std::max(1, m.units / (int)div_up(512, unit));
    auto cost = [&](int ks) { return div_up(base * ks, 256) * div_up(m.units, ks); };
    int ks = 1;
    uint64_t best = cost(1);
    for (int s = 2; s <= most; s++)
        if (cost(s) * 100 < best * 85) {
            ks = s;
            best = cost(s);
        }
    m.ups = (int)div_up(m.units, ks);
    m.ks = (int)div_up(m.units, m.ups);
}

MmSplit mm_split(uint64_t rows, uint64_t k, const kh_weight *weights, const std::vector<uint32_t> &members,
                 int planes) {
    const kh_weight &w = weights[members[0]];
    MmSplit m{};
    mm_shape(planes, (int)rows, m.wm, m.wmg);
    m.cols = mm_cols(w.format, w.group, planes, (int)rows);
    m.mtiles = (int)div_up(rows, 32 * m.wm * m.wmg);
    m.ngroups = 0;
    for (uint32_t i : members) m.ngroups += (int)div_up(weights[i].n, m.cols);
    split_k_of(m, mm_unit(w.format, w.group), k);
    return m;
}

// The decode kernel with its weights staged in LDS (gemv2_kernel): for one
// row of f32 activations or up to four of bytes, without block dots.  Tiles a
// workgroup as the small-M split picks them (halved while LDS is short);
// multiplying waves as many as fit (up to 16 with the preparing ones, not
// more than the units); copies of 1 KiB a wave for its units of every tile.
struct Gemv2 {
    bool ok = false;
    int tiles, npw, kw, tb;
};

Gemv2 gemv2_plan(uint32_t fmt, uint32_t group, uint64_t k, int rows, int planes, int tiles_total, int tiles) {
    Gemv2 p;
    const int unit = gemv_unit(fmt, group);
    const int len = (int)kh_block_len(fmt, group), bytes = (int)kh_block_bytes(fmt, group);
    if (!unit || !len) return p;
    const int ub = (len >= unit ? 1 : unit / len) * bytes;
    const int cw = (ub + (bytes % 4 ? 2 : 0) + 15) / 16;
    const int units = (int)div_up(k, unit);
    const int quads = rows * units * unit / 4;
    // IQ3_S's kernels keep a 2 KiB copy of its grid in LDS.
    const size_t limit = 160 * 1024 - (fmt == KH_IQ3_S ? 2048 : 0);
    // Preparing waves: enough for one pass of loads over the activations
    // (256 quads a wave) up to four (measured: 3 instead of 2 at K = 3072
    // shortens the [q; k; v] and o calls by 10-12 %).
    p.npw = std::max(1, std::min(4, (int)div_up(quads, 256)));
    // Multiplying waves: as many as fit (with the preparing ones, 16), then
    // as few as take the same number of units each (16 units over 13 waves
    // would leave 10 of them idle half the time; measured: Q2_K 12288 x 4096
    // at M = 1 30 % shorter, Q3_K 21 %, Q4_0 8192 x 2048 5 %).
    int most = std::min(16 - p.npw, units);
    if (most > 0) most = (int)div_up(units, div_up(units, most));
    for (int t = tiles; t >= 1; t /= 2)
        for (int kw = most; kw >= 1; kw--) {
            const int upw = (int)div_up(units, kw);
            const int tb = (int)div_up(t * 16 * cw * upw, 64);
            if (gemv2_lds(rows, planes, units, unit, t, kw, tb) <= limit) {
                p.ok = true;
                p.tiles = t;
                p.kw = kw;
                p.tb = tb;
                return p;
            }
        }
    (void)tiles_total;
    return p;
}

// The streamed decode kernel (gemv4_kernel): for one row of f32 activations
// or up to four of bytes.  `tiles` tiles a workgroup and `ks` waves a tile
// (contiguous ranges of units of K).  One matrix (`single`): one wave a tile,
// walking tiles; several: one tile of eight waves a workgroup.  Each wave's
// ring holds its whole stream when that fits, else a multiple of both a copy
// (64 chunks) and a unit.
struct Gemv4 {
    bool ok = false;
    int tiles, ks, npw, tb;
    int init = 8;  // copies a wave issues before the activations' barrier
};

static int gcd_int(int a, int b) { return b ? gcd_int(b, a % b) : a; }

Gemv4 gemv4_plan(uint32_t fmt, uint32_t group, uint64_t k, int rows, int planes, uint32_t x_kind, int tiles_total,
                 bool single) {
    Gemv4 p;
    const int unit = gemv_unit(fmt, group);
    const int len = (int)kh_block_len(fmt, group), bytes = (int)kh_block_bytes(fmt, group);
    if (!unit || !len || k == 0) return p;
    const int ub = (len >= unit ? 1 : unit / len) * bytes;
    const int cw = (ub + (bytes % 4 ? 2 : 0) + 15) / 16;
    const int uc = 16 * cw;
    const int units = (int)div_up(k, unit);
    const int quads = rows * units * unit / 4;
    const size_t limit = 160 * 1024 - (fmt == KH_IQ3_S ? 2048 : 0);
    // Preparing waves: one pass of loads over the activations where eight
    // waves take them (256 quads a wave).
    p.npw = std::max(1, std::min(8, (int)div_up(quads, 256)));
    const int step = 64 / gcd_int(64, uc) * uc / 64;  // copies of lcm(64, uc) chunks
    const size_t span = (size_t)units * unit;
    auto head_of = [&](int tiles, int waves) {
        size_t h = 16 + (size_t)rows * planes * span + span + (size_t)rows * (span / 32) * 16 +
                   (size_t)tiles * waves * 16 * rows * 4;
        return (h + 15) / 16 * 16;
    };
    if (single) {
        // One matrix: one wave a tile, each wave walking every gridDim-th
        // tile after its first in one stream of copies (the workgroups that
        // are resident at once).  The ring: the fewest whole units, at least
        // two, in whole copies (one tile's stream when that is smaller and
        // whole units).  The tiles a workgroup: the fewest rounds of walking
        // waves, then the most walking waves a CU (the runtime's count of
        // the workgroups a CU holds: registers, waves and LDS).  Measured on
        // the 151936 x 4096 Q6_K table (80 VGPRs, 24 waves a CU): two-unit
        // rings, 8 walking and 4 preparing waves a workgroup, two a CU (16
        // walking waves a CU, 3 rounds) 113-117 us; 14 walking waves a CU
        // 132 us; 12, 121-145 us; four-unit rings with 8 walking waves a CU
        // 141 us.
        int tb = (2 * uc + step * 64 - 1) / (step * 64) * step;
        const int one = (int)div_up((uint64_t)units * uc, 64);
        if (one < tb && one * 64 % uc == 0) tb = one;
        long best_rounds = 0, best_w = 0;
        for (int T = 1; p.npw + T <= 16; T++) {
            const size_t lds = head_of(T, 1) + (size_t)T * tb * 1024;
            if (lds > limit) break;
            GemvArgs q{};
            int per_cu = 0;
            q.count = 1;
            q.k = (int)k;
            q.units = units;
            q.rows = rows;
            q.rows_total = rows;
            q.mchunks = 1;
            q.total_tiles = tiles_total;
            q.x_kind = x_kind;
            q.dma = 4;
            q.npw = p.npw;
            q.tiles = T;
            q.kw = 1;
            q.tb = tb;
            q.occupancy = &per_cu;
            if (launch_gemv(fmt, group, planes, q, nullptr) != hipSuccess || per_cu < 1)
                per_cu = std::max(1, std::min((int)((160 * 1024) / lds), 32 / (p.npw + T)));
            const long W = (long)per_cu * T;  // walking waves a CU
            const long rounds = (long)div_up((uint64_t)tiles_total, (uint64_t)cu_count() * W);
            if (p.ok && (rounds > best_rounds || (rounds == best_rounds && W < best_w))) continue;
            best_rounds = rounds;
            best_w = W;
            p.ok = true;
            p.tiles = T;
            p.ks = 1;
            p.tb = tb;
        }
        return p;
    }
    // Several matrices: one tile of eight waves a workgroup (two workgroups
    // a CU).
    const int T = 1;
    int ks = std::min(units, 8);
    for (; ks >= 1; ks--) {
        if (p.npw + T * ks > 16) continue;
        const int upw = (int)div_up(units, ks);
        const size_t head = head_of(T, ks);
        if (head >= limit) return p;
        const int whole = (int)div_up((uint64_t)upw * uc, 64);
        int tb = (int)((limit - head) / ((size_t)T * ks * 1024));
        if (tb >= whole) tb = whole;
        else tb = tb / step * step;
        if (tb * 64 < 2 * uc + 64 && tb < whole) continue;
        p.ok = true;
        p.tiles = T;
        p.ks = ks;
        p.tb = tb;
        return p;
    }
    return p;
}

// The decode kernel for one row of f32 activations (or up to four of
// bytes): picked by the launch's size, or forced by KH_DECODE_KERNEL
// ("staged": weights staged in LDS a workgroup at a time; "streamed":
// streamed through per-wave rings; a test hook, read at each call).
enum class DecodeKernel { AUTO, STAGED, STREAMED };
DecodeKernel decode_kernel() {
    const char *e = getenv("KH_DECODE_KERNEL");
    if (!e) return DecodeKernel::AUTO;
    if (!strcmp(e, "staged")) return DecodeKernel::STAGED;
    if (!strcmp(e, "streamed")) return DecodeKernel::STREAMED;
    return DecodeKernel::AUTO;
}

// The many-row product of float activations: the bf16 matrix cores
// (mmf_kernel), or int8 MFMAs on three fixed-point planes of the activations
// (mm_kernel).  The first from the row counts below, measured on Q8_0, Q4_0,
// Q4_K and Q6_K shapes at 5 to 512 rows: in its dot mode (blocks of 32
// without a minimum term) bf16 at every many-row count (Q8_0 [gate; up]
// 24576 x 4096 at 5 rows 46 us against 57), f16 and f32 from 64; otherwise
// bf16 and f16 from 96 (Q6_K and Q3_K, groups of 16, from 64: Q6_K 3072 x
// 8192 at 64 rows 49 us against 57, Q3_K 12288 x 4096 58 against 83), and f32
// never (its three planes of split weights are as fast or slower than the
// int8 planes at every measured count).
// KH_MANY_KERNEL ("float", "int8") forces one (a test hook read at each call).
bool mmf_dot_format(uint32_t fmt, uint32_t group) {
    switch (fmt) {
    case KH_Q8_0: case KH_Q4_0: case KH_Q5_0: case KH_IQ4_NL: return true;
    case KH_INT8: case KH_INT4: return group == 32 || group == 64 || group == 128;
    default: return false;
    }
}
bool use_mmf(uint32_t fmt, uint32_t group, uint64_t rows, int planes, uint32_t x_kind) {
    if (planes != 3 || !mm_group(fmt, group)) return false;
    const char *e = getenv("KH_MANY_KERNEL");
    if (e && !strcmp(e, "int8")) return false;
    if (e && !strcmp(e, "float")) return true;
    if (!mmf_dot_format(fmt, group))
        return (x_kind == KH_BF16 || x_kind == KH_F16) && rows >= (fmt == KH_Q6K || fmt == KH_Q3K ? 64u : 96u);
    return x_kind == KH_BF16 || rows >= 64;
}

// The split of an mmf launch: column groups of the kernel's weight rows, row
// tiles of 128 (the kernel recounts its own), K split as mm_split does.
MmSplit mmf_split(uint64_t rows, uint64_t k, const kh_weight *weights, const std::vector<uint32_t> &members) {
    const kh_weight &w = weights[members[0]];
    MmSplit m{};
    launch_mmf(w.format, w.group, 1, MmArgs{}, nullptr, &m.cols);
    m.mtiles = (int)div_up(rows, 128);
    m.ngroups = 0;
    for (uint32_t i : members) m.ngroups += (int)div_up(weights[i].n, m.cols);
    split_k_of(m, mm_unit(w.format, w.group), k);
    return m;
}

// The small-M kernel's bounded wait for its activations: 2^24 spins, or
// KH_SPIN_LIMIT from the environment (a test hook: negative gives up at once,
// which must leave NaN outputs, never wrong numbers).
#ifdef KH_TRACE
static int *g_trace = nullptr;
extern "C" void kh_debug_trace(int *p) { g_trace = p; }
#endif
int spin_limit() {
    const char *e = getenv("KH_SPIN_LIMIT");
    return e ? atoi(e) : 1 << 24;
}

// The workspace: the counters of the segment split (fixed, first), the
// prepared activations, then the partial sums.
struct Layout {
    uint64_t kpad;
    uint64_t counters_off, planes_off, xscale_off, xsum32_off, xsum16_off, xsumi16_off, xcopy_off;
    uint64_t fplanes_off;  // bf16 planes of the float many-row product
    uint64_t partials_off, total;
};

Layout layout(uint64_t rows, uint64_t k, int planes, uint64_t partial_floats, bool mmf) {
    Layout l{};
    l.kpad = align_up(std::max<uint64_t>(k, 64), 64);
    uint64_t at = 0;
    l.counters_off = at;
    at = align_up(at + MAX_COUNTERS * 4, 256);
    l.planes_off = at;
    at = align_up(at + rows * planes * l.kpad, 256);
    l.xscale_off = at;
    at = align_up(at + rows * (k / 32) * 4, 256);
    l.xsum32_off = at;
    at = align_up(at + rows * (k / 32) * 4, 256);
    l.xsum16_off = at;
    at = align_up(at + rows * (k / 16) * 4, 256);
    l.xsumi16_off = at;
    at = align_up(at + rows * (k / 16) * 4, 256);
    // A copy of x for the small-M product when x is not aligned for its
    // vector loads.
    l.xcopy_off = at;
    if (rows <= 16) at = align_up(at + rows * k * 4, 256);
    // Three bf16 planes a row (the most the float many-row product takes).
    l.fplanes_off = at;
    if (mmf) at = align_up(at + rows * 3 * l.kpad * 2, 256);
    l.partials_off = at;
    // Partial sums of the largest launch: segments x rows x columns.
    at = align_up(at + partial_floats * 4, 256);
    l.total = at;
    return l;
}

struct Checked {
    uint64_t width = 0, max_wgs = 0, partial_floats = 0;
    bool bytes = false;
    bool any_qmv = false;  // a launch of the many-row product (prepared activations)
    bool any_mmf = false;  // a launch of the float many-row product (bf16 planes)
    bool gemv_prep = false;  // a small-M launch in row chunks (prepared activations)
};

// One launch of the MFMA product: weights `members` (one format), rows
// r0 .. r0 + rows of the activations.
struct Launch {
    std::vector<uint32_t> members;
    int tiles;
    uint64_t r0;
    int rows;
    bool gemv;        // the small-M product (all rows in one launch)
    bool mm;          // the many-row product (rows r0 .. r0 + rows)
    bool mmf;         // ... of float activations on the bf16 matrix cores
    GemvSplit gsplit;
    Gemv2 g2;         // the decode kernel staged in LDS, when it applies
    Gemv4 g4;         // the streamed decode kernel, when it applies
    Split split;
    MmSplit msplit;
};

// Every launch of a product, in order: the weights of a format and group,
// MAX_WEIGHTS at a time, by chunks of activation rows.
template <class Fn>
void each_launch(const kh_weight *weights, uint32_t count, uint64_t k, uint64_t rows, int planes,
                 uint32_t x_kind, Fn fn) {
    std::vector<bool> done(count, false);
    for (uint32_t i = 0; i < count; i++) {
        if (done[i]) continue;
        const kh_weight &w = weights[i];
        if (generic_weight(w)) {
            done[i] = true;
            continue;
        }
        Launch L;
        for (uint32_t j = i; j < count && (int)L.members.size() < MAX_WEIGHTS; j++)
            if (!done[j] && weights[j].format == w.format && weights[j].group == w.group &&
                !generic_weight(weights[j])) {
                L.members.push_back(j);
                done[j] = true;
            }
        L.tiles = 0;
        for (uint32_t m : L.members) L.tiles += (int)div_up(weights[m].n, 16);
        if (L.tiles == 0) continue;
        int steps = (int)div_up(k, 64);
        int unit = gemv_unit(w.format, w.group);
        // The small-M product reads each matrix at 32-bit offsets.
        bool offsets32 = true;
        for (uint32_t m : L.members) offsets32 = offsets32 && weights[m].bytes < (1ull << 31);
        L.mm = false;
        L.mmf = false;
        // Up to four rows the small-M product; from five the many-row
        // product is faster (measured across formats and shapes).
        bool one_chunk = rows <= (uint64_t)std::min(GEMV_DIRECT_ROWS, gemv_max_rows(planes));
        if (unit && offsets32 && (one_chunk || (rows <= GEMV_ROWS && !mm_group(w.format, w.group)))) {
            L.gemv = true;
            L.r0 = 0;
            L.rows = (int)std::min<uint64_t>(rows, gemv_max_rows(planes));
            L.gsplit = gemv_split(k, unit, L.tiles, L.rows, planes, (int)div_up(rows, L.rows), L.rows < (int)rows);
            L.g2 = Gemv2{};
            L.g4 = Gemv4{};
            if (L.rows == (int)rows && (planes == 3 ? rows == 1 : rows <= 4)) {
                // A workgroup's tiles in one matrix: several only when every
                // matrix is a whole number of them.
                int most = L.gsplit.tiles;
                for (uint32_t m : L.members)
                    while (most > 1 && div_up(weights[m].n, 16) % most) most /= 2;
                L.g2 = gemv2_plan(w.format, w.group, k, L.rows, planes, L.tiles, most);
                // The streamed kernel where a launch takes several rounds of
                // the CUs (measured: the 151936 x 4096 Q6_K table at M = 1
                // 18 % shorter; launches of one round are as fast or faster
                // staged), or where the caller asks for it.
                const DecodeKernel dk = decode_kernel();
                if (dk == DecodeKernel::STREAMED || (dk == DecodeKernel::AUTO && L.tiles >= 8 * cu_count()))
                    L.g4 = gemv4_plan(w.format, w.group, k, L.rows, planes, x_kind, L.tiles, L.members.size() == 1);
            }
            fn(L);
            continue;
        }
        L.gemv = false;
        if (unit && offsets32 && mm_group(w.format, w.group)) {
            // Launches of at most 2 GiB of prepared activations each.
            L.mm = true;
            L.mmf = use_mmf(w.format, w.group, rows, planes, x_kind);
            uint64_t kpad = align_up(std::max<uint64_t>(k, 64), 64);
            uint64_t fit = L.mmf ? ((1ull << 31) - 1) / (6 * kpad) / 128 * 128
                                 : ((1ull << 31) - 1) / ((uint64_t)planes * kpad) / 64 * 64;
            for (uint64_t r0 = 0; r0 < rows; r0 += fit) {
                L.r0 = r0;
                L.rows = (int)std::min<uint64_t>(fit, rows - r0);
                L.msplit = L.mmf ? mmf_split((uint64_t)L.rows, k, weights, L.members)
                                 : mm_split((uint64_t)L.rows, k, weights, L.members, planes);
                fn(L);
            }
            continue;
        }
        L.mm = false;
        int chunk = rows_per_launch(w.format, planes);
        for (uint64_t r0 = 0; r0 < rows; r0 += chunk) {
            L.r0 = r0;
            L.rows = (int)std::min<uint64_t>(chunk, rows - r0);
            L.split = split_k((uint64_t)L.tiles, steps, L.rows, planes, w.format);
            fn(L);
        }
    }
}

int check(const kh_weight *weights, uint32_t count, uint64_t k, uint64_t rows, uint32_t flags,
          Checked &c) {
    if (count == 0) return KH_ERR_ARITY;
    if (!weights) return KH_ERR_NULL;
    if (k > (1ull << 30) || rows > (1ull << 31)) return KH_ERR_OVERFLOW;
    bool all_bytes = true;
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < count; i++) {
        const kh_weight &w = weights[i];
        uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
        if (len == 0) return KH_ERR_DTYPE;
        if (k % len) return KH_ERR_MISALIGNED;
        if (w.n > (1ull << 31)) return KH_ERR_OVERFLOW;
        if (w.bytes != w.n * (k / len) * size) return KH_ERR_SHAPE;
        if (w.n && k && !w.data) return KH_ERR_NULL;
        // Rows are read with 4-byte loads (kapel-cuda/src/quantized.rs:123-129
        // asks the same of its fast kernels).
        if ((uintptr_t)w.data & 3u) return KH_ERR_SHAPE;
        uint64_t sum = c.width + w.n;
        if (sum < c.width) return KH_ERR_OVERFLOW;
        c.width = sum;
        all_bytes = all_bytes && byte_format(w.format, w.group);
        tiles += div_up(w.n, 16);
    }
    if (c.width > (1ull << 31)) return KH_ERR_OVERFLOW;
    // kapel-cpu/src/matmul.rs:292-306: bytes only in place, up to 16 rows
    // (IN_PLACE_ROWS), unless the caller asks for them at every row count.
    const bool byte_rows = (flags & KH_BYTE_ACTIVATIONS_ALL_ROWS) || ((flags & KH_BYTE_ACTIVATIONS) && rows <= 16);
    c.bytes = byte_rows && all_bytes;
    c.max_wgs = div_up(tiles, 4) + count;
    if (c.max_wgs > MAX_COUNTERS) return KH_ERR_OVERFLOW;
    // The workspace holds what the launches of any activation type need (the
    // many-row kernel differs between bf16 / f16 and f32 rows).
    if (k > 0 && rows > 0)
        for (uint32_t kind : {(uint32_t)KH_F32, (uint32_t)KH_BF16})
            each_launch(weights, count, k, rows, c.bytes ? 1 : 3, kind, [&](const Launch &L) {
                if (L.gemv) {
                    c.gemv_prep = c.gemv_prep || L.rows < (int)rows;
                    return;
                }
                if (L.mmf) c.any_mmf = true;
                else c.any_qmv = true;
                if (L.mm) {
                    if (L.msplit.ks > 1)
                        c.partial_floats = std::max<uint64_t>(c.partial_floats,
                                                              (uint64_t)L.msplit.ks * L.rows * c.width);
                    return;
                }
                if (L.split.segs > 1)
                    c.partial_floats = std::max<uint64_t>(
                        c.partial_floats, (uint64_t)L.split.segs * L.rows * L.tiles * 16);
            });
    return KH_OK;
}

hipError_t plan_and_launch(const kh_weight *weights, uint32_t count, uint64_t k, uint32_t x_kind,
                           const void *x, uint64_t rows, uint32_t out_kind, void *out,
                           const Checked &c, uint8_t *ws, const Layout &l, bool reuse,
                           hipStream_t s) {
    int planes = c.bytes ? 1 : 3;
    hipError_t err;
    // What this call's launches read: int8 planes, bf16 planes.
    bool need_qmv = false, need_mmf = false;
    each_launch(weights, count, k, rows, planes, x_kind, [&](const Launch &L) {
        if (L.gemv) return;
        if (L.mmf) need_mmf = true;
        else need_qmv = true;
    });
    // The activations, once for all weights.
    if ((need_qmv || c.gemv_prep) && !reuse) {
        PrepArgs p{};
        p.x_kind = x_kind;
        p.x = x;
        p.rows = rows;
        p.k = k;
        p.kpad = l.kpad;
        p.planes = planes;
        p.planes_out = reinterpret_cast<int8_t *>(ws + l.planes_off);
        p.xscale = reinterpret_cast<float *>(ws + l.xscale_off);
        p.xsum32 = reinterpret_cast<float *>(ws + l.xsum32_off);
        p.xsum16 = reinterpret_cast<float *>(ws + l.xsum16_off);
        p.xsumi16 = reinterpret_cast<int32_t *>(ws + l.xsumi16_off);
        if ((err = launch_prep(p, s)) != hipSuccess) return err;
    }
    // bf16 planes, once for all weights: bf16 rows as they are, f16 rows in
    // two planes, f32 rows in three.
    const int fplanes = x_kind == KH_BF16 ? 1 : x_kind == KH_F16 ? 2 : 3;
    // bf16 rows already are the one plane when K is a multiple of 64 (no
    // padding) and x is 16-byte aligned: the kernel reads x itself.
    const bool direct = x_kind == KH_BF16 && k % 64 == 0 && ((uintptr_t)x & 15u) == 0;
    const uint8_t *fbase = direct ? static_cast<const uint8_t *>(x) : ws + l.fplanes_off;
    if (need_mmf && !reuse && !direct) {
        PrepBf16Args p{};
        p.x_kind = x_kind;
        p.x = x;
        p.rows = rows;
        p.k = k;
        p.kpad = l.kpad;
        p.planes = fplanes;
        p.out = reinterpret_cast<uint16_t *>(ws + l.fplanes_off);
        if ((err = launch_prep_bf16(p, s)) != hipSuccess) return err;
    }
    // Column of each weight.
    std::vector<uint64_t> col0(count);
    uint64_t col = 0;
    for (uint32_t i = 0; i < count; i++) {
        col0[i] = col;
        col += weights[i].n;
    }
    for (uint32_t i = 0; i < count; i++) {
        const kh_weight &w = weights[i];
        if (!generic_weight(w) || w.n == 0) continue;
        GenericArgs g{};
        g.format = w.format;
        g.group = w.group;
        g.w = static_cast<const uint8_t *>(w.data);
        g.n = w.n;
        g.row_bytes = w.bytes / w.n;
        g.k = k;
        g.rows = rows;
        g.x_kind = x_kind;
        g.x = x;
        g.out_kind = out_kind;
        g.out = out;
        g.col0 = col0[i];
        g.out_stride = c.width;
        if ((err = launch_generic(g, s)) != hipSuccess) return err;
    }
    err = hipSuccess;
    each_launch(weights, count, k, rows, planes, x_kind, [&](const Launch &L) {
        if (err != hipSuccess) return;
        const kh_weight &w = weights[L.members[0]];
        if (L.gemv) {
            GemvArgs a{};
            a.spin_limit = spin_limit();
#ifdef KH_TRACE
            a.trace = g_trace;
#endif
            a.count = (int)L.members.size();
            int tiles = 0;
            for (int m = 0; m < a.count; m++) {
                const kh_weight &wm = weights[L.members[m]];
                a.w[m] = static_cast<const uint8_t *>(wm.data);
                a.wbytes[m] = (uint32_t)wm.bytes;
                a.n[m] = wm.n;
                a.col0[m] = col0[L.members[m]];
                a.tile0[m] = tiles;
                tiles += (int)div_up(wm.n, 16);
            }
            uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
            a.row_bytes = k / len * size;
            a.k = (int)k;
            a.units = L.gsplit.units;
            a.chunk = L.gsplit.chunk;
            a.total_tiles = tiles;
            a.tiles = L.gsplit.tiles;
            a.tiles_log2 = a.tiles == 4 ? 2 : a.tiles == 2 ? 1 : 0;
            a.kw = L.gsplit.kw;
            a.rows = L.rows;
            a.rows_total = (int)rows;
            a.mchunks = (int)div_up(rows, L.rows);
            a.hi = 65536.0f;
            a.shift = 8;
            if (a.mchunks > 1) {
                a.pplanes = reinterpret_cast<const int8_t *>(ws + l.planes_off);
                a.pkpad = l.kpad;
                a.pxscale = reinterpret_cast<const float *>(ws + l.xscale_off);
                a.pxsum32 = reinterpret_cast<const float *>(ws + l.xsum32_off);
                a.pxsum16 = reinterpret_cast<const float *>(ws + l.xsum16_off);
            }
            a.x_kind = x_kind;
            a.x = x;
            if (a.mchunks == 1 && (uintptr_t)x % (x_kind == KH_F32 ? 16 : 8)) {
                void *copy = ws + l.xcopy_off;
                hipError_t e = hipMemcpyAsync(copy, x, rows * k * kind_bytes(x_kind),
                                              hipMemcpyDeviceToDevice, s);
                if (e != hipSuccess) {
                    err = e;
                    return;
                }
                a.x = copy;
            }
            a.out_kind = out_kind;
            a.out = out;
            a.out_stride = c.width;
            a.width = c.width;
            if (L.g4.ok) {
                a.dma = 4;
                a.tiles = L.g4.tiles;
                a.npw = L.g4.npw;
                a.kw = L.g4.ks;
                a.tb = L.g4.tb;
                a.chunk = L.g4.init;  // copies before the barrier
            } else if (L.g2.ok) {
                a.dma = 1;
                a.tiles = L.g2.tiles;
                a.npw = L.g2.npw;
                a.kw = L.g2.kw;
                a.tb = L.g2.tb;
            }
            err = launch_gemv(w.format, w.group, planes, a, s);
            return;
        }
        if (L.mm) {
            MmArgs a{};
            a.count = (int)L.members.size();
            int ng = 0;
            for (int m = 0; m < a.count; m++) {
                const kh_weight &wm = weights[L.members[m]];
                a.w[m] = static_cast<const uint8_t *>(wm.data);
                a.wbytes[m] = (uint32_t)wm.bytes;
                a.n[m] = wm.n;
                a.col0[m] = col0[L.members[m]];
                a.ng0[m] = ng;
                ng += (int)div_up(wm.n, L.msplit.cols);
            }
            uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
            const int g = mm_group(w.format, w.group);
            a.row_bytes = k / len * size;
            a.k = (int)k;
            a.units = L.msplit.units;
            a.ups = L.msplit.ups;
            a.ks = L.msplit.ks;
            a.ngroups = L.msplit.ngroups;
            a.mtiles = L.msplit.mtiles;
            a.wm = L.msplit.wm;
            a.wmg = L.msplit.wmg;
            a.rows = L.rows;
            const uint64_t r0 = L.r0;
            a.out_kind = out_kind;
            a.out = static_cast<uint8_t *>(out) + r0 * c.width * kind_bytes(out_kind);
            a.out_stride = c.width;
            a.width = c.width;
            a.partials = reinterpret_cast<float *>(ws + l.partials_off);
            if (L.mmf) {
                a.planes = reinterpret_cast<const int8_t *>(fbase) + r0 * fplanes * l.kpad * 2;
                a.planes_bytes = (uint32_t)((uint64_t)L.rows * fplanes * l.kpad * 2);
                a.kpad = l.kpad;
                err = launch_mmf(w.format, w.group, fplanes, a, s, nullptr);
                if (err == hipSuccess && a.ks > 1) err = launch_mm_reduce(a, s);
                return;
            }
            a.planes = reinterpret_cast<const int8_t *>(ws + l.planes_off) + r0 * planes * l.kpad;
            a.planes_bytes = (uint32_t)((uint64_t)L.rows * planes * l.kpad);
            a.kpad = l.kpad;
            a.xscale = reinterpret_cast<const float *>(ws + l.xscale_off) + r0 * (k / 32);
            a.xsum = g == 16 ? reinterpret_cast<const float *>(ws + l.xsum16_off) + r0 * (k / 16)
                             : reinterpret_cast<const float *>(ws + l.xsum32_off) + r0 * (k / 32);
            a.hi = 65536.0f;
            a.shift = 8;
            err = launch_mm(w.format, w.group, planes, a, s);
            if (err == hipSuccess && a.ks > 1) err = launch_mm_reduce(a, s);
            return;
        }
        QmvArgs a{};
        a.count = (int)L.members.size();
        int tiles = 0;
        for (int m = 0; m < a.count; m++) {
            const kh_weight &wm = weights[L.members[m]];
            a.w[m] = static_cast<const uint8_t *>(wm.data);
            a.n[m] = wm.n;
            a.col0[m] = col0[L.members[m]];
            a.tile0[m] = tiles;
            tiles += (int)div_up(wm.n, 16);
        }
        uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
        a.row_bytes = k / len * size;
        a.k = (int)k;
        a.steps = (int)div_up(k, 64);
        a.kpad = l.kpad;
        a.out_kind = out_kind;
        a.width = c.width;
        a.out_stride = c.width;
        a.partials = reinterpret_cast<float *>(ws + l.partials_off);
        a.pwidth = (uint64_t)tiles * 16;
        a.counters = reinterpret_cast<int *>(ws + l.counters_off);
        uint64_t r0 = L.r0;
        a.rows = L.rows;
        a.segs = L.split.segs;
        a.seg_steps = L.split.seg_steps;
        a.planes = reinterpret_cast<const int8_t *>(ws + l.planes_off) + r0 * planes * l.kpad;
        a.xscale = reinterpret_cast<const float *>(ws + l.xscale_off) + r0 * (k / 32);
        a.xsum32 = reinterpret_cast<const float *>(ws + l.xsum32_off) + r0 * (k / 32);
        a.xsum16 = reinterpret_cast<const float *>(ws + l.xsum16_off) + r0 * (k / 16);
        a.xsumi16 = reinterpret_cast<const int32_t *>(ws + l.xsumi16_off) + r0 * (k / 16);
        a.out = static_cast<uint8_t *>(out) + r0 * c.width * kind_bytes(out_kind);
        dim3 grid((unsigned)div_up(tiles, 4), (unsigned)L.split.segs);
        err = launch_qmv(w.format, w.group, planes, a, grid, L.split.lds, s);
    });
    return err;
}

}  // namespace

extern "C" {

const char *kh_version(void) { return "kapel_hip 0.1 gfx950"; }

const char *kh_error_string(int status) {
    switch (status) {
    case KH_OK: return "ok";
    case KH_ERR_ARITY: return "quantized_matmul: expected 2 or more inputs";
    case KH_ERR_DTYPE: return "quantized_matmul: unsupported format or float type";
    case KH_ERR_SHAPE: return "quantized_matmul: expected x [..., K] and w [N, K]";
    case KH_ERR_MISALIGNED: return "quantized_matmul: K is not a whole number of blocks";
    case KH_ERR_OVERFLOW: return "quantized_matmul: a size overflows the kernels' range";
    case KH_ERR_WORKSPACE: return "quantized_matmul: workspace missing or too small";
    case KH_ERR_HIP: return "quantized_matmul: HIP runtime error";
    case KH_ERR_NULL: return "quantized_matmul: a required pointer is null";
    default: return "unknown status";
    }
}

uint32_t kh_block_len(uint32_t format, uint32_t group) {
    switch (format) {
    case KH_INT8: return group;
    case KH_INT4: return (group % 2 == 0) ? group : 0;
    case KH_Q8_0: case KH_Q4_0: case KH_Q4_1: case KH_Q5_0: case KH_Q5_1: case KH_IQ4_NL: return 32;
    case KH_Q2K: case KH_Q3K: case KH_Q4K: case KH_Q5K: case KH_Q6K: case KH_IQ4_XS: case KH_IQ3_S:
        return 256;
    default: return 0;
    }
}

uint32_t kh_block_bytes(uint32_t format, uint32_t group) {
    switch (format) {
    case KH_INT8: return group ? 4 + group : 0;
    case KH_INT4: return (group && group % 2 == 0) ? 4 + group / 2 : 0;
    case KH_Q8_0: return 34;
    case KH_Q4_0: return 18;
    case KH_Q4_1: return 20;
    case KH_Q5_0: return 22;
    case KH_Q5_1: return 24;
    case KH_Q2K: return 84;
    case KH_Q3K: return 110;
    case KH_Q4K: return 144;
    case KH_Q5K: return 176;
    case KH_Q6K: return 210;
    case KH_IQ4_NL: return 18;
    case KH_IQ4_XS: return 136;
    case KH_IQ3_S: return 110;
    default: return 0;
    }
}

uint64_t kh_qmatmul_workspace(const kh_weight *weights, uint32_t count, uint64_t k, uint64_t rows,
                              uint32_t flags) {
    Checked c;
    if (check(weights, count, k, rows, flags, c) != KH_OK) return 0;
    return layout(rows, k, c.bytes ? 1 : 3, c.partial_floats, c.any_mmf).total;
}

int kh_qmatmul(const kh_weight *weights, uint32_t count, uint64_t k, uint32_t x_kind,
               const void *x, uint64_t rows, uint32_t out_kind, void *out, uint32_t flags,
               void *workspace, uint64_t workspace_bytes, void *stream) {
    Checked c;
    int status = check(weights, count, k, rows, flags, c);
    if (status != KH_OK) return status;
    if (!float_kind(x_kind) || !float_kind(out_kind)) return KH_ERR_DTYPE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (rows == 0 || c.width == 0) return KH_OK;
    if (!out) return KH_ERR_NULL;
    if (k == 0) {
        // A sum over nothing: zeros (conformity.rs:1424-1428).
        return launch_fill_bytes(static_cast<uint8_t *>(out), rows * c.width * kind_bytes(out_kind), s) ==
                       hipSuccess
                   ? KH_OK
                   : KH_ERR_HIP;
    }
    if (!x) return KH_ERR_NULL;
    Layout l = layout(rows, k, c.bytes ? 1 : 3, c.partial_floats, c.any_mmf);
    if (!workspace || workspace_bytes < l.total || ((uintptr_t)workspace & 255u))
        return KH_ERR_WORKSPACE;
    hipError_t err = plan_and_launch(weights, count, k, x_kind, x, rows, out_kind, out, c,
                                     static_cast<uint8_t *>(workspace), l,
                                     (flags & KH_REUSE_ACTIVATIONS) != 0, s);
    return err == hipSuccess ? KH_OK : KH_ERR_HIP;
}

}  // extern "C"

// The scratch of kh_qmatmul_static: one array per device, for callers that
// cannot allocate.  Host code never names it after set-up: the array's
// device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) uint8_t scratch[KH_STATIC_SCRATCH_BYTES];

namespace {

struct ScratchOf {
    std::once_flag flag;
    uint8_t *ptr = nullptr;
    hipError_t err = hipSuccess;
};
ScratchOf scratch_of[MAX_DEVICES];

// This device's copy of the array; the first call on the device also clears
// its counters (on the caller's stream, by a fill kernel: no memset node for
// a caller that captures the call in a graph).
hipError_t device_scratch(hipStream_t s, uint8_t *&out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    ScratchOf &slot = scratch_of[dev];
    std::call_once(slot.flag, [&] {
        void *p = nullptr;
        slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (slot.err == hipSuccess) {
            slot.ptr = static_cast<uint8_t *>(p);
            slot.err = launch_fill(reinterpret_cast<uint32_t *>(slot.ptr), MAX_COUNTERS, s);
        }
    });
    out = slot.ptr;
    return slot.err;
}

}  // namespace

extern "C" {

int kh_qmatmul_static(const kh_weight *weights, uint32_t count, uint64_t k, uint32_t x_kind,
                      const void *x, uint64_t rows, uint32_t out_kind, void *out, uint32_t flags,
                      void *stream) {
    // The sizes are checked before anything touches the device.
    const uint64_t need = kh_qmatmul_workspace(weights, count, k, rows, flags);
    if (need > KH_STATIC_SCRATCH_BYTES) return KH_ERR_WORKSPACE;
    // A refused call (its status from kh_qmatmul) touches no scratch.
    if (need == 0) return kh_qmatmul(weights, count, k, x_kind, x, rows, out_kind, out, flags, nullptr, 0, stream);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t *ws = nullptr;
    if (device_scratch(s, ws) != hipSuccess) return KH_ERR_HIP;
    return kh_qmatmul(weights, count, k, x_kind, x, rows, out_kind, out, flags, ws, KH_STATIC_SCRATCH_BYTES,
                      stream);
}

int kh_quantize_x(uint32_t x_kind, const void *x, uint64_t rows, uint64_t k, int8_t *q,
                  float *scale, float *sums32, void *stream) {
    if (!float_kind(x_kind)) return KH_ERR_DTYPE;
    if (k % 32) return KH_ERR_MISALIGNED;
    if (rows * k == 0) return KH_OK;
    if (!x || !q || !scale) return KH_ERR_NULL;
    PrepArgs p{};
    p.x_kind = x_kind;
    p.x = x;
    p.rows = rows;
    p.k = k;
    p.kpad = k;
    p.planes = 1;
    p.q_out = q;
    p.q_scale = scale;
    p.q_sums = sums32;
    return launch_prep(p, static_cast<hipStream_t>(stream)) == hipSuccess ? KH_OK : KH_ERR_HIP;
}

int kh_block_dots(const kh_weight *weight, uint64_t k, const int8_t *q, uint64_t rows,
                  int32_t *dots, void *workspace, uint64_t workspace_bytes, void *stream) {
    Checked c;
    int status = check(weight, 1, k, rows, KH_BYTE_ACTIVATIONS_ALL_ROWS, c);
    if (status != KH_OK) return status;
    if (!c.bytes) return KH_ERR_DTYPE;
    if (rows == 0 || weight->n == 0 || k == 0) return KH_OK;
    if (!q || !dots) return KH_ERR_NULL;
    Layout l = layout(rows, k, 1, c.partial_floats, false);
    if (!workspace || workspace_bytes < l.total || ((uintptr_t)workspace & 255u))
        return KH_ERR_WORKSPACE;
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    PrepArgs p{};
    p.q_in = q;
    p.rows = rows;
    p.k = k;
    p.kpad = l.kpad;
    p.planes = 1;
    p.planes_out = reinterpret_cast<int8_t *>(ws + l.planes_off);
    p.xscale = reinterpret_cast<float *>(ws + l.xscale_off);
    p.xsum32 = reinterpret_cast<float *>(ws + l.xsum32_off);
    p.xsum16 = reinterpret_cast<float *>(ws + l.xsum16_off);
    p.xsumi16 = reinterpret_cast<int32_t *>(ws + l.xsumi16_off);
    const kh_weight &w = *weight;
    int unit = gemv_unit(w.format, w.group);
    if (unit && rows <= GEMV_ROWS && (uintptr_t)q % 4 == 0 && w.bytes < (1ull << 31)) {
        // The bytes go through the small-M product's own preparation.
        GemvArgs g{};
        g.spin_limit = spin_limit();
        g.count = 1;
        g.w[0] = static_cast<const uint8_t *>(w.data);
        g.wbytes[0] = (uint32_t)w.bytes;
        g.n[0] = w.n;
        uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
        g.row_bytes = k / len * size;
        g.k = (int)k;
        const int chunk_rows = (int)std::min<uint64_t>(rows, gemv_max_rows(1));
        GemvSplit sp = gemv_split(k, unit, (int)div_up(w.n, 16), chunk_rows, 1, (int)div_up(rows, chunk_rows), false);
        g.units = sp.units;
        g.chunk = sp.chunk;
        g.total_tiles = (int)div_up(w.n, 16);
        g.tiles = sp.tiles;
        g.tiles_log2 = g.tiles == 4 ? 2 : g.tiles == 2 ? 1 : 0;
        g.kw = sp.kw;
        g.rows = chunk_rows;
        g.rows_total = (int)rows;
        g.mchunks = (int)div_up(rows, chunk_rows);
        g.x_kind = KH_I8_INTERNAL;
        g.x = q;
        g.dots = dots;
        g.width = w.n;
        return launch_gemv(w.format, w.group, 1, g, s) == hipSuccess ? KH_OK : KH_ERR_HIP;
    }
    if (launch_prep(p, s) != hipSuccess) return KH_ERR_HIP;
    QmvArgs a{};
    a.count = 1;
    a.w[0] = static_cast<const uint8_t *>(w.data);
    a.n[0] = w.n;
    a.col0[0] = 0;
    a.tile0[0] = 0;
    uint32_t len = kh_block_len(w.format, w.group), size = kh_block_bytes(w.format, w.group);
    a.row_bytes = k / len * size;
    a.k = (int)k;
    a.steps = (int)div_up(k, 64);
    a.kpad = l.kpad;
    a.width = w.n;
    a.out_stride = w.n;
    a.dots = dots;
    a.signed_offset = w.format == KH_Q6K ? 32 : 0;
    int tiles = (int)div_up(w.n, 16);
    int chunk = rows_per_launch(w.format, 1);
    for (uint64_t r0 = 0; r0 < rows; r0 += chunk) {
        int rc = (int)std::min<uint64_t>(chunk, rows - r0);
        Split sp = split_k((uint64_t)tiles, a.steps, rc, 1, w.format);
        a.rows = rc;
        a.segs = sp.segs;
        a.seg_steps = sp.seg_steps;
        a.planes = reinterpret_cast<const int8_t *>(ws + l.planes_off) + r0 * l.kpad;
        a.xscale = reinterpret_cast<const float *>(ws + l.xscale_off) + r0 * (k / 32);
        a.xsum32 = reinterpret_cast<const float *>(ws + l.xsum32_off) + r0 * (k / 32);
        a.xsum16 = reinterpret_cast<const float *>(ws + l.xsum16_off) + r0 * (k / 16);
        a.xsumi16 = reinterpret_cast<const int32_t *>(ws + l.xsumi16_off) + r0 * (k / 16);
        a.dots = dots + r0 * w.n * (k / 16);
        dim3 grid((unsigned)div_up(tiles, 4), (unsigned)sp.segs);
        if (launch_qmv(w.format, w.group, 1, a, grid, sp.lds, s) != hipSuccess) return KH_ERR_HIP;
    }
    return KH_OK;
}

static int dequant(const kh_weight *weight, uint64_t k, uint64_t first, uint64_t count,
                   const uint32_t *indices, uint32_t out_kind, void *out, void *stream) {
    if (!weight) return KH_ERR_NULL;
    uint32_t len = kh_block_len(weight->format, weight->group);
    uint32_t size = kh_block_bytes(weight->format, weight->group);
    if (len == 0) return KH_ERR_DTYPE;
    if (!float_kind(out_kind)) return KH_ERR_DTYPE;
    if (k % len) return KH_ERR_MISALIGNED;
    if (weight->bytes != weight->n * (k / len) * size) return KH_ERR_SHAPE;
    if (!indices && first + count > weight->n) return KH_ERR_SHAPE;
    if (count * k == 0) return KH_OK;
    if (!out || !weight->data) return KH_ERR_NULL;
    DequantArgs a{};
    a.format = weight->format;
    a.group = weight->group;
    a.w = static_cast<const uint8_t *>(weight->data);
    a.n = weight->n;
    a.row_bytes = k / len * size;
    a.k = k;
    a.first = first;
    a.count = count;
    a.indices = indices;
    a.out_kind = out_kind;
    a.out = out;
    return launch_dequantize(a, static_cast<hipStream_t>(stream)) == hipSuccess ? KH_OK : KH_ERR_HIP;
}

int kh_dequantize(const kh_weight *weight, uint64_t k, uint64_t first, uint64_t count,
                  uint32_t out_kind, void *out, void *stream) {
    return dequant(weight, k, first, count, nullptr, out_kind, out, stream);
}

int kh_dequantize_rows(const kh_weight *weight, uint64_t k, const uint32_t *indices, uint64_t count,
                       uint32_t out_kind, void *out, void *stream) {
    if (count && !indices) return KH_ERR_NULL;
    return dequant(weight, k, 0, count, indices, out_kind, out, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- experts
namespace {

// The shapes of an experts' product (kapel-ops/src/experts.rs:166-225).
struct Experts {
    uint64_t n = 0, expert_bytes = 0, routes = 0, xrows = 0, xcopy = 0;
    int planes = 3;
    bool mfma = false;
};

int expert_check(const kh_weight *w, uint32_t experts, uint64_t k, uint64_t tokens, uint32_t topk,
                 uint32_t per_route, uint32_t x_kind, uint32_t flags, Experts &e) {
    if (!w) return KH_ERR_NULL;
    if (!float_kind(x_kind)) return KH_ERR_DTYPE;
    const uint32_t len = kh_block_len(w->format, w->group), size = kh_block_bytes(w->format, w->group);
    if (len == 0) return KH_ERR_DTYPE;
    if (experts == 0 || w->n % experts) return KH_ERR_SHAPE;
    if (k % len) return KH_ERR_MISALIGNED;
    if (k > (1ull << 30) || tokens > (1ull << 31) || topk > (1u << 16)) return KH_ERR_OVERFLOW;
    if (w->bytes != w->n * (k / len) * size) return KH_ERR_SHAPE;
    if (w->n && k && !w->data) return KH_ERR_NULL;
    if ((uintptr_t)w->data & 3u) return KH_ERR_SHAPE;
    e.n = w->n / experts;
    e.expert_bytes = e.n * (k / len) * size;
    // Each expert's matrix is read at 32-bit offsets.
    if (e.expert_bytes >= (1ull << 31)) return KH_ERR_OVERFLOW;
    e.routes = tokens * topk;
    if (e.routes > (1ull << 31)) return KH_ERR_OVERFLOW;
    e.xrows = per_route ? e.routes : tokens;
    e.xcopy = align_up(e.xrows * k * kind_bytes(x_kind), 256);
    e.planes = (flags & KH_BYTE_ACTIVATIONS) && byte_format(w->format, w->group) ? 1 : 3;
    e.mfma = mfma_format(w->format, w->group) && gemv_unit(w->format, w->group) != 0;
    return KH_OK;
}

}  // namespace

extern "C" {

uint64_t kh_expert_matmul_workspace(const kh_weight *weight, uint32_t experts, uint64_t k,
                                    uint64_t tokens, uint32_t topk, uint32_t per_route,
                                    uint32_t x_kind, uint32_t flags) {
    Experts e;
    if (expert_check(weight, experts, k, tokens, topk, per_route, x_kind, flags, e) != KH_OK) return 0;
    return e.xcopy;
}

int kh_expert_matmul(const kh_weight *weight, uint32_t experts, uint64_t k, uint32_t x_kind,
                     const void *x, uint64_t tokens, uint32_t topk, uint32_t per_route,
                     const uint32_t *idx, uint32_t out_kind, void *out, uint32_t flags,
                     void *workspace, uint64_t workspace_bytes, void *stream) {
    Experts e;
    int status = expert_check(weight, experts, k, tokens, topk, per_route, x_kind, flags, e);
    if (status != KH_OK) return status;
    if (!float_kind(out_kind)) return KH_ERR_DTYPE;
    if (e.routes == 0 || e.n == 0) return KH_OK;
    if (!out || !idx) return KH_ERR_NULL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (k == 0)
        return launch_fill_bytes(static_cast<uint8_t *>(out), e.routes * e.n * kind_bytes(out_kind), s) ==
                       hipSuccess
                   ? KH_OK
                   : KH_ERR_HIP;
    if (!x) return KH_ERR_NULL;
    // The small-M kernel reads activations by 16 (f32) or 8 bytes.
    if ((uintptr_t)x % (x_kind == KH_F32 ? 16 : 8)) {
        if (!workspace || workspace_bytes < e.xcopy || ((uintptr_t)workspace & 255u)) return KH_ERR_WORKSPACE;
        if (hipMemcpyAsync(workspace, x, e.xrows * k * kind_bytes(x_kind), hipMemcpyDeviceToDevice, s) !=
            hipSuccess)
            return KH_ERR_HIP;
        x = workspace;
    }
    const uint32_t len = kh_block_len(weight->format, weight->group);
    const uint32_t size = kh_block_bytes(weight->format, weight->group);
    const uint8_t *data = static_cast<const uint8_t *>(weight->data);
    if (!e.mfma) {
        GenericArgs g{};
        g.format = weight->format;
        g.group = weight->group;
        g.w = data;
        g.n = e.n;
        g.row_bytes = k / len * size;
        g.k = k;
        g.rows = e.routes;
        g.x_kind = x_kind;
        g.x = x;
        g.out_kind = out_kind;
        g.out = out;
        g.col0 = 0;
        g.out_stride = e.n;
        g.experts = idx;
        g.n_experts = experts;
        g.topk = (int)topk;
        g.per_route = per_route ? 1 : 0;
        g.expert_bytes = e.expert_bytes;
        return launch_generic(g, s) == hipSuccess ? KH_OK : KH_ERR_HIP;
    }
    // One route a chunk of the small-M kernel: its expert's tiles.
    const int unit = gemv_unit(weight->format, weight->group);
    const int tiles = (int)div_up(e.n, 16);
    GemvSplit sp = gemv_split(k, unit, tiles, 1, e.planes, (int)e.routes, false);
    const uint64_t groups = div_up(div_up(tiles, sp.tiles), 8) * 8;
    if (groups * e.routes >= (1ull << 31)) return KH_ERR_OVERFLOW;
    GemvArgs a{};
    a.spin_limit = spin_limit();
    a.count = 1;
    a.w[0] = data;
    a.wbytes[0] = (uint32_t)e.expert_bytes;
    a.n[0] = e.n;
    a.row_bytes = k / len * size;
    a.k = (int)k;
    a.units = sp.units;
    a.chunk = sp.chunk;
    a.total_tiles = tiles;
    a.tiles = sp.tiles;
    a.tiles_log2 = a.tiles == 4 ? 2 : a.tiles == 2 ? 1 : 0;
    a.kw = sp.kw;
    a.rows = 1;
    a.rows_total = (int)e.routes;
    a.mchunks = (int)e.routes;
    a.hi = 65536.0f;
    a.shift = 8;
    a.x_kind = x_kind;
    a.x = x;
    a.out_kind = out_kind;
    a.out = out;
    a.out_stride = e.n;
    a.width = e.n;
    a.experts = idx;
    a.n_experts = experts;
    a.topk = (int)topk;
    a.per_route = per_route ? 1 : 0;
    return launch_gemv(weight->format, weight->group, e.planes, a, s) == hipSuccess ? KH_OK : KH_ERR_HIP;
}

}  // extern "C"
