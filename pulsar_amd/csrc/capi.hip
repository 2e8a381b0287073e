// C ABI of libpulsar_w4a16.so: argument checks, kernel selection, workspace
// carving, launches.  Declarations and reference citations: include/pulsar_w4a16.h.
#include "pulsar_w4a16.h"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "w4a16_common.h"
#include "w4a16_kernels.h"

using namespace pw4;

namespace pw4 {
// pw4_time_next_kernel's events, armed for the calling thread's next GEMM call
thread_local KernelEvents g_armed_events;

KernelEvents take_kernel_events() {
    const KernelEvents ev = g_armed_events;
    g_armed_events = KernelEvents{};
    return ev;
}
}  // namespace pw4

namespace {

thread_local char g_last_hip_error[256] = "";

int hip_fail(hipError_t e) {
    std::snprintf(g_last_hip_error, sizeof(g_last_hip_error), "%s (%d)", hipGetErrorString(e), (int)e);
    return PW4_ERR_HIP;
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int v = g_cu_count[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        g_cu_count[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// LDS of one decode workgroup: the hard limit (160 KB per CU minus the
// static part) and the per-CU capacity used to judge residency.
constexpr size_t kDecodeLdsLimit = 152 * 1024;
constexpr size_t kLdsPerCu = 160 * 1024;
// Arrival counters of the decode K split: one int32 per workgroup column.
// Zero region of a workspace: arrival counters, then exchange-tree slots.
constexpr size_t kZeroRegion = PW4_ZERO_REGION_BYTES;
constexpr size_t kCounterBytes = 65536;
constexpr int64_t kMaxCounterCols = (int64_t)(kCounterBytes / sizeof(int32_t));
constexpr size_t kSlotBytes = kZeroRegion - kCounterBytes;

// Plan overrides for tuning sweeps and tests.  They are read from the
// environment on every call only when PW4_PLAN_OVERRIDES=1 was set when the
// process first planned a GEMM; otherwise no call reads the environment (six
// lookups cost ~0.5 us of host time per call with a typical environment).
const char* plan_env(const char* name) {
    static const bool enabled = [] {
        const char* e = std::getenv("PW4_PLAN_OVERRIDES");
        return e != nullptr && e[0] == '1';
    }();
    return enabled ? std::getenv(name) : nullptr;
}

// Act-order repack overrides for tuning sweeps and tests: the column block
// width (8, 16, 32 or 64) and the number of workgroups; unset = heuristic.
int repack_cols_override() {
    const char* e = plan_env("PW4_REPACK_COLS");
    const int v = e ? std::atoi(e) : 0;
    return (v == 8 || v == 16 || v == 32 || v == 64) ? v : 0;
}
int repack_grid_override() {
    const char* e = plan_env("PW4_REPACK_GRID");
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 0;
}

// Act-order gather override for tuning sweeps: 1 stages the rows in LDS, 0
// reads them directly, -1 (unset) = heuristic.
int gather_staged_override() {
    const char* e = plan_env("PW4_GATHER_STAGED");
    return e ? std::atoi(e) : -1;
}

// Decode column width override (16, 32 or 64) for tuning sweeps; 0 = heuristic.
int decode_nb_override() {
    const char* e = plan_env("PW4_DECODE_NB");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v == 16 || v == 32 || v == 64) ? v : 0;
}

// Prefill tile override (128 or 256) for tuning sweeps; 0 = heuristic.
int prefill_tile_override() {
    const char* e = plan_env("PW4_PREFILL_TILE");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v == 128 || v == 256) ? v : 0;
}

// Rows of the 256-wide prefill tiles (256 or 128) and the K-slice count of
// an unforced prefill plan (1..64), for tuning sweeps; 0 = heuristic.
int prefill_rows_override() {
    const char* e = plan_env("PW4_PREFILL_ROWS");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v == 128 || v == 256) ? v : 0;
}
int prefill_splits_override() {
    const char* e = plan_env("PW4_PREFILL_SPLITS");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v >= 1 && v <= 64) ? v : 0;
}
// K halves of the 128-row tiles (1 or 2), for tuning sweeps; 0 = heuristic.
int prefill_khalves_override() {
    const char* e = plan_env("PW4_PREFILL_KHALVES");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v == 1 || v == 2) ? v : 0;
}

// Decode kernel override for tuning sweeps: 0 keeps every M off the decode
// kernel (prefill kernels only), 1 keeps M <= 32 on it; unset = heuristic.
int decode_mode_override() {
    const char* e = plan_env("PW4_DECODE");
    if (!e) return -1;
    return e[0] == '0' ? 0 : e[0] == '1' ? 1 : -1;
}

// Decode K-split override for tuning sweeps (2, 4 or 8: exchange-tree
// slices even where the activations fit in LDS); 0 = heuristic.
int decode_splits_override() {
    const char* e = plan_env("PW4_DECODE_SPLITS");
    if (!e) return 0;
    const int v = std::atoi(e);
    return (v == 2 || v == 4 || v == 8) ? v : 0;
}
// Act-order gathered in the decode kernel's LDS: 0 never (the gather
// launch), else where it applies; for tests and sweeps.
int decode_perm_lds_override() {
    const char* e = plan_env("PW4_DECODE_PERM_LDS");
    return e && e[0] == '0' ? 0 : 1;
}
// Decode block scales forced on (1) or off (0) where they apply, for tests and
// sweeps; -1 = by layer size.
int decode_block_scales_override() {
    const char* e = plan_env("PW4_DECODE_BLOCK_SCALES");
    if (!e) return -1;
    return e[0] == '0' ? 0 : e[0] == '1' ? 1 : -1;
}

// Windowed decode plans (one unit per workgroup, the activations staged in K
// windows by copy waves) where the activation slice does not fit in LDS: by
// default only in place of the counter path (slices the exchange tree cannot
// take); PW4_DECODE_WIN=1 takes them wherever they apply, =0 never (A/B
// sweeps and tests only).
enum { kWinNever = 0, kWinAlways = 1, kWinForCounter = 2 };
int decode_win_mode() {
    const char* e = plan_env("PW4_DECODE_WIN");
    if (e && e[0] == '0') return kWinNever;
    if (e && e[0] == '1') return kWinAlways;
    return kWinForCounter;
}

// Plan of the 256-wide prefill kernel: tile rows (256 or 128) and K slices,
// from a cost model in microseconds fitted to a sweep of every (rows, slices)
// pair over the Llama-3-8B and -70B layer shapes at M = 72..4096 on one MI355X
// (bf16 activations; the fitted picks total 8628 us over 37 shapes against
// 8617 for the per-shape best and 9185 for the former fp16-fitted model):
//   * a 64-K chunk of a 256-row tile (8 waves, one workgroup per CU) takes
//     1.6 us; such tiles run in waves of the CU count, and an unsplit launch
//     balances its last wave with 128-row tiles;
//   * 128-row tiles (4 waves) run two workgroups per CU: a chunk takes 1.1 us
//     on a CU of its own, and a round of two per CU takes 1.6 us (a last
//     round of at most one per CU runs at the solo rate: measured, 70B qkv
//     8192 x 10240 at M = 2048 343 us on 2 K slices against 372 on the 3
//     the model picked without it, at M = 4096 579 unsplit against 666 on 2);
//   * K slices add their fp32 partials' round trip, s * M * N * 8 bytes at
//     6 TB/s, plus 1 us for the combine launch.  (At 8 TB/s the model took 2
//     slices for Llama-3-8B o at M = 1024 and 2048 and gate_up at M = 256,
//     measured 1-8% slower than its picks at 6 TB/s -- o M = 2048 unsplit 74-82
//     us against 80-84 on 2 slices; every other 8B and 70B pick at M = 256..4096
//     is the same at both rates and the measured fastest, within 1 us.)
// fp16 activations with exact scaling use 128-row tiles only: on the same
// sweep the model's 128-row picks are within 0.6% of the per-shape best (8367
// against 8322 us); 256-row tiles were ahead on down_proj of 70B alone, by 1-3%.
//   * 128-row tiles in K halves (k_halves = 2: one 8-wave workgroup per CU
//     runs both halves of its slice and sums them through LDS): a CU advances
//     two chunks per 1.8 us, whatever the number of tiles (the two halves
//     share one barrier per chunk, about 10% slower than two independent
//     4-wave workgroups, far faster than one alone); the LDS sum adds 0.5 us
//     per round.  Fitted to graph periods of every (k_halves, slices) plan on
//     the Llama-3-8B layers at M = 256..4096 and the 70B layers at M =
//     256..2048 (29 shapes): the picks total 7844 us against 7841 for the
//     per-shape best and 7892 without K halves.  They win where the tiles
//     leave CUs alone or would need fp32 partials: 8B qkv M = 1024 56.6 us
//     (69.0 unsplit or on 2 slices), o M = 2048 65.7 (73.2), gate_up M = 256
//     63.1 (69.8), o M = 1024 on 2 slices 46.9 (50.0).
struct Prefill256Plan {
    int rows;
    int64_t splits;
    int k_halves = 1;
};

// Exact scaling of the 256-wide prefill kernel with fp16 activations (see
// gemm_prefill_256.hip): on unless overridden with PW4_PREFILL_EXACT=0 (A/B
// sweeps only).
bool prefill_exact_enabled() {
    const char* e = plan_env("PW4_PREFILL_EXACT");
    return !(e && e[0] == '0');
}

// only128: 128-row tiles only (exact scaling); max_splits: the most K slices
// the plan may use; khalves: 0 the model's choice, 1 or 2 that many K halves
// for 128-row tiles.
Prefill256Plan plan_prefill256(int64_t M, int64_t N, int64_t nchunks, int cus, bool only128, int64_t max_splits,
                               double* cost_us = nullptr, int khalves = 0) {
    constexpr double kChunk256 = 1.6, kChunk128Solo = 1.1, kChunk128Pair = 1.6, kChunkHalves = 1.8,
                     kHalvesSum = 0.5, kPartialBps = 6.0e12, kCombineUs = 1.0;
    Prefill256Plan best{256, 1};
    double best_us = 0.0;
    bool have = false;
    const int64_t num_n = ceil_div(N, 256);
    for (int rows : {256, 128}) {
        if (only128 && rows != 128) continue;
        for (int kh : {1, 2}) {
            if (kh == 2 && rows != 128) continue;
            if (khalves != 0 && rows == 128 && kh != khalves) continue;
            for (int64_t s : {1, 2, 3, 4, 6, 8}) {
                if (s > nchunks || s > max_splits) break;
                const int64_t cps = ceil_div(nchunks, s);
                const int64_t sl = ceil_div(nchunks, cps);
                if (s > 1 && sl != s) continue;  // the same plan as a smaller s
                double us;
                if (rows == 256) {
                    double waves = (double)ceil_div(ceil_div(M, 256) * num_n * s, cus);
                    if (s == 1) prefill256_tail_cols(M, N, cus, &waves);
                    us = waves * (double)cps * kChunk256;
                } else if (kh == 2) {
                    const int64_t rounds = ceil_div(ceil_div(M, 128) * num_n * s, (int64_t)cus);
                    us = (double)rounds * ((double)ceil_div(cps, 2) * kChunkHalves + kHalvesSum);
                } else {
                    // rounds of two per CU, and a last round of at most one per CU
                    // at the solo rate
                    const int64_t wgs = ceil_div(M, 128) * num_n * s;
                    const int64_t pairs = wgs / (2 * (int64_t)cus), rest = wgs - pairs * 2 * (int64_t)cus;
                    us = (double)cps * ((double)pairs * kChunk128Pair +
                                        (rest == 0 ? 0.0 : rest <= cus ? kChunk128Solo : kChunk128Pair));
                }
                if (s > 1) us += (double)s * (double)M * (double)N * 8.0 / kPartialBps * 1e6 + kCombineUs;
                if (!have || us < best_us) {
                    best = {rows, s, kh};
                    best_us = us;
                    have = true;
                }
            }
        }
    }
    if (cost_us) *cost_us = best_us;
    return best;
}

// Decode kernel or 128-row prefill tile at M = 29..32 (MARLIN layout).  There
// the decode kernel runs two 16-row tiles per wave and K slices of the
// activations, and streams a large layer's weights at about 1.6 TB/s; the
// prefill tile's time follows the plan model above, which reads up to 1.25x
// low at these M.  Measured on MI355X (graph periods, us, decode / prefill
// tile, fp16 x): Llama-3-70B gate_up 8192 x 57344 M = 24 101 / 115, M = 28
// 123 / 116, M = 32 128 / 118; 70B down 28672 x 8192 M = 24 52 / 62, M = 28
// 55.5 / 61.6, M = 32 69.5 / 61.7 (K halves, 8 slices); every other 8B and 70B
// layer faster on the decode kernel at M = 17..32 (70B qkv M = 32 27.0 / 30.0,
// 8B gate_up 29.1 / 36.3, 8B down 25.0 / 32.0).  The prefill model is nearly
// flat over M = 28..32 while the decode kernel slows down, so the crossing is
// placed by M: from M = 29 on (at M = 28 that leaves 70B gate_up 7% slower on
// the decode kernel and 70B down 11% faster).
bool prefer_prefill_tile(int xt, int64_t M, int64_t N, int64_t K, int64_t G, int cus) {
    constexpr double kDecodeBps = 1.6e12, kModelLow = 1.25;
    if (M < 29 || !prefill256_ok(LAYOUT_MARLIN, xt, N, K, G)) return false;
    double prefill_us = 0.0;
    plan_prefill256(M, N, ceil_div(round_up(K, kMarlinBK), 64), cus, xt == X_F16 && prefill_exact_enabled(), 8,
                    &prefill_us);
    const double decode_us = (double)N * (double)K / 2.0 / kDecodeBps * 1e6;
    return kModelLow * prefill_us < decode_us;
}

struct Plan {
    bool decode = false;
    bool tree = false;       // decode K slices reduced through the exchange tree
    bool p256 = false;       // prefill on the 256 x 256 tile kernel
    bool p_exact = false;    // ... with exact scaling (fp16 x, 128-row tiles)
    DecodeConfig dc{};
    int p_splits = 1;        // prefill K splits
    int p_cps = 0;           // prefill chunks per split
    int p_tile_rows = 256;   // 256-wide kernel: rows per tile
    int p_k_halves = 1;      // 256-wide kernel, 128-row tiles: K halves per workgroup (1 or 2)
    bool use_partial = false;
    int splits = 1;
    size_t partial_bytes = 0;
    size_t xperm_bytes = 0;
    size_t silu_tmp_bytes = 0;  // SiLU-gated plans whose kernels cannot pair the columns themselves
    size_t repack_bytes = 0;    // CT weights repacked per call for the 256-wide kernel (words, then scales)
    // Every non-empty workspace starts with the fixed zero region, so the
    // bytes a decode call uses as counters or exchange slots are never
    // scratch for another call that shares the workspace.
    size_t workspace() const {
        const size_t rest =
            align_up(partial_bytes) + align_up(xperm_bytes) + align_up(silu_tmp_bytes) + align_up(repack_bytes);
        return (rest || tree) ? kZeroRegion + rest : 0;
    }
};

// layout: LAYOUT_MARLIN or LAYOUT_CT.  num_splits: 0 auto, >= 1 forced.
// ws_cap: 0, or the most workspace bytes the caller has (the no-alloc entry
// point's scratch): an automatic prefill plan whose K-slice partials would
// not fit it runs unsplit instead.
Plan make_plan(int layout, int x_dtype, int stype, bool zp, int64_t M, int64_t N, int64_t K, int64_t G, bool has_perm,
               int64_t num_splits, bool silu = false, size_t ws_cap = 0) {
    Plan p;
    const int cus = cu_count();
    const int64_t kext = layout == LAYOUT_MARLIN ? round_up(K, kMarlinBK) : round_up(K, 32);
    const int64_t ktiles = kext / 32;
    const bool forced = num_splits >= 1;
    const bool zp_any = true;  // size the LDS for the asymmetric variant (a few hundred bytes more)
    // The decode kernel takes power-of-two group sizes: 128 K steps hold 128 / G
    // whole groups (G = 16..64, one masked MFMA per group) or lie inside one
    // (G >= 128).
    const int64_t ngrp = G >= 128 ? 1 : 128 / std::max<int64_t>(G, 1);
    // Up to M = 32: from M = 33 the 128-row prefill tile is faster at every
    // Llama-3 8B and 70B layer (measured on MI355X, kernel only, us, decode at
    // M = 33 and 64 / prefill at M = 65: 8B gate_up 58 and 136 / 35, down 36
    // and 145 / 36, 70B gate_up 218 and 852 / 114, down 210 and 1031 / 74).
    bool decode_ok = M <= 32 && G >= 16 && (G & (G - 1)) == 0;
    const int decode_mode = decode_mode_override();
    if (decode_mode == 0) decode_ok = false;
    if (decode_ok && decode_mode != 1 && !forced && layout == LAYOUT_MARLIN &&
        prefer_prefill_tile(x_dtype == PW4_DTYPE_BF16 ? X_BF16 : X_F16, M, N, K, G, cus)) {
        decode_ok = false;
    }
    if (decode_ok) {
        DecodeConfig dc{};
        dc.mt = M <= 16 ? 1 : 2;
        dc.ngrp = (int)ngrp;
        const bool bf = x_dtype == PW4_DTYPE_BF16;
        // Columns the units cover (MARLIN pads N to 64; CT columns past N are
        // clamped loads whose results are dropped).
        const int64_t ncols = layout == LAYOUT_MARLIN ? round_up(N, kMarlinBN) : round_up(N, 16);
        const int64_t steps = std::max<int64_t>(ceil_div(ktiles * 32, 128), 1);
        auto kps_for = [&](int64_t sp) { return std::max<int64_t>(round_up(ceil_div(ktiles * 32, sp), 128), 128); };
        bool red_single = false;
        auto lds_for = [&](int64_t sp) {
            return decode_lds_bytes((int)M, (int)kps_for(sp), dc.ngrp, zp_any, bf, red_single);
        };
        // K slices only when the activation slice does not fit in LDS: each
        // slice costs a partial round trip per unit.  A single reduction
        // buffer is used when it saves slices.
        int64_t s = 1;
        if (forced) {
            // slices past the last 128-K step would be empty (they add zero):
            // at most one per step
            s = std::min<int64_t>(num_splits, steps);
        } else {
            while (s < steps && lds_for(s) > kDecodeLdsLimit) ++s;
            if (s > 1) {
                red_single = true;
                int64_t s1 = 1;
                while (s1 < steps && lds_for(s1) > kDecodeLdsLimit) ++s1;
                if (s1 < s) {
                    s = s1;
                } else {
                    red_single = false;
                }
            }
        }
        // Exchange-tree slices (no partial round trip, no ring drain): a power
        // of two up to 8, M <= 32 (tree kernels exist for 16- and 32-row
        // tiles), at most two output elements per thread.  Units as wide as
        // that allows while every CU still gets three unit slices to balance
        // over at 64 columns, two at 32: a wider unit gives each K wave more
        // steps between unit ends (measured: gate_up at M = 32 30 us with
        // 32-column units against 37 with 16, down at M = 16 13.8 against 15.1).
        // Where the slice's LDS leaves room for one workgroup per CU, 32
        // columns also win at one slice per CU when the busiest CU gets no more
        // columns than at 16 (down at M = 8 11.6 us against 12.5, o at M = 24
        // 8.7 against 9.2); qkv at M = 24-32 (1.5 slices per CU at 32) stays at
        // 16, and so do slices small enough for two workgroups per CU (down at
        // M = 5: 11.1 us at 16 against 14.3).
        // Windowed plan instead of K slices: one slice, units of the narrowest
        // width that gives every workgroup one unit on at least half the CUs
        // (so the activations are read once per workgroup), the largest K
        // window whose two buffers fit in LDS with a power-of-two number of
        // steps per K wave and at least two windows.  Every workgroup reads
        // the whole M x K activations from L2, against 1/slices of them with
        // K slices: measured on MI355X (kernel only, us, windowed / sliced),
        // Llama-3-8B down M = 6-16 12.6-17.2 / 10.0-13.0, M = 24-32 22.4-26.0
        // / 21.3-23.2, 70B qkv and o M = 9-16 13.3-18.6 / 12.1-16.0, all with
        // the exchange tree; 70B down M = 32 68.7 / 148.8, where the slices
        // exceed the tree's eight and take the counter path.
        const int win_mode = decode_win_mode();
        int64_t kwin = 0;
        int win_nb = 16;
        bool win_red_single = false;
        if (!forced && s > 1 && layout == LAYOUT_MARLIN && dc.ngrp <= 2 && M <= 32 && K == kext && K % 128 == 0 &&
            decode_splits_override() == 0 && win_mode != kWinNever) {
            const int nb_forced = decode_nb_override();
            for (int w : {16, 32, 64}) {
                if (ncols % w != 0 || (nb_forced && w != nb_forced)) continue;
                const int64_t ncg_w = ncols / w;
                if (ncg_w > cus || 2 * ncg_w <= cus) continue;
                const int64_t wstep = 128 * (8 / (w / 16));  // K of one step of every K wave
                for (bool rs1 : {false, true}) {
                    for (int64_t jw = 64; jw >= 1 && kwin == 0; jw /= 2) {
                        const int64_t kw = jw * wstep;
                        if (kw >= kext || kext % kw != 0) continue;
                        if (decode_lds_bytes((int)M, (int)kw, dc.ngrp, zp_any, bf, rs1, true) > kDecodeLdsLimit) continue;
                        kwin = kw;
                        win_red_single = rs1;
                    }
                    if (kwin) break;
                }
                if (kwin) {
                    win_nb = w;
                    break;
                }
            }
        }
        bool tree = false;
        int tree_nb = 16;
        if (!forced && !(kwin > 0 && win_mode == kWinAlways) && dc.ngrp <= 2) {  // no tree for groups under 64
            int64_t s2 = std::max<int64_t>(s, decode_splits_override());
            if (s2 > 1) {
                int64_t p2 = 2;
                while (p2 < s2) p2 *= 2;
                const int nb_forced = decode_nb_override();
                const bool one_wg_per_cu = 2 * lds_for(p2) > kLdsPerCu;
                const int64_t busiest16 = ceil_div(ceil_div(ncols, 16) * p2, (int64_t)cus) * 16;
                // 64-column units also where their slices split evenly over the
                // CUs and each of a unit's two K waves streams 24 steps or more:
                // 70B down (K = 28672) at M = 4 / 8, 32 / 64 columns, kernel only,
                // 24.4 / 22.6 and 27.9 / 24.7 us.  With shorter units 32 columns
                // stay faster (70B o at M = 16, 16 steps per wave at 64: 12.4 us
                // at 32).
                const bool long_units64 = ceil_div(ceil_div(kps_for(p2), 128), 2) >= 24;
                for (int w : {64, 32, 16}) {
                    const bool fits = M * w <= 1024 && ncols % w == 0;
                    const int64_t q = ceil_div(ncols, w) * p2;  // unit slices
                    const bool wide = q >= (w == 64 ? 3 : 2) * cus ||
                                      (w == 64 && q % cus == 0 && long_units64) ||
                                      (w == 32 && one_wg_per_cu && ceil_div(q, (int64_t)cus) * 32 <= busiest16);
                    if (nb_forced ? (w == nb_forced && fits) || w == 16 : (fits && wide) || w == 16) {
                        tree_nb = w;
                        break;
                    }
                }
                const int64_t ncgw = ceil_div(ncols, tree_nb);
                if (p2 <= 8 && p2 <= steps && M <= 32 && M * tree_nb <= 1024 &&
                    (size_t)(p2 - 1) * ncgw * M * tree_nb * sizeof(uint64_t) <= kSlotBytes) {
                    s = p2;
                    tree = true;
                }
            }
        }
        const bool win = kwin > 0 && !tree;
        if (win) {
            s = 1;
            red_single = win_red_single;
        }
        const int64_t kps = kps_for(s);
        if (!forced && !tree) s = std::max<int64_t>(ceil_div(ktiles * 32, kps), 1);
        const size_t lds = win ? decode_lds_bytes((int)M, (int)kwin, dc.ngrp, zp_any, bf, red_single, true) : lds_for(s);
        // Units: 16 columns (eight K waves per strip, the finest balance), or
        // 64 when K is sliced, to keep the per-unit partial round trips few.
        int nb = win ? win_nb : tree ? tree_nb : decode_nb_override();
        if (nb == 0) nb = s > 1 ? 64 : 16;
        while (nb > 16 && ncols % nb != 0) nb /= 2;
        int64_t ncg = ceil_div(ncols, nb);
        // ring depth: a unit of at most 4 steps per wave needs no more (its
        // steps pad to the ring depth).  Up to M = 8 the 4-step ring also
        // wins on long units: 8 waves x 4 x 1 KB is 32 KB of weight loads in
        // flight per CU, where a streaming read peaks; 64 KB per CU queues
        // behind itself (a copy of the kernel's load walk, no compute: down
        // 6.5 us with 4 steps in flight against 7.2 with 8; the kernel: down
        // M = 1 -8%, Llama-70B layers at M = 1 -3..-8%).  At M = 16 the
        // deeper ring still covers the 16-row MFMA work (70B layers +2% at 4).
        const int64_t kwn = 8 / (nb / 16);
        const int64_t spu = std::max<int64_t>(ceil_div(ceil_div(kps, 128), kwn), 1);
        dc.ring = spu <= 4 || dc.ngrp > 2 || M <= 8 ? 4 : 8;
        // Block scales (one scale load per four steps, handed between lane
        // groups) on layers of 24 MiB of weights or more.  Measured on MI355X,
        // kernel only, medians of six interleaved runs over the 8B decode sweep
        // (fp16 x, G = 128): gate_up 3.0-3.2% and down 0.8-2.6% faster at M = 1..16;
        // o 3.8-6.1% and qkv 0-3.6% slower.  The small layers run at their
        // read floor, where the exchange on a wave's first block (its only one
        // on o) costs more than the three scale loads it saves.
        const int bs_mode = decode_block_scales_override();
        dc.block_scales = layout == LAYOUT_MARLIN && dc.ngrp == 1 && !win &&
                          (bs_mode < 0 ? N * K / 2 >= (int64_t{24} << 20) : bs_mode == 1);
        // Act-order gathered in LDS by the decode kernel (x as given staged
        // whole beside the slice), in place of a separate gather launch: one
        // slice over all of K, 16-row tiles, the 4-step ring, one quant group
        // per step, and both copies of x in LDS.
        size_t lds_run = lds;
        if (has_perm && decode_perm_lds_override() != 0 && layout == LAYOUT_MARLIN && !forced && s == 1 && !tree &&
            !win && dc.mt == 1 && dc.ring == 4 && dc.ngrp == 1 && K % 8 == 0 && decode_perm_cols(K) > 0) {
            const size_t lpx = decode_lds_bytes((int)M, (int)kps, dc.ngrp, zp_any, bf, red_single, false, (int)K);
            if (lpx <= kDecodeLdsLimit) {
                dc.perm_cols = decode_perm_cols(K);
                lds_run = lpx;
            }
        }
        // Persistent grid: one or two workgroups per CU (register and LDS
        // budget), then as few units per workgroup as possible with the
        // least per-CU load.
        int64_t per_cu_max =
            lds_run <= kDecodeLdsLimit
                ? decode_blocks_per_cu(layout, bf ? X_BF16 : X_F16, stype, zp, dc.mt, dc.ngrp, dc.ring, tree, lds_run,
                                       win, dc.block_scales, dc.perm_cols)
                : 0;
        if (per_cu_max <= 0) {
            per_cu_max = std::max<int64_t>(std::min<int64_t>(2, (int64_t)(kLdsPerCu / std::max<size_t>(lds_run, 1))), 1);
        }
        per_cu_max = std::min<int64_t>(per_cu_max, 2);
        // workgroups per slice for ncg units, and the busiest CU's units
        auto pick_wps = [&](int64_t units, int64_t* cost_out) {
            int64_t wps_best = 1, cost_best = INT64_MAX;
            for (int64_t per_cu = 1; per_cu <= per_cu_max; ++per_cu) {
                const int64_t wps_max = std::max<int64_t>((int64_t)cus * per_cu / s, 1);
                const int64_t ups = ceil_div(units, std::min(wps_max, units));
                const int64_t wps = ceil_div(units, ups);
                const int64_t cost = ups * ceil_div(wps * s, (int64_t)cus);
                if (cost < cost_best || (cost == cost_best && wps > wps_best)) {
                    cost_best = cost;
                    wps_best = wps;
                }
            }
            if (cost_out) *cost_out = cost_best;
            return wps_best;
        };
        int64_t best_cost = 0;
        int64_t best_wps = pick_wps(ncg, &best_cost);
        // One slice over a long K (8192 and up): 32-column units where the
        // busiest CU gets no more columns than with 16.  Each K wave then
        // streams twice the steps between unit ends, one workgroup per CU
        // where 16 columns would take two.  Measured on MI355X (kernel only,
        // us, 16 / 32 columns): Llama-3-70B o 8192 x 8192 M = 1 9.56 / 8.28,
        // M = 4 9.28 / 8.84, M = 8 10.32 / 9.72; gate_up 8192 x 57344 M = 1
        // 45.6 / 40.3, M = 4 43.7 / 40.9, M = 8 46.2 / 41.5.  70B qkv (48
        // columns on the busiest CU at 16, 64 at 32) and every Llama-3-8B
        // layer (K = 4096, or more columns per CU at 32) keep 16.
        // (The ring depth does not change: at K >= 8192 a wave has at least 8
        // steps per unit either way.)
        if (!forced && !win && !tree && s == 1 && nb == 16 && decode_nb_override() == 0 && K >= 8192 &&
            ncols % 32 == 0) {
            int64_t cost32 = 0;
            const int64_t wps32 = pick_wps(ceil_div(ncols, 32), &cost32);
            if (cost32 * 32 <= best_cost * 16) {
                nb = 32;
                ncg = ceil_div(ncols, nb);
                best_wps = wps32;
                best_cost = cost32;
            }
        }
        // One slice over a short K (below 8192) at M <= 8: 16-column units give
        // each K wave only K / 1024 steps per unit (4 at K = 4096).  The widest
        // of 64 and 32 columns with at most 16 steps per K wave, whose
        // workgroups cover at least 3/4 of the CUs and whose busiest CU gets at
        // most 1.15x the columns it would at 16.  Measured on MI355X (kernel
        // only, us, 16 columns / wider): Llama-3-8B qkv 4096 x 6144 at 32
        // columns M = 1 5.64 / 5.28, M = 4 6.40 / 5.66, M = 8 6.52 / 6.28;
        // gate_up 4096 x 28672 at 64 columns M = 1 13.28 / 12.36, M = 4 13.60 /
        // 12.76, M = 8 14.28 / 14.12.  o (32 columns would leave half the CUs
        // idle) and down (K = 14336) keep 16; at M = 12 the wider units were
        // no faster.
        if (!forced && !win && !tree && s == 1 && nb == 16 && decode_nb_override() == 0 && K < 8192 && M <= 8) {
            for (int w : {64, 32}) {
                if (ncols % w != 0 || ceil_div(kps, 128) * w > 16 * 128) continue;
                int64_t cost_w = 0;
                const int64_t wps_w = pick_wps(ceil_div(ncols, w), &cost_w);
                if (4 * wps_w < 3 * (int64_t)cus || 20 * cost_w * w > 23 * best_cost * 16) continue;
                nb = w;
                ncg = ceil_div(ncols, nb);
                best_wps = wps_w;
                best_cost = cost_w;
                break;
            }
        }
        if (const char* e = plan_env("PW4_DECODE_WPS")) {  // tuning sweeps only
            const int64_t v = std::atoll(e);
            if (v >= 1 && v <= 4 * (int64_t)cus) best_wps = std::min<int64_t>(v, ncg);
        }
        if (win) best_wps = ncg;  // one unit per workgroup
        dc.nb = nb;
        dc.wps = (int)best_wps;
        dc.k_per_split = (int)kps;
        dc.splits = (int)s;
        dc.lds_bytes = lds_run;
        dc.red_single = red_single;
        dc.tree = tree;
        dc.kwin = win ? (int)kwin : 0;
        const bool partial = !tree && (forced || s > 1);
        if (lds <= kDecodeLdsLimit && !(partial && ncg > kMaxCounterCols) && best_wps * s <= INT32_MAX &&
            s <= 65535) {
            p.decode = true;
            p.tree = tree;
            p.dc = dc;
            p.splits = (int)s;
            p.use_partial = partial;
            if (partial) p.partial_bytes = (size_t)ncg * s * M * nb * sizeof(float);
        }
    }
    if (!p.decode) {
        const int64_t nchunks = ceil_div(kext, 64);
        // The 256-wide kernel (MARLIN, fp16) needs whole 64-K chunks inside one
        // quant group; with its 128-row tiles and K slices it is measured 20-45%
        // faster than the 128 x 128 kernel at M = 72..160 on every Llama-3-8B
        // layer shape, so it takes every M past the decode kernel's.
        const int xt = x_dtype == PW4_DTYPE_BF16 ? X_BF16 : X_F16;
        const int tile_pref = prefill_tile_override();
        p.p256 = prefill256_ok(LAYOUT_MARLIN, xt, N, K, G) && tile_pref != 128;
        p.p_exact = p.p256 && xt == X_F16 && prefill_exact_enabled();
        // The CT layout (gemm_w4a16) reaches the 256-wide kernel through a
        // per-call repack into the workspace: one pass over the weights
        // (~5 us for 4096 x 4096) against the 128 x 128 kernel's ~2x slower
        // GEMM at every M past the decode range.  At M = 33..64 it also beats
        // decode calls over 32-row blocks on every Llama-3 8B and 70B layer
        // but 8B o (graph periods, us, M = 33 and 64, this plan / 128 x 128
        // on CT / decode blocks: 8B gate_up 64.4 and 66.2 / 109 and 109 /
        // 70.2 and 83.4, 70B down 113 and 114 / 271 and 275 / 216 and 346;
        // 8B o 27.1 and 27.4 / 30.7 and 33.5 / 22.8 and 26.3).
        if (p.p256 && layout == LAYOUT_CT) {
            p.repack_bytes = align_up((size_t)round_up(N, kMarlinBN) * round_up(K, kMarlinBK) / 2) +
                             (size_t)(K / G) * N * sizeof(float);
        }
        const int64_t tm = p.p256 ? prefill256_tile() : prefill_tile_m();
        const int64_t tn = p.p256 ? prefill256_tile() : prefill_tile_n();
        const int64_t base = ceil_div(M, tm) * ceil_div(N, tn);
        // K slices fill the chip when the tiles do not, but each costs an fp32
        // partial round trip of the output: keep at least 16 chunks per slice.
        // does a plan of sl slices fit ws_cap (when there is one)?
        auto fits = [&](int64_t sl) {
            if (ws_cap == 0 || sl <= 1) return true;
            const size_t need = kZeroRegion + align_up((size_t)sl * M * N * 4) +
                                align_up(has_perm ? (size_t)M * K * 2 : 0) + align_up(p.repack_bytes);
            return need <= ws_cap;
        };
        int64_t s;
        if (forced) {
            s = std::min<int64_t>(num_splits, std::max<int64_t>(nchunks, 1));  // more would be empty slices
        } else if (p.p256 && prefill_splits_override()) {
            s = std::min<int64_t>(prefill_splits_override(), std::max<int64_t>(nchunks, 1));
        } else if (p.p256) {
            const int kh = prefill_khalves_override();
            Prefill256Plan pp = plan_prefill256(M, N, nchunks, cus, p.p_exact, 8, nullptr, kh);
            if (!fits(pp.splits)) pp = plan_prefill256(M, N, nchunks, cus, p.p_exact, 1, nullptr, kh);
            s = pp.splits;
            p.p_tile_rows = pp.rows;
            p.p_k_halves = pp.k_halves;
        } else if (base >= cus || nchunks < 8) {
            s = 1;
        } else {
            s = std::min<int64_t>(ceil_div(cus, std::max<int64_t>(base, 1)), p.p256 ? nchunks / 16 : nchunks / 4);
            s = std::max<int64_t>(s, 1);
            if (!fits(s)) s = 1;
        }
        int64_t cps = std::max<int64_t>(ceil_div(std::max<int64_t>(nchunks, 1), s), 1);
        if (!forced) s = std::max<int64_t>(ceil_div(nchunks, cps), 1);
        p.p_splits = (int)s;
        p.p_cps = (int)cps;
        p.splits = (int)s;
        p.use_partial = forced || s > 1;
        if (p.use_partial) p.partial_bytes = (size_t)p.splits * M * N * 4;
        if (p.p256 && prefill_rows_override()) p.p_tile_rows = prefill_rows_override();
        if (p.p_exact && !prefill_rows_override()) p.p_tile_rows = 128;
        // forced and overridden slice counts take one K half unless overridden too
        if (p.p256 && (forced || prefill_splits_override())) p.p_k_halves = std::max(prefill_khalves_override(), 1);
        if (p.p_tile_rows != 128) p.p_k_halves = 1;
    }
    // act-order: x is gathered once per call into the workspace, for either
    // kernel (each decode workgroup would otherwise gather the same slice),
    // unless the decode kernel gathers it in LDS; the buffer is kept in the
    // workspace either way, for a permutation that is not 16-byte aligned
    if (has_perm) p.xperm_bytes = (size_t)M * K * 2;
    // SiLU gating is fused into the decode kernel's direct store, the 256-wide
    // prefill kernel's unsplit epilogue and the split-K combine; the other
    // plans (decode K slices, the unsplit 128 x 128 kernel) write the GEMM
    // output to the workspace and gate it in a second pass
    if (silu && ((p.decode && (p.tree || p.use_partial)) || (!p.decode && !p.p256 && !p.use_partial))) {
        p.silu_tmp_bytes = (size_t)M * N * 2;
    }
    return p;
}

int check_common(int64_t M, int64_t N, int64_t K, int64_t G, int x_dtype) {
    if (M < 0 || N < 0 || K < 0) return PW4_ERR_ARG;
    if (x_dtype != PW4_DTYPE_F16 && x_dtype != PW4_DTYPE_BF16) return PW4_ERR_ARG;
    if (G <= 0 || G % 16 != 0) return PW4_ERR_SHAPE;
    if (K % 8 != 0 || K % G != 0) return PW4_ERR_SHAPE;
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return PW4_ERR_SHAPE;
    return PW4_OK;
}

// ev: the call's armed timing events, taken by the entry point (they time the
// GEMM kernel launches only, not the repack, gather, combine or SiLU passes).
int run_gemm(int layout, const void* x, int x_dtype, const uint32_t* w, const void* scales, int stype,
             const uint32_t* qzeros, const int32_t* perm, void* y, int64_t M, int64_t N, int64_t K, int64_t G,
             int64_t num_splits, void* workspace, size_t ws_bytes, hipStream_t stream, KernelEvents ev,
             bool silu = false, size_t ws_cap = 0) {
    // x and the weight words are read as 16-byte vectors
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) return PW4_ERR_ARG;
    const Plan p = make_plan(layout, x_dtype, stype, qzeros != nullptr, M, N, K, G, perm != nullptr, num_splits, silu,
                             ws_cap);
    if (p.workspace() > 0 && (workspace == nullptr || ws_bytes < p.workspace())) return PW4_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    int32_t* counters = p.workspace() ? reinterpret_cast<int32_t*>(ws) : nullptr;
    unsigned long long* slots = p.tree ? reinterpret_cast<unsigned long long*>(ws + kCounterBytes) : nullptr;
    float* partial = p.partial_bytes ? reinterpret_cast<float*>(ws + kZeroRegion) : nullptr;
    uint16_t* xperm =
        p.xperm_bytes ? reinterpret_cast<uint16_t*>(ws + kZeroRegion + align_up(p.partial_bytes)) : nullptr;
    uint16_t* silu_tmp = p.silu_tmp_bytes ? reinterpret_cast<uint16_t*>(ws + kZeroRegion + align_up(p.partial_bytes) +
                                                                        align_up(p.xperm_bytes))
                                          : nullptr;
    // the GEMM's own output: y, or the workspace copy a second pass gates into y
    uint16_t* y_gemm = silu_tmp ? silu_tmp : reinterpret_cast<uint16_t*>(y);
    const int xt = x_dtype == PW4_DTYPE_BF16 ? X_BF16 : X_F16;
    hipError_t e;
    if (p.repack_bytes) {
        // CT weights -> MARLIN words and fp32 [K/G, N] scales in the workspace,
        // then the MARLIN path
        char* rp = ws + kZeroRegion + align_up(p.partial_bytes) + align_up(p.xperm_bytes) + align_up(p.silu_tmp_bytes);
        uint32_t* words = reinterpret_cast<uint32_t*>(rp);
        float* sm = reinterpret_cast<float*>(rp + align_up((size_t)round_up(N, kMarlinBN) * round_up(K, kMarlinBK) / 2));
        e = launch_repack_ct(w, scales, S_F32, words, sm, (int)N, (int)K, (int)G, stream);
        if (e != hipSuccess) return hip_fail(e);
        layout = LAYOUT_MARLIN;
        w = words;
        scales = sm;
        stype = S_F32;
    }
    const int64_t kext = layout == LAYOUT_MARLIN ? round_up(K, kMarlinBK) : round_up(K, 32);
    const uint16_t* xin = reinterpret_cast<const uint16_t*>(x);
    // act-order in the decode kernel's LDS reads the permutation as 16-byte
    // vectors; another alignment takes the gather launch and the plain plan
    DecodeConfig dc = p.dc;
    if (p.decode && dc.perm_cols && (reinterpret_cast<uintptr_t>(perm) & 15) != 0) {
        dc.perm_cols = 0;
        dc.lds_bytes = decode_lds_bytes((int)M, dc.k_per_split, dc.ngrp, true, xt == X_BF16, dc.red_single);
    }
    const bool perm_in_lds = p.decode && dc.perm_cols > 0;
    if (perm && !perm_in_lds) {
        e = launch_gather_x(xin, perm, xperm, (int)M, (int)K, stream, gather_staged_override());
        if (e != hipSuccess) return hip_fail(e);
        xin = xperm;
    }
    if (p.decode) {
        DecodeArgs a{};
        a.x = xin;
        a.perm = perm_in_lds ? perm : nullptr;
        a.w = w;
        a.scales = scales;
        a.qzeros = qzeros;
        a.y = y_gemm;
        a.partial = p.use_partial ? partial : nullptr;
        a.counters = counters;
        a.silu = silu && !silu_tmp ? 1 : 0;
        a.y32 = silu ? nullptr : ev.y32;
        a.slots = slots;
        a.tree_levels = p.tree ? __builtin_ctz((unsigned)p.dc.splits) : 0;
        a.red_single = p.dc.red_single ? 1 : 0;
        a.nb = p.dc.nb;
        a.wps = p.dc.wps;
        a.M = (int)M;
        a.N = (int)N;
        a.K = (int)K;
        a.G = (int)G;
        a.Kg = (int)(K / G);
        a.G_log2 = __builtin_ctzll((unsigned long long)G);
        a.ktiles = (int)(kext / 32);
        a.nchunks = (int)(round_up(K, kMarlinBK) / kMarlinBK);
        a.k_per_split = p.dc.k_per_split;
        a.kwin = p.dc.kwin > 0 ? p.dc.kwin : p.dc.k_per_split;
        a.rowstride = a.kwin + 8;
        a.jw_log2 = p.dc.kwin > 0 ? __builtin_ctz((unsigned)(p.dc.kwin / 128 / (8 / (p.dc.nb / 16)))) : 0;
        a.splits = p.dc.splits;
        const int64_t ncols = layout == LAYOUT_MARLIN ? round_up(N, kMarlinBN) : round_up(N, 16);
        a.ncg = (int)ceil_div(ncols, p.dc.nb);
        a.ups = (int)ceil_div(a.ncg, p.dc.wps);
        a.spr_recip = (uint32_t)(((uint64_t{1} << 32) + (uint64_t)(a.kwin / 8 + 1) - 1) / (uint64_t)(a.kwin / 8 + 1));
        e = launch_decode(layout, xt, stype, qzeros != nullptr, dc, a, stream, ev);
        if (e != hipSuccess) return hip_fail(e);
    } else {
        PrefillArgs a{};
        a.x = xin;
        a.w = w;
        a.scales = scales;
        a.qzeros = qzeros;
        a.y = y_gemm;
        a.partial = p.use_partial ? partial : nullptr;
        a.silu = silu && p.p256 && !p.use_partial ? 1 : 0;
        a.M = (int)M;
        a.N = (int)N;
        a.K = (int)K;
        a.G = (int)G;
        a.Kg = (int)(K / G);
        a.ktiles = (int)(kext / 32);
        a.nchunks = (int)ceil_div(kext, 64);
        a.chunks_per_split = p.p_cps;
        a.splits = p.p_splits;
        a.n_begin = 0;
        a.n_end = (int)N;
        a.cus = cu_count();
        a.tile_rows = p.p_tile_rows;
        a.k_halves = p.p_k_halves;
        a.exact = p.p_exact ? 1 : 0;
        a.y32 = silu || p.use_partial ? nullptr : ev.y32;
        e = p.p256 ? launch_prefill256(xt, stype, qzeros != nullptr, a, stream, ev)
                   : launch_prefill(layout, xt, stype, qzeros != nullptr, a, stream, ev);
        if (e != hipSuccess) return hip_fail(e);
    }
    if (p.use_partial && !p.decode) {
        e = silu ? launch_combine_silu(partial, reinterpret_cast<uint16_t*>(y), M, N, p.splits, xt, stream)
                 : launch_combine(partial, reinterpret_cast<uint16_t*>(y), M * N, p.splits, xt, stream, ev.y32);
        if (e != hipSuccess) return hip_fail(e);
    }
    if (silu_tmp) {
        e = launch_silu_mul(silu_tmp, reinterpret_cast<uint16_t*>(y), M, N, xt, stream);
        if (e != hipSuccess) return hip_fail(e);
    }
    return PW4_OK;
}

// ---- the no-alloc entry point's scratch -------------------------------------
// One array per device (each GPU the library runs on holds its own copy until
// the process exits).  Host code never names it directly: in host code the
// symbol is a stand-in, not a device address, so its address on each device
// comes from hipGetSymbolAddress once, with that device current.  Its first
// PW4_ZERO_REGION_BYTES are the zero region of a workspace; the rest is
// scratch (partials, the act-order copy of x, SiLU staging).
constexpr size_t kStaticScratchBytes = PW4_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

__global__ __launch_bounds__(256) void zero_fill_kernel(u32x4* __restrict__ p, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) p[i] = u32x4{0u, 0u, 0u, 0u};
}

struct DeviceScratch {
    void* ptr = nullptr;    // this device's copy of `scratch`
    bool cleared = false;   // its zero region was cleared by a fill that ran (not one only recorded into a graph)
    bool fill_captured = false;         // a fill was recorded into the capture `fill_capture_id`
    unsigned long long fill_capture_id = 0;
};
std::mutex g_scratch_mu;
DeviceScratch g_scratch[kMaxDevices];

// The scratch of the device `stream` runs on, set up on the first call on that
// device: its address, then a fill of the zero region on the caller's stream
// (a fill kernel, not a memset, so that a capturing caller's graph can hold
// it).  The GEMM kernels leave the region zero when they end, so one fill that
// has run is enough for every later call.  A fill only recorded into a graph
// has not run: it is recorded once per capture (the graph's first no-alloc
// call; replays run it ahead of that call's kernels, and the calls after it in
// the graph find the region as the earlier ones left it), and the next call
// from a stream that is not capturing fills eagerly.
int device_scratch(hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    if (dev < 0 || dev >= kMaxDevices) return PW4_ERR_ARG;
    // the array is per device: a stream of another device would have its
    // kernels use memory of the current one (the null stream is the current
    // device's)
    if (stream != nullptr) {
        hipDevice_t sdev = 0;
        e = hipStreamGetDevice(stream, &sdev);
        if (e != hipSuccess) return hip_fail(e);
        if ((int)sdev != dev) return PW4_ERR_ARG;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    DeviceScratch& d = g_scratch[dev];
    if (d.ptr == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e);
        d.ptr = ptr;
    }
    if (!d.cleared) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        unsigned long long cid = 0;
        e = hipStreamGetCaptureInfo(stream, &cs, &cid);
        if (e != hipSuccess) return hip_fail(e);
        const bool capturing = cs == hipStreamCaptureStatusActive;
        if (!(capturing && d.fill_captured && d.fill_capture_id == cid)) {
            const int64_t n16 = (int64_t)(kZeroRegion / 16);
            hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)ceil_div(n16, 256)), dim3(256), 0, stream,
                               reinterpret_cast<u32x4*>(d.ptr), n16);
            e = hipGetLastError();
            if (e != hipSuccess) return hip_fail(e);
            if (capturing) {
                d.fill_captured = true;
                d.fill_capture_id = cid;
            } else {
                d.cleared = true;
            }
        }
    }
    *out = d.ptr;
    return PW4_OK;
}

}  // namespace

extern "C" {

const char* pw4_status_string(int status) {
    switch (status) {
        case PW4_OK: return "ok";
        case PW4_ERR_ARG: return "invalid argument (null pointer, dtype or negative size)";
        case PW4_ERR_SHAPE: return "inconsistent shape or group size";
        case PW4_ERR_WORKSPACE: return "workspace missing or too small";
        case PW4_ERR_HIP: return "HIP runtime error";
        case PW4_ERR_GIDX: return "g_idx is not a grouping of exactly group_size rows per group";
        default: return "unknown status";
    }
}

const char* pw4_last_hip_error(void) { return g_last_hip_error; }

int pw4_time_next_kernel(void* start_event, void* stop_event) {
    if ((start_event == nullptr) != (stop_event == nullptr)) return PW4_ERR_ARG;
    pw4::g_armed_events.start = static_cast<hipEvent_t>(start_event);
    pw4::g_armed_events.stop = static_cast<hipEvent_t>(stop_event);
    return PW4_OK;
}

int pw4_observe_next_call(float* y32) {
    pw4::g_armed_events.y32 = y32;
    return PW4_OK;
}

int pw4_plan_describe(int layout, int x_dtype, int scale_dtype, int has_zp, int has_perm, int silu, int64_t M,
                      int64_t N, int64_t K, int64_t group_size, int64_t num_splits, char* buf, size_t len) {
    if (layout != PW4_LAYOUT_CT && layout != PW4_LAYOUT_MARLIN) return PW4_ERR_ARG;
    int rc = check_common(M, N, K, group_size, x_dtype);
    if (rc != PW4_OK) return rc;
    if (num_splits < 0 || buf == nullptr || len == 0) return PW4_ERR_ARG;
    if (scale_dtype != PW4_DTYPE_F32 && scale_dtype != PW4_DTYPE_F16) return PW4_ERR_ARG;
    if (M == 0 || N == 0) return PW4_ERR_SHAPE;
    const int lay = layout == PW4_LAYOUT_MARLIN ? LAYOUT_MARLIN : LAYOUT_CT;
    const Plan p = make_plan(lay, x_dtype, scale_dtype == PW4_DTYPE_F32 ? S_F32 : S_F16, has_zp != 0, M, N, K,
                             group_size, has_perm != 0, num_splits, silu != 0);
    int n;
    if (p.decode) {
        n = std::snprintf(buf, len, "decode nb=%d wps=%d splits=%d tree=%d win=%d ring=%d mt=%d bs=%d px=%d", p.dc.nb,
                          p.dc.wps, p.dc.splits, p.tree ? 1 : 0, p.dc.kwin > 0 ? 1 : 0, p.dc.ring, p.dc.mt,
                          p.dc.block_scales ? 1 : 0, p.dc.perm_cols);
    } else if (p.p256) {
        n = std::snprintf(buf, len, "prefill256 rows=%d splits=%d exact=%d khalves=%d%s", p.p_tile_rows, p.p_splits,
                          p.p_exact ? 1 : 0, p.p_k_halves, p.repack_bytes ? " repack" : "");
    } else {
        n = std::snprintf(buf, len, "prefill128 splits=%d", p.p_splits);
    }
    return n < 0 || (size_t)n >= len ? PW4_ERR_ARG : PW4_OK;
}

int pw4_abi_version(void) { return PW4_ABI_VERSION; }

int64_t pw4_marlin_words(int64_t N, int64_t K) {
    if (N < 0 || K < 0) return 0;
    return round_up(N, kMarlinBN) * round_up(K, kMarlinBK) / 8;
}

int pw4_repack_w4a16(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int64_t N, int64_t K,
                     int64_t group_size, int32_t* weight_marlin, float* scale_marlin, pw4_stream_t stream) {
    // armed timing events: the repack kernel's start and end
    const KernelEvents ev = take_kernel_events();
    if (N < 0 || K < 0) return PW4_ERR_ARG;
    if (group_size <= 0 || group_size % 16 != 0) return PW4_ERR_SHAPE;
    if (K % 8 != 0 || K % group_size != 0) return PW4_ERR_SHAPE;
    if (N > INT32_MAX || K > INT32_MAX) return PW4_ERR_SHAPE;
    int st;
    switch (scale_dtype) {
        case PW4_DTYPE_F32: st = 0; break;
        case PW4_DTYPE_F16: st = 1; break;
        case PW4_DTYPE_BF16: st = 2; break;
        default: return PW4_ERR_ARG;
    }
    if (N > 0 && K > 0 && (!weight_packed || !weight_marlin)) return PW4_ERR_ARG;
    if (N > 0 && K > 0 && (!weight_scale || !scale_marlin)) return PW4_ERR_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = launch_repack_ct(reinterpret_cast<const uint32_t*>(weight_packed), weight_scale, st,
                                          reinterpret_cast<uint32_t*>(weight_marlin), scale_marlin, (int)N, (int)K,
                                          (int)group_size, s, ev.start, ev.stop);
    if (e != hipSuccess) return hip_fail(e);
    return PW4_OK;
}

size_t pw4_gemm_w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int64_t num_splits) {
    if (check_common(M, N, K, group_size, PW4_DTYPE_F16) != PW4_OK || M == 0 || N == 0) return 0;
    // the plan may differ by activation dtype (LDS budget): size for both
    return std::max(make_plan(LAYOUT_CT, PW4_DTYPE_F16, S_F32, false, M, N, K, group_size, false, num_splits).workspace(),
                    make_plan(LAYOUT_CT, PW4_DTYPE_BF16, S_F32, false, M, N, K, group_size, false, num_splits).workspace());
}

int pw4_gemm_w4a16(const void* x, int x_dtype, const int32_t* weight_packed, const float* weight_scale, void* y,
                   int64_t M, int64_t N, int64_t K, int64_t group_size, int64_t num_splits, void* workspace,
                   size_t workspace_bytes, pw4_stream_t stream) {
    const KernelEvents ev = take_kernel_events();
    int rc = check_common(M, N, K, group_size, x_dtype);
    if (rc != PW4_OK) return rc;
    if (num_splits < 0) return PW4_ERR_ARG;
    if (M == 0 || N == 0) return PW4_OK;
    if (!x || !weight_packed || !weight_scale || !y) return PW4_ERR_ARG;
    return run_gemm(LAYOUT_CT, x, x_dtype, reinterpret_cast<const uint32_t*>(weight_packed), weight_scale, S_F32,
                    nullptr, nullptr, y, M, N, K, group_size, num_splits, workspace, workspace_bytes,
                    reinterpret_cast<hipStream_t>(stream), ev);
}

size_t pw4_gemm_w4a16_marlin_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm,
                                            int64_t num_splits) {
    if (check_common(M, N, K, group_size, PW4_DTYPE_F16) != PW4_OK || M == 0 || N == 0) return 0;
    return std::max(
        make_plan(LAYOUT_MARLIN, PW4_DTYPE_F16, S_F16, true, M, N, K, group_size, has_perm != 0, num_splits).workspace(),
        make_plan(LAYOUT_MARLIN, PW4_DTYPE_BF16, S_F16, true, M, N, K, group_size, has_perm != 0, num_splits).workspace());
}

int pw4_gemm_w4a16_marlin(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                          int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M, int64_t N,
                          int64_t K, int64_t group_size, int64_t num_splits, void* workspace,
                          size_t workspace_bytes, pw4_stream_t stream) {
    const KernelEvents ev = take_kernel_events();
    int rc = check_common(M, N, K, group_size, x_dtype);
    if (rc != PW4_OK) return rc;
    if (num_splits < 0) return PW4_ERR_ARG;
    if (scale_dtype != PW4_DTYPE_F32 && scale_dtype != PW4_DTYPE_F16) return PW4_ERR_ARG;
    if (qzeros && N % 8 != 0) return PW4_ERR_SHAPE;
    if (M == 0 || N == 0) return PW4_OK;
    if (!x || !weight_marlin || !scales || !y) return PW4_ERR_ARG;
    return run_gemm(LAYOUT_MARLIN, x, x_dtype, reinterpret_cast<const uint32_t*>(weight_marlin), scales,
                    scale_dtype == PW4_DTYPE_F32 ? S_F32 : S_F16, reinterpret_cast<const uint32_t*>(qzeros), perm, y,
                    M, N, K, group_size, num_splits, workspace, workspace_bytes,
                    reinterpret_cast<hipStream_t>(stream), ev);
}

int pw4_gemm_w4a16_marlin_noalloc(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                                  int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M,
                                  int64_t N, int64_t K, int64_t group_size, int64_t num_splits, pw4_stream_t stream) {
    const KernelEvents ev = take_kernel_events();
    int rc = check_common(M, N, K, group_size, x_dtype);
    if (rc != PW4_OK) return rc;
    if (num_splits < 0) return PW4_ERR_ARG;
    if (scale_dtype != PW4_DTYPE_F32 && scale_dtype != PW4_DTYPE_F16) return PW4_ERR_ARG;
    if (qzeros && N % 8 != 0) return PW4_ERR_SHAPE;
    if (M == 0 || N == 0) return PW4_OK;
    if (!x || !weight_marlin || !scales || !y) return PW4_ERR_ARG;
    // the plan run_gemm will make, sized before anything is launched
    const size_t need = make_plan(LAYOUT_MARLIN, x_dtype, scale_dtype == PW4_DTYPE_F32 ? S_F32 : S_F16,
                                  qzeros != nullptr, M, N, K, group_size, perm != nullptr, num_splits, false,
                                  kStaticScratchBytes)
                            .workspace();
    if (need > kStaticScratchBytes) return PW4_ERR_WORKSPACE;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    void* ws = nullptr;
    if (need > 0) {
        rc = device_scratch(s, &ws);
        if (rc != PW4_OK) return rc;
    }
    return run_gemm(LAYOUT_MARLIN, x, x_dtype, reinterpret_cast<const uint32_t*>(weight_marlin), scales,
                    scale_dtype == PW4_DTYPE_F32 ? S_F32 : S_F16, reinterpret_cast<const uint32_t*>(qzeros), perm, y,
                    M, N, K, group_size, num_splits, ws, need > 0 ? kStaticScratchBytes : 0, s, ev, false,
                    kStaticScratchBytes);
}

size_t pw4_gemm_w4a16_silu_mul_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm) {
    if (check_common(M, N, K, group_size, PW4_DTYPE_F16) != PW4_OK || M == 0 || N == 0 || N % 16 != 0) return 0;
    return std::max(
        make_plan(LAYOUT_MARLIN, PW4_DTYPE_F16, S_F16, true, M, N, K, group_size, has_perm != 0, 0, true).workspace(),
        make_plan(LAYOUT_MARLIN, PW4_DTYPE_BF16, S_F16, true, M, N, K, group_size, has_perm != 0, 0, true).workspace());
}

int pw4_gemm_w4a16_silu_mul(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                            int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M, int64_t N,
                            int64_t K, int64_t group_size, void* workspace, size_t workspace_bytes,
                            pw4_stream_t stream) {
    const KernelEvents ev = take_kernel_events();
    int rc = check_common(M, N, K, group_size, x_dtype);
    if (rc != PW4_OK) return rc;
    if (scale_dtype != PW4_DTYPE_F32 && scale_dtype != PW4_DTYPE_F16) return PW4_ERR_ARG;
    if (N % 16 != 0) return PW4_ERR_SHAPE;  // whole gate|up strips of 8 + 8 columns
    if (M == 0 || N == 0) return PW4_OK;
    if (!x || !weight_marlin || !scales || !y) return PW4_ERR_ARG;
    return run_gemm(LAYOUT_MARLIN, x, x_dtype, reinterpret_cast<const uint32_t*>(weight_marlin), scales,
                    scale_dtype == PW4_DTYPE_F32 ? S_F32 : S_F16, reinterpret_cast<const uint32_t*>(qzeros), perm, y,
                    M, N, K, group_size, 0, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream), ev,
                    /*silu=*/true);
}

int pw4_gidx_to_perm(const int32_t* g_idx, int64_t K, int64_t group_size, int32_t* perm, int32_t* status_dev,
                     pw4_stream_t stream) {
    if (K < 0 || K > INT32_MAX) return PW4_ERR_ARG;
    if (group_size <= 0 || K % group_size != 0) return PW4_ERR_SHAPE;
    if (!status_dev || (K > 0 && (!g_idx || !perm))) return PW4_ERR_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = launch_gidx_perm(g_idx, perm, status_dev, (int)K, (int)group_size, s);
    if (e != hipSuccess) return hip_fail(e);
    return PW4_OK;
}

int pw4_repack_gptq(const int32_t* qweight, const int32_t* perm, int64_t N, int64_t K, int32_t* weight_marlin,
                    pw4_stream_t stream) {
    // armed timing events: the repack kernel's start and end
    const KernelEvents ev = take_kernel_events();
    if (N < 0 || K < 0 || N > INT32_MAX || K > INT32_MAX) return PW4_ERR_ARG;
    if (K % 8 != 0) return PW4_ERR_SHAPE;
    if (N > 0 && K > 0 && (!qweight || !weight_marlin)) return PW4_ERR_ARG;
    hipError_t e = launch_repack_gptq(reinterpret_cast<const uint32_t*>(qweight), perm,
                                      reinterpret_cast<uint32_t*>(weight_marlin), (int)N, (int)K,
                                      reinterpret_cast<hipStream_t>(stream), ev.start, ev.stop, cu_count(),
                                      repack_cols_override(), repack_grid_override());
    if (e != hipSuccess) return hip_fail(e);
    return PW4_OK;
}

}  // extern "C"
