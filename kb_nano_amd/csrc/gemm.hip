// Host side of the block-scaled FP8 GEMMs: the tile planner, the split-K
// arrival counters, the sorted-token launches and the C-ABI entry points.
// The kernels are in gemm_kernel.h.  This file is built with the VGPR-form
// MFMA option (kb_nano_amd/_build.py): its tiles keep their accumulators in
// VGPRs, where the FP32 contract's per-block rescale is one multiply per
// element instead of a read, multiply and write of an AGPR.  The 256x256
// tiles are launched from gemm_big.hip, built without it.
#include "gemm_kernel.h"

#include <algorithm>
#include <cstdio>
#include <map>
#include <mutex>
#include <tuple>

namespace kbn {

// Contiguous-layout grouped GEMMs read their padding rows as zeros up to this K.
#ifndef KBN_PAD_ZERO_MAX_K
#define KBN_PAD_ZERO_MAX_K 2048
#endif
constexpr int64_t kPadZeroMaxK = KBN_PAD_ZERO_MAX_K;

// Only tails whose split workgroups fit in one wave are split (more waves
// never measured faster, and the allocation-free entry point's scratch is
// sized for one wave).  Cost model in microseconds, fitted to sweeps of the
// split count over the 64x128, 128x128 and 256x256 tiles on MI355X:
//  * a workgroup streams about 55 KB of A and W tile rows per microsecond,
//    so a K block takes (bm + bn) * 128 B / 55 KB/us, and every workgroup
//    pays a pipeline fill of about two blocks;
//  * a split plan adds a fixed cost (slab stores and the reduction: about
//    3 us with the separate reduction launch, 2 us when the split launch
//    sums the slabs itself, as fused_split_sum allows), a cost per split (the depth of each tile's
//    sum: 0.2 / 0.4 us) and the slab traffic (0.45 us per MB of fp32
//    partials).
// Short K therefore stays unsplit (e.g. 128 x 12288 x 1536: 11.2 us data-
// parallel against 20.0 us split in two), and long K takes fewer, longer
// splits than a traffic-only model picks.
// Splits of the 64x64 tiles run at most this many K blocks: longer ones lose
// to 64x128 when the GEMM quantizes 33-64 bf16 rows itself (1024 x 28672 at
// 48 rows, 8 splits of 28 blocks: 27.5 us against 19.9 us; 1024 x 24576 at
// 64 rows, 8 of 24: 25.4 against 20.1 us), while 14-16 block splits measured
// faster on both paths (1024 x 28672 at 32 rows, 14 of 16: fp8 input 16.0 ->
// 14.5 us, bf16 input 19.7 -> 18.9 us).
constexpr int kNarrowMaxKb = 16;

// Returns the modelled time of the whole plan (data-parallel waves plus the
// tail).  The 64x64 tiles (narrow) stream fewer bytes per K block but not
// proportionally faster: their split sweeps fit about 0.40 us per block
// (41 KB of tile rows per us and workgroup), against 0.30 us at the 55 KB/us
// of the larger tiles; they count one workgroup slot per CU, as measured,
// and split K whenever a split fits (unsplit, they measured slower than
// every split plan at K = 2048: 1024 x 2048 M = 64 above 7.7 us against
// 7.4 us for three splits).
static double plan_tail(Schedule& s, int64_t M, int KBT, bool allow_split = true, bool narrow = false) {
    const int occ = narrow ? 1 : gemm_occupancy(s.bm, s.bn, s.stages, s.fuse_a);
    const int cus = cu_count();
    const int64_t slots = (int64_t)occ * cus;
    s.dp_tiles = s.tiles;
    s.splits = 1;
    s.kb_per_split = KBT;
    const double fill = 2.0;
    const double t_block = (double)(s.bm + s.bn) * kRowB / (narrow ? 41e3 : 55e3);   // us per K block
    const int64_t waves = s.tiles / slots, rem = s.tiles - waves * slots;
    const double t_wave = (KBT + fill) * t_block;
    if (rem == 0 || KBT < 8 || !allow_split) return (double)(waves + (rem > 0)) * t_wave;
    const double per_mb = 0.45;
    const double slab_mb = (double)std::min<int64_t>(M, s.bm) * s.bn * 4 / 1e6;   // one partial slab
    // the tail as one more data-parallel wave (narrow tiles: only if no split fits)
    double best = narrow ? 1e30 : t_wave;
    for (int sp = 2; sp <= 32 && sp <= KBT / 4; ++sp) {
        const int kbps = (KBT + sp - 1) / sp;
        const int ss = (KBT + kbps - 1) / kbps;
        const int64_t wgs = rem * ss;
        if (wgs > slots) break;
        const bool fused = fused_split_sum(s.bm, s.bn, M, ss, kbps);
        if (narrow && (!fused || kbps > kNarrowMaxKb)) continue;   // narrow tiles: the measured regime
        const double fixed = fused ? 2.0 : 3.0, per_split = fused ? 0.4 : 0.2;
        const double cost = (kbps + fill) * t_block + fixed + per_split * ss + per_mb * slab_mb * ss * rem;
        if (cost < best - 1e-9) {
            best = cost;
            s.splits = ss;
            s.kb_per_split = kbps;
            s.fused = fused;
        }
    }
    if (s.splits > 1) {
        s.dp_tiles = waves * slots;
        s.ws_bytes = (int64_t)s.splits * rem * s.bm * s.bn * 4;
    } else {
        best = t_wave;
    }
    return (double)waves * t_wave + best;
}

// Weight-streaming plans (M <= 64, UE8M0).  Narrow weights (at most
// kNarrowTiles 64x128 tiles, N <= 4096) take 64x64 tiles (four stages, one
// workgroup per CU): twice the tiles, so the same CUs stream with fewer K
// splits per tile and half the slab per split.  Measured on MI355X
// (HIP-graph replays, us per call, best 64x128 plan -> 64x64) at every
// N in {1024, 2048, 3072, 4096}, K in {2048, 7168}, M in {1, 32, 64}, the
// fp8-input GEMM was 2-25% faster: 2048 x 2048 M = 64 9.7 -> 7.4, M = 1
// 7.3 -> 6.3; 4096 x 7168 M = 64 14.0 -> 11.3, M = 1 10.9 -> 9.5.  From 48
// tiles (6144 columns) up, 64x128 measured as fast or faster (6144 x 7168
// M = 1 12.6 against 13.7).
constexpr int64_t kNarrowTiles = 32;

static void plan_weight_stream(Schedule& s, int64_t M, int64_t N, int64_t K, bool allow_split, bool narrow_ok) {
    const int KBT = (int)(K / kGroup);
    s.bm = 64; s.bn = 128;
    s.tiles = ((M + 63) / 64) * ((N + 127) / 128);
    if (narrow_ok && allow_split && s.tiles <= kNarrowTiles) {
        // 64x64 only with a split summed in the launch (the measured regime;
        // long K at 49-64 rows, e.g. 1024 x 28672, finds none and keeps
        // 64x128 with the separate reduction)
        Schedule n = s;
        n.bn = 64;
        n.tiles = ((M + 63) / 64) * ((N + 63) / 64);
        n.stages = 4;
        plan_tail(n, M, KBT, true, true);
        if (n.splits > 1) {
            s = n;
            return;
        }
    }
    s.stages = s.tiles > cu_count() ? 3 : 4;
    plan_tail(s, M, KBT, allow_split);
}

// Arrival counters of the fused split-K reduction, in a region of a static
// device array.  A region serves one stream's eager launches (launches on
// one stream never overlap) or the launches captured on one stream under one
// capture: streams forked into a capture share its id, but the nodes
// captured on one of them form a dependency chain, and a captured graph is
// never replayed concurrently with itself.  Distinct (capture, stream) pairs
// and eager streams get distinct regions, so concurrent launches never share
// a counter.  Every launch leaves its counters at zero.  When the regions are
// used up (or the array's address cannot be had), launches fall back to the
// separate reduction kernel: the results are the same, each such call costs
// one more launch (about 3 us of host time).  The fallbacks are counted
// (kbn_splitk_counter_stats) and the first one is reported once on stderr.
// A tail of the 64-row tiles (the only ones whose split launch sums its own
// slabs) has fewer tiles than two workgroups per CU, i.e. at most 512 on a
// 256-CU device; larger tails never take a region.
constexpr int kFlagRegion = 512;    // tail tiles per launch
constexpr int kFlagRegions = 1024;
constexpr int kFlagDevices = 64;
__device__ __attribute__((aligned(256))) unsigned g_splitk_flags[kFlagRegions * kFlagRegion];

// Which region each (device, capture id + 1 or 0 for eager launches, stream)
// key holds.  Host bookkeeping only (no HIP calls), so the CPU tests can
// drive a private instance through kbn_debug_splitk_regions.
struct FlagRegionTable {
    std::map<std::tuple<int, uint64_t, uint64_t>, int> region;
    int used[kFlagDevices] = {};
    int64_t fallbacks = 0;
    // The key's region, a new one if it has none, or -1 (counted) when the
    // device's regions are all taken.
    int acquire(int dev, uint64_t cap_key, uint64_t stream) {
        const auto key = std::make_tuple(dev, cap_key, stream);
        auto it = region.find(key);
        if (it != region.end()) return it->second;
        if (used[dev] >= kFlagRegions) {
            ++fallbacks;
            return -1;
        }
        region.emplace(key, used[dev]);
        return used[dev]++;
    }
};

static std::mutex g_flag_mu;
static FlagRegionTable g_flag_table;

unsigned* splitk_flags_for(hipStream_t st, int64_t tail_tiles) {
    static unsigned* base[kFlagDevices] = {};
    if (tail_tiles > kFlagRegion) return nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kFlagDevices) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(st, &cs, &cid) != hipSuccess) return nullptr;
    if (cs != hipStreamCaptureStatusNone && cs != hipStreamCaptureStatusActive) return nullptr;
    const bool cap = cs == hipStreamCaptureStatusActive;
    std::lock_guard<std::mutex> lock(g_flag_mu);
    if (!base[dev]) {
        if (cap) return nullptr;   // resolved on the first eager launch, not inside a capture
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_splitk_flags)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        base[dev] = static_cast<unsigned*>(p);
    }
    // eager launches key on 0, captured ones on capture id + 1
    const int r = g_flag_table.acquire(dev, cap ? (uint64_t)cid + 1 : (uint64_t)0, (uint64_t)(uintptr_t)st);
    if (r < 0) {
        if (g_flag_table.fallbacks == 1)
            std::fprintf(stderr,
                         "kb_nano_amd: all %d split-K counter regions of device %d are taken (one per eager stream "
                         "and per captured stream); later small-M split launches on new streams or captures use "
                         "the separate reduction kernel (same results, one launch more)\n",
                         kFlagRegions, dev);
        return nullptr;
    }
    return base[dev] + (int64_t)r * kFlagRegion;
}

}  // namespace kbn

// Regions in use on the busiest device, regions per device, and split
// launches that took the separate reduction because no region was free.
extern "C" int kbn_splitk_counter_stats(int64_t* regions_used, int64_t* regions_total, int64_t* fallbacks) {
    using namespace kbn;
    std::lock_guard<std::mutex> lock(g_flag_mu);
    int most = 0;
    for (int d = 0; d < kFlagDevices; ++d) most = std::max(most, g_flag_table.used[d]);
    if (regions_used) *regions_used = most;
    if (regions_total) *regions_total = kFlagRegions;
    if (fallbacks) *fallbacks = g_flag_table.fallbacks;
    return 0;
}

// Test hook: n_keys distinct eager streams on device 0 of a fresh region
// table, then the first key again; out_region[i] gets key i's region (-1:
// none left) and out_region[n_keys] the repeated key's; *out_fallbacks the
// table's fallback count.  No HIP calls.
extern "C" int kbn_debug_splitk_regions(int64_t n_keys, int32_t* out_region, int64_t* out_fallbacks) {
    using namespace kbn;
    KBN_CHECK_ARG(n_keys >= 1 && n_keys <= 4 * kFlagRegions && out_region && out_fallbacks,
                  "debug_splitk_regions: bad arguments");
    FlagRegionTable t;
    for (int64_t i = 0; i < n_keys; ++i) out_region[i] = t.acquire(0, 0, 0x1000 + 8 * (uint64_t)i);
    out_region[n_keys] = t.acquire(0, 0, 0x1000);
    *out_fallbacks = t.fallbacks;
    return 0;
}

namespace kbn {

// Sorted-token layout: the activation scales of every row R below the padded
// total, gathered into column-major [KB, EM] order (row R of block kb at
// kb * EM + R; padding rows get 0), so the GEMM's per-row scale loads are
// contiguous across lanes instead of one cache line per lane.
__global__ __launch_bounds__(256) void sorted_scale_gather_kernel(const GemmArgs a, float* out, int KB) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int R = (int)(i % a.M);
    const int kb = (int)(i / a.M);
    if (kb >= KB || R >= a.num_post_pad[0]) return;
    const int t = a.sorted_ids ? a.sorted_ids[R] : (R % a.block_m == 0 ? R / a.block_m : -1);
    float v = 0.f;
    if (t >= 0 && t < a.num_valid) v = a.sA[(int64_t)(t / a.a_row_div) * a.sA_sm + (int64_t)kb * a.sA_sk];
    out[(int64_t)kb * a.M + R] = v;
}

// Sorted-token (fused MoE) launch: one workgroup per BM x BN tile of the
// padded row grid; tiles past the padded total exit at once.
template <int BM, int BN, int kStages>
static int launch_sorted(GemmArgs a, hipStream_t st, const char* what) {
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    KBN_CHECK_ARG(tiles <= 0x7FFFFFFFLL, "%s: too many tiles", what);
    if (tiles == 0) return 0;
    a.tile_base = 0;
    a.tile_count = (int)tiles;
    a.splits = 1;
    a.kb_per_split = a.K / kRowB;
    a.group_m = moe_group_m(a.K);
    const int64_t grid = moe_dealt_grid(a.tiles_m, a.tiles_n, a.group_m);
    KBN_CHECK_ARG(grid <= 0x7FFFFFFFLL, "%s: too many tiles", what);
    gemm_bs_kernel<BM, BN, kStages, false, false, false, 4, true><<<dim3((unsigned)grid), dim3(256), 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

}  // namespace kbn

using namespace kbn;

static int check_common(const char* what, const void* A, int64_t lda, const void* W, int64_t ldw, const void* D,
                        int64_t ldd, int64_t M, int64_t N, int64_t K) {
    KBN_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
    KBN_CHECK_ARG(K % kGroup == 0, "%s: K=%lld must be a multiple of 128", what, (long long)K);
    KBN_CHECK_ARG(M <= 0x7FFFFFFFLL && N <= 0x7FFFFFFFLL && K <= 0x7FFFFFFFLL, "%s: shape too large", what);
    KBN_CHECK_ARG(lda >= K && ldw >= K && ldd >= N, "%s: leading dimension too small", what);
    KBN_CHECK_ARG(aligned16(A) && aligned16(W) && lda % 16 == 0 && ldw % 16 == 0,
                  "%s: A and W rows must be 16-byte aligned", what);
    KBN_CHECK_ARG(((reinterpret_cast<uintptr_t>(D) & 1u) == 0), "%s: D must be 2-byte aligned", what);
    // every per-tile byte offset handed to the buffer unit must fit 32 bits
    KBN_CHECK_ARG(lda * 256 + K < 0x7FFFFFFFLL && ldw * 256 + K < 0x7FFFFFFFLL && ldd * 2 * 256 < 0x7FFFFFFFLL,
                  "%s: leading dimension too large", what);
    return 0;
}

// Bytes spanned by a [rows, kb] fp32 scale view with the given strides.
static int64_t scale_bytes(int64_t rows, int64_t kb, int64_t sm, int64_t sk) {
    if (rows <= 0 || kb <= 0) return 0;
    return ((rows - 1) * sm + (kb - 1) * sk + 1) * 4;
}

// The kernels address scales with 32-bit byte offsets from the buffer base.
static int check_scale_ranges(const char* what, int64_t M, int64_t K, int64_t sm, int64_t sk, int64_t nb,
                              int64_t sw_ld) {
    KBN_CHECK_ARG(sm >= 0 && sk >= 0, "%s: negative activation-scale stride", what);
    KBN_CHECK_ARG(scale_bytes(M, K / kGroup, sm, sk) < 0x7FFFFFFFLL, "%s: activation scales span >= 2 GiB", what);
    KBN_CHECK_ARG(nb * sw_ld * 4 < 0x7FFFFFFFLL, "%s: weight scales span >= 2 GiB", what);
    return 0;
}

// Measured in one process against the 256x256-only plan, same data (DeepSeek-V3
// recipe, inputs rotated past the MALL): down 7168 x 18432 and o 7168 x 16384
// at M = 4096 422-425 / 384-389 us against 431-434 / 394-396 us; the partial
// wave it removes runs at a higher clock (fewer CUs busy under the power
// cap), so the gain is 2%, not the 11% the wave count suggests.  With short K
// the second launch's fill costs more than that (3000 x 7168 x 4096: 100 us
// against 97), so only K of at least 8192 takes it.
constexpr int64_t kMixedMinK = 8192;

// 256x256 tiles whose last wave would run partly empty: move the last n192
// columns to 256x192 tiles in a second launch when both launches then fill
// whole waves.  Cost in units of a 256x256 wave: a wave of 256x192 tiles
// does 3/4 of the work with about 4% more fetch and fragment traffic per
// FLOP, so it is counted as 0.78; the mixed plan is taken when it saves at
// least 5%.  (DeepSeek-V3 down / o at M = 4096: 448 tiles = 1.75 waves on
// 256 CUs become one wave of 256x256 and one of 256x192 tiles.)
static void plan_mixed_192(Schedule& s, int64_t M, int64_t N) {
    const int64_t cus = cu_count();
    const int64_t tm = (M + 255) / 256;
    auto waves = [&](int64_t t) { return (t + cus - 1) / cus; };
    const double base = (double)waves(s.tiles);
    double best = base * 0.95;
    for (int64_t b = 1; 192 * b <= N; ++b) {
        const int64_t rest = N - 192 * b;
        if (rest % 256) continue;
        const double cost = (double)waves(tm * (rest / 256)) + 0.78 * (double)waves(tm * b);
        if (cost < best - 1e-9) {
            best = cost;
            s.n192 = (int)(192 * b);
        }
    }
    if (s.n192) s.tiles = s.dp_tiles = tm * ((N - s.n192) / 256 + s.n192 / 192);
}

// Dense tile configuration: 256x256 (2 LDS stages) when M > 128 (128x256,
// 3 stages, under the FP32 contract, whose per-row mantissa state does not
// fit next to a 256x256 tile's accumulators), 128x128 (4 stages) for
// 64 < M <= 128, 64x128 (3 stages, two workgroups per CU) for M <= 64,
// where the weights dominate the traffic.
static Schedule dense_schedule(int64_t M, int64_t N, int64_t K, int ue8m0, bool allow_split) {
    Schedule s;
    if (M > 128 && !ue8m0) {
        s.bm = 128; s.bn = 256; s.stages = 3;
    } else if (M > 128) {
        s.bm = 256; s.bn = 256; s.stages = 2;
    } else if (M > 64) {
        s.bm = 128; s.bn = 128; s.stages = 4;
    } else {
        // weight-streaming tiles: two workgroups per CU (3 stages) when there
        // are more tiles than CUs; otherwise one per CU with a deeper
        // pipeline (4 stages) and the tail split over K over fewer, longer
        // workgroups (Llama-70B decode qkv / o / down: 8-20% faster than 3
        // stages at two per CU; gate_up's 448 tiles: 6% slower); narrow
        // weights may take 64x64 tiles (plan_weight_stream)
        plan_weight_stream(s, M, N, K, allow_split, ue8m0 != 0);
        return s;
    }
    s.tiles = ((M + s.bm - 1) / s.bm) * ((N + s.bn - 1) / s.bn);
    s.dp_tiles = s.tiles;
    s.kb_per_split = (int)(K / kGroup);
    if (allow_split) plan_tail(s, M, (int)(K / kGroup));
    if (s.bm == 256 && s.splits == 1 && K >= kMixedMinK) plan_mixed_192(s, M, N);
    return s;
}

// Tile plan of the GEMM over bf16 activations (M <= 64, quantized by the
// kernel): the 64x128 weight-streaming tiles with 16, 32 or 64 bf16 A rows
// of 256 B per stage (as M needs), 4 stages when the tiles do not fill the
// CUs, else 3 (two workgroups per CU up to 32 rows: 66 / 78 KB).
// The tiles and K partition are those of the fp8-input GEMM's plan for the
// same shape (plan_weight_stream), so the results are bit-identical to
// quant + fp8_gemm_nt.
static Schedule bf16a_schedule(int64_t M, int64_t N, int64_t K, bool allow_split) {
    Schedule s;
    s.fuse_a = M <= 16 ? 1 : M <= 32 ? 2 : 4;
    plan_weight_stream(s, M, N, K, allow_split, true);
    return s;
}

// Dense UE8M0 tiles with packed per-row weight scales (a.sWp).
static int dispatch_dense_roww(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    if (sc.bm == 256 && sc.bn == 256) return launch_gemm_256_roww(a, sc, K, st, what);
    if (sc.bm == 128 && sc.bn == 128) return launch_gemm<128, 128, 4, true, false, 4, 0, true>(a, sc, st, what);
    if (sc.bm == 64 && sc.bn == 128) {
        if (sc.stages == 4) return launch_gemm<64, 128, 4, true, false, 4, 0, true>(a, sc, st, what);
        return launch_gemm<64, 128, 3, true, false, 4, 0, true>(a, sc, st, what);
    }
    if (sc.bm == 64 && sc.bn == 64 && sc.stages == 4)
        return launch_gemm<64, 64, 4, true, false, 4, 0, true>(a, sc, st, what);
    set_error("%s: no packed-scale kernel for %dx%d tiles", what, sc.bm, sc.bn);
    return 1;
}

template <bool kUe8m0>
static int dispatch_dense(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    if constexpr (kUe8m0) {
        if (sc.bm == 256 && sc.bn == 256) return launch_gemm_256(a, sc, K, st, what);
    } else {
        if (sc.bm == 128 && sc.bn == 256) return launch_gemm<128, 256, 3, false, false>(a, sc, st, what);
    }
    if (sc.bm == 128 && sc.bn == 128) return launch_gemm<128, 128, 4, kUe8m0, false>(a, sc, st, what);
    if (sc.bm == 64 && sc.bn == 128) {
        if (sc.stages == 4) return launch_gemm<64, 128, 4, kUe8m0, false>(a, sc, st, what);
        return launch_gemm<64, 128, 3, kUe8m0, false>(a, sc, st, what);
    }
    if constexpr (kUe8m0) {
        if (sc.bm == 64 && sc.bn == 64 && sc.stages == 4) return launch_gemm<64, 64, 4, true, false>(a, sc, st, what);
    }
    set_error("%s: no kernel for %dx%d tiles", what, sc.bm, sc.bn);
    return 1;
}

// Device scratch of the allocation-free GEMM entry point: the split-K slabs
// of kbn_fp8_gemm_nt_noalloc.  One copy per GPU (its own address on each),
// held until the process ends.  The size covers every split plan on a
// 256-CU device: a tail is split only when its split workgroups fit in one
// wave of at most 256 workgroup slots for the 256x256 tiles, i.e. at most
// 256 fp32 slabs of 256 x 256.  Calls on one GPU share it.
constexpr int64_t kScratchBytes = 64ll << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device with that device current (host code never uses the symbol itself,
// which is only a host-side stand-in).  nullptr (and the error set) if the
// lookup fails.
static void* scratch_ptr(const char* what) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* ptr[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        set_error("%s: no current HIP device (or device index >= %d)", what, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev, hipGetErrorString(e));
            return nullptr;
        }
        ptr[dev] = p;
    }
    return ptr[dev];
}

// The checks launch_gemm makes before each launch, made ahead of any launch
// (kbn_fp8_linear_forward validates its GEMM before it enqueues the quant).
static int check_plan(const GemmArgs& a, const Schedule& sc, const char* what) {
    const int64_t tiles = sc.n192 ? (((int64_t)a.M + 255) / 256) * ((a.N - sc.n192) / 256 + sc.n192 / 192)
                                  : (((int64_t)a.M + sc.bm - 1) / sc.bm) * (((int64_t)a.N + sc.bn - 1) / sc.bn);
    KBN_CHECK_ARG(!sc.n192 || (sc.bm == 256 && sc.splits == 1 && (a.N - sc.n192) % 256 == 0 && sc.n192 % 192 == 0),
                  "%s: bad mixed 256/192 plan", what);
    KBN_CHECK_ARG(tiles == sc.tiles && tiles <= 0x7FFFFFFFLL, "%s: too many tiles", what);
    if (a.P && sc.splits > 1 && sc.dp_tiles < tiles) {
        const int64_t need = (int64_t)sc.splits * (tiles - sc.dp_tiles) * sc.bm * sc.bn * 4;
        KBN_CHECK_ARG(need < 0x7FFFFFFFLL && need <= a.ws_bytes && aligned16(a.P),
                      "%s: workspace of %lld bytes is smaller than the %lld the split plan writes", what,
                      (long long)a.ws_bytes, (long long)need);
        KBN_CHECK_ARG((int64_t)sc.splits * sc.kb_per_split >= a.K / kRowB &&
                          (int64_t)(sc.splits - 1) * sc.kb_per_split < a.K / kRowB,
                      "%s: split plan does not cover K in %d non-empty splits", what, sc.splits);
    }
    return 0;
}

// Arguments, tile plan and workspace of a dense GEMM, all validated; nothing
// is launched.  gemm_nt_launch then enqueues it.
// Packed per-row UE8M0 weight scales (sWp != nullptr, scale_ue8m0 = 1):
// int32 [N, ceil(K/512)] with strides (sWp_sn, sWp_sk) in elements.
struct PackedW {
    const int32_t* p = nullptr;
    int64_t sn = 0, sk = 0;
};

static int gemm_nt_prepare(const char* what, const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                           int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                           void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0,
                           void* workspace, int64_t workspace_bytes, bool use_scratch, GemmArgs& a, Schedule& sc,
                           const PackedW& pw = PackedW{}) {
    if (int rc = check_common(what, A, lda, W, ldw, D_bf16, ldd, M, N, K)) return rc;
    a = GemmArgs{};
    if (M == 0 || N == 0) return 0;
    KBN_CHECK_ARG(K > 0, "%s: K must be positive", what);
    KBN_CHECK_ARG(sA && (sW || pw.p), "%s: null scale pointer", what);
    a.A = (const uint8_t*)A; a.lda = lda;
    if (pw.p) {
        KBN_CHECK_ARG(scale_ue8m0, "%s: packed weight scales are UE8M0 exponents", what);
        const int64_t words = (K / kGroup + 3) / 4;
        KBN_CHECK_ARG(pw.sn >= 0 && pw.sk >= 0 && (N == 1 || pw.sn > 0) && (words == 1 || pw.sk > 0),
                      "%s: bad packed weight-scale strides", what);
        const int64_t span = ((N - 1) * pw.sn + (words - 1) * pw.sk + 1) * 4;
        KBN_CHECK_ARG(span < 0x7FFFFFFFLL, "%s: packed weight scales span >= 2 GiB", what);
        KBN_CHECK_ARG(((reinterpret_cast<uintptr_t>(pw.p) & 3u) == 0), "%s: packed weight scales must be 4-byte aligned",
                      what);
        a.sWp = pw.p; a.sWp_sn = pw.sn; a.sWp_sk = pw.sk; a.sWp_bytes = span;
        sW_ld = K / kGroup;   // the block-scale path is not used
        if (int rc = check_scale_ranges(what, M, K, sA_stride_m, sA_stride_k, 1, 1)) return rc;
    } else {
        KBN_CHECK_ARG(sW_ld >= K / kGroup, "%s: weight-scale row stride %lld < K/128", what, (long long)sW_ld);
        if (int rc = check_scale_ranges(what, M, K, sA_stride_m, sA_stride_k, (N + kGroup - 1) / kGroup, sW_ld))
            return rc;
    }
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
    a.sA_bytes = scale_bytes(M, K / kGroup, sA_stride_m, sA_stride_k);
    a.W = (const uint8_t*)W; a.ldw = ldw; a.w_estride = 0;
    a.sW = sW; a.sW_ld = sW_ld; a.sW_estride = 0;
    a.D = (uint16_t*)D_bf16; a.ldd = ldd;
    a.vec_store = (reinterpret_cast<uintptr_t>(D_bf16) % 16 == 0) && (ldd % 8 == 0);
    a.expert_ids = nullptr;
    a.M = (int)M; a.N = (int)N; a.K = (int)K; a.E = 1;
    sc = dense_schedule(M, N, K, scale_ue8m0, workspace != nullptr || use_scratch);
    if (use_scratch && sc.splits > 1) {
        KBN_CHECK_ARG(sc.ws_bytes <= kScratchBytes,
                      "%s: the split plan of M=%lld N=%lld K=%lld needs %lld bytes of scratch, more than the %lld "
                      "this library holds per GPU",
                      what, (long long)M, (long long)N, (long long)K, (long long)sc.ws_bytes, (long long)kScratchBytes);
        workspace = scratch_ptr(what);
        if (!workspace) return 1;
        workspace_bytes = kScratchBytes;
    }
    if (sc.splits > 1) {
        if (workspace_bytes >= sc.ws_bytes) {
            KBN_CHECK_ARG(aligned16(workspace), "%s: workspace must be 16-byte aligned", what);
            a.P = (float*)workspace;
            a.ws_bytes = workspace_bytes;
        } else {
            sc = dense_schedule(M, N, K, scale_ue8m0, false);
        }
    }
    return check_plan(a, sc, what);
}

static int gemm_nt_launch(const GemmArgs& a, const Schedule& sc, int scale_ue8m0, void* stream, const char* what) {
    if (a.M == 0 || a.N == 0) return 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (a.sWp) return dispatch_dense_roww(a, sc, a.K, st, what);
    return scale_ue8m0 ? dispatch_dense<true>(a, sc, a.K, st, what) : dispatch_dense<false>(a, sc, a.K, st, what);
}

static int gemm_nt_impl(const char* what, const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                        int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld, void* D_bf16,
                        int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0, void* workspace,
                        int64_t workspace_bytes, void* stream, bool use_scratch = false) {
    GemmArgs a;
    Schedule sc;
    if (int rc = gemm_nt_prepare(what, A, lda, sA, sA_stride_m, sA_stride_k, W, ldw, sW, sW_ld, D_bf16, ldd, M, N, K,
                                 scale_ue8m0, workspace, workspace_bytes, use_scratch, a, sc))
        return rc;
    return gemm_nt_launch(a, sc, scale_ue8m0, stream, what);
}

extern "C" int kbn_fp8_gemm_nt(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                               int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                               void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0,
                               void* stream) {
    return gemm_nt_impl("fp8_gemm_nt", A, lda, sA, sA_stride_m, sA_stride_k, W, ldw, sW, sW_ld, D_bf16, ldd, M, N,
                        K, scale_ue8m0, nullptr, 0, stream);
}

extern "C" int64_t kbn_fp8_gemm_nt_workspace_bytes(int64_t M, int64_t N, int64_t K, int scale_ue8m0) {
    if (M <= 0 || N <= 0 || K <= 0 || K % kGroup != 0 || M > 0x7FFFFFFFLL || N > 0x7FFFFFFFLL) return 0;
    return dense_schedule(M, N, K, scale_ue8m0, true).ws_bytes;
}

extern "C" int kbn_fp8_gemm_nt_ws(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                  int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                                  void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
    return gemm_nt_impl("fp8_gemm_nt_ws", A, lda, sA, sA_stride_m, sA_stride_k, W, ldw, sW, sW_ld, D_bf16, ldd, M,
                        N, K, scale_ue8m0, workspace, workspace_bytes, stream);
}

extern "C" int kbn_fp8_gemm_nt_packed_ws(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                         int64_t sA_stride_k, const void* W, int64_t ldw, const int32_t* sW_packed,
                                         int64_t sWp_stride_n, int64_t sWp_stride_k, void* D_bf16, int64_t ldd,
                                         int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
    const char* what = "fp8_gemm_nt_packed_ws";
    GemmArgs a;
    Schedule sc;
    PackedW pw;
    pw.p = sW_packed; pw.sn = sWp_stride_n; pw.sk = sWp_stride_k;
    if (int rc = gemm_nt_prepare(what, A, lda, sA, sA_stride_m, sA_stride_k, W, ldw, nullptr, 0, D_bf16, ldd, M, N, K,
                                 1, workspace, workspace_bytes, false, a, sc, pw))
        return rc;
    return gemm_nt_launch(a, sc, 1, stream, what);
}

extern "C" int kbn_per_token_group_quant_fp8(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x, void* q_fp8,
                                             int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g,
                                             float eps, int use_ue8m0, void* stream);

// Fp8Linear.forward's two launches behind one call: the 1x128 quant of the
// bf16 input into q / scale, then the block-scaled GEMM of q with W.  Every
// argument of both is checked before either launches.
extern "C" int kbn_fp8_linear_forward(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x, void* q_fp8,
                                      int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g, float eps,
                                      int quant_ue8m0, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                                      void* D_bf16, int64_t ldd, int64_t N, int scale_ue8m0, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
    const char* what = "fp8_linear_forward";
    if (int rc = check_common(what, q_fp8, ld_q, W, ldw, D_bf16, ldd, M, N, K)) return rc;
    if (M == 0 || N == 0) return 0;
    KBN_CHECK_ARG(K > 0 && x_bf16 && scale && sW, "%s: null pointer or empty K", what);
    KBN_CHECK_ARG(aligned16(x_bf16) && ld_x % 8 == 0 && ld_x >= K, "%s: input rows must be 16-byte aligned", what);
    KBN_CHECK_ARG(M <= 0x3FFFFFFFLL, "%s: shape too large", what);
    KBN_CHECK_ARG(sW_ld >= K / kGroup, "%s: weight-scale row stride %lld < K/128", what, (long long)sW_ld);
    if (int rc = check_scale_ranges(what, M, K, s_stride_m, s_stride_g, (N + kGroup - 1) / kGroup, sW_ld)) return rc;
    GemmArgs a;
    Schedule sc;
    if (int rc = gemm_nt_prepare(what, q_fp8, ld_q, scale, s_stride_m, s_stride_g, W, ldw, sW, sW_ld, D_bf16, ldd, M,
                                 N, K, scale_ue8m0, workspace, workspace_bytes, false, a, sc))
        return rc;
    if (int rc = kbn_per_token_group_quant_fp8(x_bf16, M, K, ld_x, q_fp8, ld_q, scale, s_stride_m, s_stride_g, eps,
                                               quant_ue8m0, stream))
        return rc;
    return gemm_nt_launch(a, sc, scale_ue8m0, stream, what);
}

extern "C" int64_t kbn_fp8_gemm_bf16a_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || M > 64 || N <= 0 || K <= 0 || K % kGroup != 0 || N > 0x7FFFFFFFLL) return 0;
    return bf16a_schedule(M, N, K, true).ws_bytes;
}

// Whether the bf16-activation GEMM is expected to beat quant + GEMM (the
// separate quant launch costs 3-5 us per call on MI355X).  Up to 32 rows the
// in-kernel quant of the 16 or 32 loaded rows costs each workgroup well under
// that (measured on every Llama-70B decode shape and 2048/7168 x 2048: 0.5-4.7
// us faster, gate_up at 32 rows even).  With 64 rows (16 per wavefront) it
// costs about 0.1-0.3 us per K block, so it is taken only when the plan
// splits K into workgroups of at most 16 blocks within one wave of tiles
// (2048 x 2048, o); long K per workgroup (qkv 22, down 56 blocks), more
// tiles than CUs (gate_up: its 102 KB stage set drops to one workgroup per
// CU) and unsplit plans stay with quant + GEMM.  On the 64x64 tiles of narrow
// weights the fp8 GEMM gains more than the in-kernel quant, so 64 rows take
// it only for K <= 4096 (4096 x 7168: 17.5 us, against 11.3 us of GEMM plus
// the 3-5 us quant launch; 2048 x 2048: 9.8 us against 7.4 us plus the quant).
extern "C" int kbn_fp8_gemm_bf16a_preferred(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || M > 64 || N <= 0 || K <= 0 || K % kGroup != 0 || N > 0x7FFFFFFFLL) return 0;
    if (M <= 32) return 1;
    const Schedule s = bf16a_schedule(M, N, K, true);
    if (s.bn == 64 && K > 4096) return 0;
    return (s.tiles <= (int64_t)cu_count() && s.splits > 1 && s.kb_per_split <= 16) ? 1 : 0;
}

extern "C" int kbn_debug_gemm_plan(int64_t M, int64_t N, int64_t K, int scale_ue8m0, int bf16a, int64_t* out) {
    KBN_CHECK_ARG(out && M > 0 && N > 0 && K > 0 && K % kGroup == 0 && (!bf16a || M <= 64),
                  "debug_gemm_plan: bad arguments");
    const Schedule s = bf16a ? bf16a_schedule(M, N, K, true) : dense_schedule(M, N, K, scale_ue8m0, true);
    const int64_t v[9] = {s.bm, s.bn, s.stages, s.tiles, s.dp_tiles, s.splits, s.kb_per_split, s.fused ? 1 : 0,
                          s.ws_bytes};
    for (int i = 0; i < 9; ++i) out[i] = v[i];
    return 0;
}

extern "C" int kbn_fp8_gemm_bf16a(const void* x_bf16, int64_t ld_x, float eps, const void* W, int64_t ldw,
                                  const float* sW, int64_t sW_ld, void* D_bf16, int64_t ldd, int64_t M, int64_t N,
                                  int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
    const char* what = "fp8_gemm_bf16a";
    KBN_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
    KBN_CHECK_ARG(M <= 64, "%s: M=%lld; the bf16-activation GEMM covers M <= 64 (quantize, then fp8_gemm_nt)", what,
                  (long long)M);
    KBN_CHECK_ARG(K % kGroup == 0, "%s: K=%lld must be a multiple of 128", what, (long long)K);
    KBN_CHECK_ARG(N <= 0x7FFFFFFFLL && K <= 0x3FFFFFFFLL, "%s: shape too large", what);
    if (M == 0 || N == 0) return 0;
    KBN_CHECK_ARG(K > 0 && x_bf16 && W && sW && D_bf16, "%s: null pointer or empty K", what);
    KBN_CHECK_ARG(ld_x >= K && ldw >= K && ldd >= N, "%s: leading dimension too small", what);
    KBN_CHECK_ARG(aligned16(x_bf16) && ld_x % 8 == 0, "%s: activation rows must be 16-byte aligned", what);
    KBN_CHECK_ARG(aligned16(W) && ldw % 16 == 0, "%s: weight rows must be 16-byte aligned", what);
    KBN_CHECK_ARG(((reinterpret_cast<uintptr_t>(D_bf16) & 1u) == 0), "%s: D must be 2-byte aligned", what);
    KBN_CHECK_ARG(ld_x * 2 * 64 + K * 2 < 0x7FFFFFFFLL && ldw * 256 + K < 0x7FFFFFFFLL && ldd * 2 * 256 < 0x7FFFFFFFLL,
                  "%s: leading dimension too large", what);
    KBN_CHECK_ARG(sW_ld >= K / kGroup, "%s: weight-scale row stride %lld < K/128", what, (long long)sW_ld);
    KBN_CHECK_ARG((N + kGroup - 1) / kGroup * sW_ld * 4 < 0x7FFFFFFFLL, "%s: weight scales span >= 2 GiB", what);
    GemmArgs a{};
    a.X = (const uint16_t*)x_bf16; a.ldx = ld_x; a.eps = eps;
    a.W = (const uint8_t*)W; a.ldw = ldw;
    a.sW = sW; a.sW_ld = sW_ld;
    a.D = (uint16_t*)D_bf16; a.ldd = ldd;
    a.vec_store = (reinterpret_cast<uintptr_t>(D_bf16) % 16 == 0) && (ldd % 8 == 0);
    a.M = (int)M; a.N = (int)N; a.K = (int)K; a.E = 1;
    Schedule sc = bf16a_schedule(M, N, K, workspace != nullptr);
    if (sc.splits > 1) {
        if (workspace_bytes >= sc.ws_bytes) {
            KBN_CHECK_ARG(aligned16(workspace), "%s: workspace must be 16-byte aligned", what);
            a.P = (float*)workspace;
            a.ws_bytes = workspace_bytes;
        } else {
            sc = bf16a_schedule(M, N, K, false);
        }
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // rows of four each wavefront loads and quantizes: just enough for M
    if (sc.bn == 64) {
        KBN_CHECK_ARG(sc.stages == 4, "%s: no %d-stage kernel for 64x64 tiles", what, sc.stages);
        if (sc.fuse_a == 1) return launch_gemm<64, 64, 4, true, false, 4, 1>(a, sc, st, what);
        if (sc.fuse_a == 2) return launch_gemm<64, 64, 4, true, false, 4, 2>(a, sc, st, what);
        return launch_gemm<64, 64, 4, true, false, 4, 4>(a, sc, st, what);
    }
    if (sc.fuse_a == 1) {
        if (sc.stages == 4) return launch_gemm<64, 128, 4, true, false, 4, 1>(a, sc, st, what);
        return launch_gemm<64, 128, 3, true, false, 4, 1>(a, sc, st, what);
    }
    if (sc.fuse_a == 2) {
        if (sc.stages == 4) return launch_gemm<64, 128, 4, true, false, 4, 2>(a, sc, st, what);
        return launch_gemm<64, 128, 3, true, false, 4, 2>(a, sc, st, what);
    }
    if (sc.stages == 4) return launch_gemm<64, 128, 4, true, false, 4, 4>(a, sc, st, what);
    return launch_gemm<64, 128, 3, true, false, 4, 4>(a, sc, st, what);
}

extern "C" int64_t kbn_fp8_gemm_nt_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int kbn_fp8_gemm_nt_noalloc(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                       int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                                       void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0,
                                       void* stream) {
    return gemm_nt_impl("fp8_gemm_nt_noalloc", A, lda, sA, sA_stride_m, sA_stride_k, W, ldw, sW, sW_ld, D_bf16, ldd,
                        M, N, K, scale_ue8m0, nullptr, 0, stream, true);
}

extern "C" int kbn_fp8_grouped_gemm_nt_contiguous(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                                  int64_t sA_stride_k, const void* B, const float* sB, void* C_bf16,
                                                  int64_t ldc, const int32_t* expert_ids, int64_t M_sum, int64_t N,
                                                  int64_t K, int64_t E, int scale_ue8m0, void* stream) {
    const char* what = "m_grouped_fp8_gemm_nt_contiguous";
    if (int rc = check_common(what, A, lda, B, K, C_bf16, ldc, M_sum, N, K)) return rc;
    if (M_sum == 0 || N == 0) return 0;
    KBN_CHECK_ARG(K > 0 && E > 0, "%s: K and E must be positive", what);
    KBN_CHECK_ARG(sA && sB && expert_ids, "%s: null pointer", what);
    KBN_CHECK_ARG(M_sum % 128 == 0, "%s: M_sum=%lld must be a multiple of the 128-row alignment", what,
                  (long long)M_sum);
    const int64_t NB = (N + kGroup - 1) / kGroup, KB = K / kGroup;
    GemmArgs a{};
    a.A = (const uint8_t*)A; a.lda = lda;
    if (int rc = check_scale_ranges(what, M_sum, K, sA_stride_m, sA_stride_k, NB, KB)) return rc;
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
    a.sA_bytes = scale_bytes(M_sum, KB, sA_stride_m, sA_stride_k);
    a.W = (const uint8_t*)B; a.ldw = K; a.w_estride = N * K;
    a.sW = sB; a.sW_ld = KB; a.sW_estride = NB * KB;
    a.D = (uint16_t*)C_bf16; a.ldd = ldc;
    a.vec_store = (reinterpret_cast<uintptr_t>(C_bf16) % 16 == 0) && (ldc % 8 == 0);
    a.expert_ids = expert_ids;
    KBN_CHECK_ARG(E <= 0x7FFFFFFFLL, "%s: too many experts", what);
    a.M = (int)M_sum; a.N = (int)N; a.K = (int)K; a.E = (int)E;
    // Padding rows read as zeros for short K only: at cfg4 the down GEMM
    // (K = 2048) gains, while over gate_up's K = 7168 an expert's nearly
    // empty second row tile runs ahead of its first and the two stop sharing
    // the expert's weight panel in L2.
    a.a_pad_zero = K <= kPadZeroMaxK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Schedule sc;   // grouped: data-parallel, one workgroup per 128-row block x N tile
    if (scale_ue8m0) return launch_gemm<128, 256, 3, true, true>(a, sc, st, what);
    return launch_gemm<128, 256, 3, false, true>(a, sc, st, what);
}

extern "C" int kbn_fp8_grouped_gemm_silu_quant(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                               int64_t sA_stride_k, const void* B, const float* sB,
                                               const int32_t* expert_ids, int64_t M_sum, int64_t N2, int64_t K,
                                               int64_t E, int scale_ue8m0, void* q_fp8, int64_t ldq, float* q_scale,
                                               int64_t qs_stride_m, int64_t qs_stride_g, float eps, int q_ue8m0,
                                               void* stream) {
    const char* what = "grouped_gemm_silu_quant";
    KBN_CHECK_ARG(N2 >= 0 && N2 % 256 == 0, "%s: N2=%lld must be a multiple of 256 ([gate | up], 1x128 groups)",
                  what, (long long)N2);
    if (int rc = check_common(what, A, lda, B, K, q_fp8, ldq, M_sum, N2 / 2, K)) return rc;
    if (M_sum == 0 || N2 == 0) return 0;
    KBN_CHECK_ARG(K > 0 && E > 0, "%s: K and E must be positive", what);
    KBN_CHECK_ARG(sA && sB && expert_ids && q_fp8 && q_scale, "%s: null pointer", what);
    KBN_CHECK_ARG(M_sum % 128 == 0, "%s: M_sum=%lld must be a multiple of the 128-row alignment", what,
                  (long long)M_sum);
    KBN_CHECK_ARG((reinterpret_cast<uintptr_t>(q_fp8) & 7u) == 0 && ldq % 8 == 0,
                  "%s: output rows must be 8-byte aligned", what);
    KBN_CHECK_ARG(qs_stride_m >= 0 && qs_stride_g >= 0 && (reinterpret_cast<uintptr_t>(q_scale) & 3u) == 0,
                  "%s: bad output scale strides or alignment", what);
    KBN_CHECK_ARG(N2 * K < 0x7FFFFFFFLL, "%s: an expert's weights span 2 GiB or more", what);
    const int64_t NB = N2 / kGroup, KB = K / kGroup;
    GemmArgs a{};
    a.A = (const uint8_t*)A; a.lda = lda;
    if (int rc = check_scale_ranges(what, M_sum, K, sA_stride_m, sA_stride_k, NB, KB)) return rc;
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
    a.sA_bytes = scale_bytes(M_sum, KB, sA_stride_m, sA_stride_k);
    a.W = (const uint8_t*)B; a.ldw = K; a.w_estride = N2 * K;
    a.sW = sB; a.sW_ld = KB; a.sW_estride = NB * KB;
    a.D = nullptr; a.ldd = 0;
    a.vec_store = 1;
    a.expert_ids = expert_ids;
    KBN_CHECK_ARG(E <= 0x7FFFFFFFLL, "%s: too many experts", what);
    a.M = (int)M_sum; a.N = (int)N2; a.K = (int)K; a.E = (int)E;
    a.a_pad_zero = K <= kPadZeroMaxK;
    a.glu_half = (int)(N2 / 2);
    a.glu_ue8m0 = q_ue8m0 ? 1 : 0;
    a.glu_eps = eps;
    a.q2 = static_cast<uint8_t*>(q_fp8); a.ldq2 = ldq;
    a.s2 = q_scale; a.s2_sm = qs_stride_m; a.s2_sg = qs_stride_g;
    a.silu_lut = silu_lut_device(what);
    if (!a.silu_lut) return 1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Schedule sc;
    if (scale_ue8m0) return launch_gemm<128, 256, 3, true, true, 4, 0, false, true>(a, sc, st, what);
    return launch_gemm<128, 256, 3, false, true, 4, 0, false, true>(a, sc, st, what);
}

extern "C" int64_t kbn_fp8_fused_moe_gemm_workspace_bytes(int64_t EM, int64_t K) {
    if (EM < 0 || K <= 0 || K % kGroup != 0 || EM > 0x7FFFFFFFLL) return -1;
    return EM * (K / kGroup) * 4;
}

extern "C" int kbn_fp8_fused_moe_gemm(const void* A, int64_t lda, int64_t rows_A, const float* sA, int64_t sA_stride_m,
                                      int64_t sA_stride_k, const void* B, const float* sB, void* C_bf16, int64_t ldc,
                                      const int32_t* sorted_token_ids, const int32_t* expert_ids,
                                      const int32_t* num_tokens_post_padded, int64_t EM, int64_t block_m,
                                      int64_t num_valid, int64_t top_k, const float* topk_weights, int64_t N,
                                      int64_t K, int64_t E, void* workspace, int64_t workspace_bytes, void* stream) {
    const char* what = "fused_moe_gemm";
    KBN_CHECK_ARG(rows_A >= 0 && N >= 0 && K > 0 && E > 0 && EM >= 0 && num_valid >= 0 && top_k >= 1,
                  "%s: bad shape", what);
    KBN_CHECK_ARG(K % kGroup == 0, "%s: K=%lld must be a multiple of 128", what, (long long)K);
    KBN_CHECK_ARG(block_m >= 64 && block_m % 64 == 0, "%s: block_m=%lld must be a multiple of 64", what,
                  (long long)block_m);
    if (EM == 0 || N == 0 || num_valid == 0) return 0;
    KBN_CHECK_ARG(A && sA && B && sB && C_bf16 && expert_ids && num_tokens_post_padded, "%s: null pointer", what);
    KBN_CHECK_ARG((num_valid - 1) / top_k < rows_A, "%s: %lld pairs over top_k %lld need %lld A rows, got %lld", what,
                  (long long)num_valid, (long long)top_k, (long long)((num_valid - 1) / top_k + 1), (long long)rows_A);
    KBN_CHECK_ARG(lda >= K && lda % 16 == 0 && aligned16(A) && aligned16(B), "%s: A and B rows must be 16-byte aligned",
                  what);
    KBN_CHECK_ARG(ldc >= N && ((reinterpret_cast<uintptr_t>(C_bf16) & 1u) == 0), "%s: bad C", what);
    // gathered rows and scattered stores use 32-bit byte offsets
    KBN_CHECK_ARG(rows_A * lda < 0x7FFFFFFFLL && num_valid * ldc * 2 < 0x7FFFFFFFLL && EM <= 0x7FFFFFFFLL &&
                      N <= 0x7FFFFFFFLL && K <= 0x7FFFFFFFLL && E <= 0x7FFFFFFFLL && num_valid <= 0x7FFFFFFFLL,
                  "%s: operands span >= 2 GiB", what);
    const int64_t NB = (N + kGroup - 1) / kGroup, KB = K / kGroup;
    if (int rc = check_scale_ranges(what, rows_A, K, sA_stride_m, sA_stride_k, NB, KB)) return rc;
    GemmArgs a{};
    a.A = (const uint8_t*)A; a.lda = lda; a.A_bytes = rows_A * lda;
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
    a.sA_bytes = scale_bytes(rows_A, KB, sA_stride_m, sA_stride_k);
    a.W = (const uint8_t*)B; a.ldw = K; a.w_estride = N * K;
    a.sW = sB; a.sW_ld = KB; a.sW_estride = NB * KB;
    a.D = (uint16_t*)C_bf16; a.ldd = ldc; a.D_bytes = (num_valid - 1) * ldc * 2 + N * 2;
    a.vec_store = (reinterpret_cast<uintptr_t>(C_bf16) % 16 == 0) && (ldc % 8 == 0);
    a.expert_ids = expert_ids;
    a.sorted_ids = sorted_token_ids;
    a.num_post_pad = num_tokens_post_padded;
    a.block_m = (int)block_m;
    a.num_valid = (int)num_valid;
    a.a_row_div = (int)top_k;
    a.row_weight = topk_weights;
    a.M = (int)EM; a.N = (int)N; a.K = (int)K; a.E = (int)E;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (workspace) {
        // gather the scales into sorted order first; the GEMM then reads them
        // like the contiguous layout's
        const int64_t need = EM * KB * 4;
        KBN_CHECK_ARG(workspace_bytes >= need && aligned16(workspace) && need < 0x7FFFFFFFLL,
                      "%s: workspace of %lld bytes (16-byte aligned) needed, got %lld", what, (long long)need,
                      (long long)workspace_bytes);
        const int64_t threads = EM * KB;
        sorted_scale_gather_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st>>>(
            a, static_cast<float*>(workspace), (int)KB);
        KBN_CHECK_LAUNCH(what);
        a.sA = static_cast<const float*>(workspace);
        a.sA_sm = 1;
        a.sA_sk = EM;
        a.sA_bytes = need;
        a.sa_sorted = 1;
    }
    // the scales are taken as given (fp32 contract), as the reference's
    // per-block promotion does
    if (block_m % 128 == 0) return launch_sorted<128, 256, 3>(a, st, what);
    return launch_sorted<64, 256, 3>(a, st, what);
}
