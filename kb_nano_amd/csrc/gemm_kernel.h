// Block-scaled FP8 GEMM  D[M,N] (bf16) = A[M,K] (e4m3) x W[N,K]^T (e4m3)
// with one fp32 scale per (row, 128-K block) of A and per (128-N, 128-K)
// block of W, plus the contiguous-layout grouped (MoE) variant.
//
// Contract (tasks/baseline/L1/fp8_linear.py:97-110 -> deep_gemm.fp8_gemm_nt,
// tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:109-118):
//   D[m,n] = bf16_rne( sum_kb sA[m,kb] * sW[n/128,kb] * sum_{k in kb} A[m,k] W[n,k] )
// accumulated in fp32.
//
// Two scale contracts:
//  * UE8M0 (the default, DeepGEMM's UE8M0 cast): every scale is rounded up to
//    a power of two and applied inside the block-scaled MFMA
//    (v_mfma_scale_f32_32x32x64_f8f6f4) as an E8M0 operand, so one fp32
//    accumulator set runs across all of K with no promotion epilogue.
//  * FP32 (disable_ue8m0_cast): scales are used as given.  Each scale splits
//    exactly into a power of two, applied by the MFMA as above, and a
//    significand in [1, 2).  The accumulators hold the running sum in units
//    of the current block's significand product (per row) and are rescaled
//    by the ratio of consecutive products when a block starts; the last
//    product multiplies the sum before the store.  Power-of-two scales give
//    ratios of 1 and skip the rescale, so such scales cost what UE8M0 does.
//
// Dataflow per workgroup (256 lanes = 4 wavefronts, one per SIMD):
//   HBM --buffer_load_dwordx4 ... lds (direct DMA)--> LDS (kStages x (BM+BN) x 128 B)
//   LDS --ds_read_b128--> VGPR fragments --MFMA 32x32x64--> fp32 accumulators
// Each LDS row is 128 B (one 128-K scale block); its eight 16-B chunks are
// XOR-swizzled so the rows read by one ds_read_b128 hit distinct banks.  The
// swizzle is applied on the global side of the DMA (lane i of a load
// instruction always writes LDS chunk i), so no extra LDS pass is needed.
// Out-of-range rows read as zero through the buffer descriptor's range check.

#pragma once

#include "kbn_common.h"

#include <algorithm>

namespace kbn {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));


// FP32 scale contract: s = 2^(byte - 127) * mant with byte the biased
// exponent field (the block-scaled MFMA's E8M0 operand, exact) and mant the
// significand in [1, 2).  Zero and subnormal scales get byte 0 (2^-127), so
// their block adds at most 2^-127 of the value it would have at scale 1;
// inf/NaN scales get 255, the E8M0 NaN.
__device__ __forceinline__ int scale_exp_byte(float s) { return (int)((__float_as_uint(s) >> 23) & 0xFFu); }
__device__ __forceinline__ float scale_mant(float s) {
    return __uint_as_float((__float_as_uint(s) & 0x007FFFFFu) | 0x3F800000u);
}

struct GemmArgs {
    const uint8_t* A;
    int64_t lda;
    const float* sA;
    int64_t sA_sm, sA_sk;
    int64_t sA_bytes;            // byte range of the scale buffer the kernel may read
    const uint8_t* W;            // [N, K] (dense) or [E, N, K] (grouped)
    int64_t ldw;
    int64_t w_estride;           // bytes between experts (grouped)
    const float* sW;             // [ceil(N/128), KB] (+ expert stride)
    int64_t sW_ld;
    int64_t sW_estride;
    uint16_t* D;
    int64_t ldd;
    const int32_t* expert_ids;   // grouped only
    int M, N, K, E;
    int tiles_m, tiles_n;
    int group_m;                 // MoE layouts: row tiles per column group (moe_group_m)
    int vec_store;               // D rows allow aligned 16-B stores
    // This launch covers tiles [tile_base, tile_base + tile_count) of the
    // grouped tile order.  Split-K: workgroup (tile, split) accumulates K
    // blocks [split * kb_per_split, +kb_per_split) into the fp32 slab
    // P[split][tile - tile_base][BM][BN], summed by splitk_reduce_kernel.
    int tile_base, tile_count;
    float* P;
    int64_t ws_bytes;            // bytes at P
    int splits, kb_per_split;
    // Arrival counters of the split launch, one per tile (nullptr: a separate
    // splitk_reduce_kernel launch sums the slabs).  Zero on entry; the last
    // workgroup of a tile to finish sums the slabs and resets its counter.
    unsigned* flags;
    // Sorted-token layout (fused MoE): row R of the tile grid holds routed pair
    // sorted_ids[R] (or, with no list, pair R / block_m on the first row of
    // each block and nothing elsewhere); a pair t >= num_valid is padding.
    // A row of pair t: t / a_row_div.  Output row: t.  Expert of block b:
    // expert_ids[b], blocks at or past *num_post_pad are skipped.
    const int32_t* sorted_ids;
    const int32_t* num_post_pad;
    int block_m, num_valid, a_row_div;
    int64_t A_bytes;             // bytes at A the gathers may read
    int64_t D_bytes;             // bytes at D the scattered stores may write
    const float* row_weight;     // [num_valid] fp32 factors of the output rows, or nullptr
    int sa_sorted;               // sA already holds row R's scales at R (gathered by sorted_scale_gather_kernel)
    // Grouped: A rows of a tile that belong to no expert or another one (the
    // layout's padding) are read as zeros instead of fetched.
    int a_pad_zero;
    // bf16 activations quantized by the kernel itself (1x128 groups, UE8M0):
    // X [M, K] with row stride ldx elements, group absmax floor eps.
    const uint16_t* X;
    int64_t ldx;
    float eps;
    // Packed per-row UE8M0 weight scales (DeepGEMM's int32 layout): word
    // (n, i) at sWp[n * sWp_sn + i * sWp_sk] holds the E8M0 exponents of
    // weight row n for K blocks 4i .. 4i + 3, byte j for block 4i + j.
    const int32_t* sWp;
    int64_t sWp_sn, sWp_sk;
    int64_t sWp_bytes;
    // Grouped gate/up GEMM with SiLU*Mul + 1x128 quant in its epilogue
    // (kGlu): W rows [0, glu_half) are the gate, [glu_half, 2 glu_half) the
    // up rows; tile column block t covers gate columns [128 t, 128 t + 128)
    // and the same up columns.  Row r's y = bf16(silu(bf16 gate) * bf16 up)
    // leaves as fp8 codes q2[r, 128 t + j] with scale s2[r * s2_sm + t * s2_sg].
    int glu_half, glu_ue8m0;
    float glu_eps;
    uint8_t* q2;
    int64_t ldq2;
    float* s2;
    int64_t s2_sm, s2_sg;
    const uint16_t* silu_lut;    // device address of the bf16 SiLU table
};

// Raw buffer descriptor (base, byte range) built from uniform values so it
// lives in SGPRs.  Loads past `bytes` return zero.
__device__ __forceinline__ v4i make_desc(const void* base, int64_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    const uint32_t n = bytes <= 0 ? 0u : (bytes >= 0xFFFFFFFFLL ? 0xFFFFFFFFu : (uint32_t)bytes);
    v4i r;
    r[0] = (int)(uint32_t)p;
    r[1] = (int)((p >> 32) & 0xFFFFu);
    r[2] = (int)n;
    r[3] = (int)kRsrcWord3;
    return r;
}

// Direct global->LDS DMA.  Issued as inline asm so the compiler's waitcnt
// pass does not serialise every LDS read behind the in-flight DMA of the
// other stage; completion is awaited explicitly (wait_dma) before the
// barrier that publishes a stage.  Lane i writes LDS bytes
// [lds + 16*i, lds + 16*i + 16) (dwordx4) or [lds + 4*i, lds + 4*i + 4) (dword).
__device__ __forceinline__ void dma_b128(const v4i& desc, uint32_t lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(desc)
                 : "memory");
}
// The same load with the non-temporal hint: the weight rows of a tile are
// read once per workgroup and should not push the activation rows (read by
// every workgroup of a tile row) out of L2.
__device__ __forceinline__ void dma_b128_nt(const v4i& desc, uint32_t lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(lds), "v"(voff), "s"(desc)
                 : "memory");
}
__device__ __forceinline__ void dma_b32(const v4i& desc, uint32_t lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(desc)
                 : "memory");
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N vector-memory loads of this wavefront are outstanding
// (loads complete in issue order, so everything older than the last N has landed).
template <int N>
__device__ __forceinline__ void wait_dma_n() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }


// LDS row layout.  A stage holds one 128-K scale block per row (128 B =
// eight 16-B chunks); chunk c of row r lives in slot c ^ swz(r).  A
// ds_read_b128 is served 16 lanes (256 B, all 64 banks) per cycle; the 16
// consecutive rows read by 16 lanes alternate between the two halves of a
// 256-B bank line (r % 2) and take 8 distinct slots per half (r >> 1), so
// fragment reads are conflict-free.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

constexpr int kRowB = 128;   // LDS row bytes = K per stage = one scale block

// XCD-aware tile order.  Consecutive workgroup ids are dispatched round-robin
// over the 8 XCDs; give each XCD a contiguous range of the (tile, split)
// sequence so the tiles resident on one XCD (and its L2) share A row panels
// and W panels, and walk that sequence in column groups of kGroupM row tiles
// (the K splits of one tile are neighbours).
template <int kGroupM>
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int tile_base, int splits, int& tm, int& tn,
                                            int& trel, int& split) {
    const int nblk = gridDim.x;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, i = bid >> 3;
    const int per = nblk >> 3, rem = nblk & 7;
    const int ts = xcd * per + (xcd < rem ? xcd : rem) + i;
    trel = ts / splits;
    split = ts - trel * splits;
    const int t = tile_base + trel;
    const int group = kGroupM * tiles_n;
    const int g = t / group;
    const int first_m = g * kGroupM;
    const int gm = min(tiles_m - first_m, kGroupM);
    const int w = t - g * group;
    tm = first_m + w % gm;
    tn = w / gm;
}

// Tile order of the MoE layouts.  Their padded row grid ends in row tiles no
// expert owns (those workgroups exit at once), so contiguous per-XCD ranges
// would give the last XCDs nothing but empty tiles (cfg4: two of eight idle).
// The tile sequence (column groups of group_m row tiles, as tile_coords) is
// split in two parts:
//   - as many whole column groups as make full rounds of eight are dealt to
//     the XCDs round-robin: XCD x runs groups x, x + 8, x + 16, ... in order;
//   - the rest (fewer than eight groups) is cut into eight contiguous ranges.
// Every XCD then gets the same number of tiles, the empty tail is shared out
// with the rest, and an expert's row tiles still meet its weight panel in one
// L2.  The grid has moe_dealt_grid slots; a slot past an XCD's share returns
// false.
__device__ __forceinline__ bool tile_coords_dealt(int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int bid = blockIdx.x;
    const int xcd = bid & 7, i = bid >> 3;
    const int total = tiles_m * tiles_n;
    const int group = group_m * tiles_n;
    const int rounds = total / group / 8;          // dealt groups per XCD
    const int dealt = rounds * group;              // dealt tiles per XCD
    int t;
    if (i < dealt) {
        const int j = i / group;
        t = (xcd + 8 * j) * group + (i - j * group);
    } else {
        const int rest = total - 8 * dealt, per = rest >> 3, rem = rest & 7;
        const int r = i - dealt;
        if (r >= per + (xcd < rem ? 1 : 0)) return false;
        t = 8 * dealt + xcd * per + min(xcd, rem) + r;
    }
    const int g = t / group;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int w = t - g * group;
    tm = first_m + w % gm;
    tn = w / gm;
    return true;
}
// Row tiles per column group.  An XCD runs 32 tiles at once, i.e. 32 /
// group_m columns of the group, and an activation panel is fetched again for
// each such set of columns; smaller groups cut those fetches but cut more
// experts' row tiles apart, so more weight panels are fetched twice.  At cfg4
// (UE8M0, HIP events; HBM fetch per call) gate_up (K = 7168) took 1718 us
// with 16 (10.65 GB), 1658 with 8 (9.44 GB), 1674 with 4 (9.05 GB) and 1772
// with 2 (9.57 GB); down (K = 2048) 940 / 943 / 954 / 988 us.
static inline int moe_group_m(int64_t K) { return K >= 4096 ? 8 : 16; }
// Workgroups of a dealt launch over tiles_m x tiles_n tiles.
static inline int64_t moe_dealt_grid(int64_t tiles_m, int64_t tiles_n, int64_t group_m) {
    const int64_t total = tiles_m * tiles_n;
    if (total <= 0) return 0;
    const int64_t group = group_m * tiles_n;
    const int64_t dealt = total / group / 8 * group;
    return 8 * (dealt + (total - 8 * dealt + 7) / 8);
}


__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const bf16x2 p = __builtin_convertvector((f32x2{lo, hi}), bf16x2);  // v_cvt_pk_bf16_f32, RNE
    return __builtin_bit_cast(uint32_t, p);
}
// Cache-policy operand of the split-K slab stores and loads: the SC1 bit,
// which the compiler emits for agent-scope relaxed atomic accesses.  Such an
// access is coherent across the XCDs' L2s, and a store is visible device-wide
// once it has completed (vmcnt), so a slab written this way needs no L2
// write-back before its arrival is counted.
constexpr int kDeviceCoherent = 16;

// Split-K sum of rows r0, r0 + r_step, ... (< r_end, at most kPass of them)
// of one tile's slabs: D = bf16(((s_0 + s_1) + s_2) + ...), in split order,
// one float4 run of columns per lane (c = the run's first column within the
// tile).  Every row's loads of one split are issued together (two splits per
// step), so a workgroup that sums a whole tile keeps kPass x 2 loads in
// flight instead of walking its rows one dependent pass at a time.
template <int BM, int BN, int kAux, int kPass>
__device__ __forceinline__ void splitk_sum_rows(const GemmArgs& a, int trel, int m0, int n0, int r0, int r_end,
                                                int r_step, int c) {
    const int slab = a.tile_count * BM * BN * 4;   // bytes between splits (the workspace is below 2 GiB)
    const __amdgpu_buffer_rsrc_t dP = __builtin_amdgcn_make_buffer_rsrc(
        a.P + (int64_t)trel * BM * BN, (short)0, (int)((a.splits - 1) * slab + BM * BN * 4), (int)kRsrcWord3);
    auto ld = [&](int off) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(dP, off, 0, kAux));
    };
    int off[kPass];
    float4 acc[kPass];
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
        const int r = r0 + p * r_step;
        off[p] = r < r_end ? (r * BN + c) * 4 : kOob;   // rows past the tile's last read zeros, never stored
        acc[p] = ld(off[p]);
    }
    int sp = 1;
    for (; sp + 1 < a.splits; sp += 2) {
        float4 v0[kPass], v1[kPass];
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            v0[p] = ld(off[p] == kOob ? kOob : off[p] + sp * slab);
            v1[p] = ld(off[p] == kOob ? kOob : off[p] + (sp + 1) * slab);
        }
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            acc[p].x = (acc[p].x + v0[p].x) + v1[p].x;
            acc[p].y = (acc[p].y + v0[p].y) + v1[p].y;
            acc[p].z = (acc[p].z + v0[p].z) + v1[p].z;
            acc[p].w = (acc[p].w + v0[p].w) + v1[p].w;
        }
    }
    if (sp < a.splits) {
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            const float4 v = ld(off[p] == kOob ? kOob : off[p] + sp * slab);
            acc[p].x += v.x;
            acc[p].y += v.y;
            acc[p].z += v.z;
            acc[p].w += v.w;
        }
    }
    const int n = n0 + c;
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
        if (off[p] == kOob) continue;
        uint16_t* d = a.D + (int64_t)(m0 + r0 + p * r_step) * a.ldd + n;
        const uint32_t lo = pack_bf16(acc[p].x, acc[p].y), hi = pack_bf16(acc[p].z, acc[p].w);
        if (a.vec_store && n + 3 < a.N) {
            *reinterpret_cast<uint2*>(d) = make_uint2(lo, hi);
        } else {
            if (n < a.N) d[0] = (uint16_t)lo;
            if (n + 1 < a.N) d[1] = (uint16_t)(lo >> 16);
            if (n + 2 < a.N) d[2] = (uint16_t)hi;
            if (n + 3 < a.N) d[3] = (uint16_t)(hi >> 16);
        }
    }
}

// LDS bytes of a tile configuration of four wavefronts: a stage holds BM A
// rows of 128 fp8 bytes, or, when the kernel quantizes bf16 activations
// itself (fuse_a = rows of four per wavefront, 1, 2 or 4), 16 fuse_a bf16
// rows of 256 bytes; configurations that fit twice into a CU's 160 KB run
// two workgroups per CU.
constexpr int gemm_a_stage_bytes(int bm, int fuse_a) { return fuse_a ? 16 * fuse_a * 2 * kRowB : bm * kRowB; }
constexpr int gemm_lds_bytes(int bm, int bn, int stages, int fuse_a = 0) {
    return stages * (gemm_a_stage_bytes(bm, fuse_a) + bn * kRowB + 2048);
}
constexpr int gemm_occupancy(int bm, int bn, int stages, int fuse_a = 0) {
    return gemm_lds_bytes(bm, bn, stages, fuse_a) <= 80 * 1024 ? 2 : 1;
}

// Block-scaled GEMM tile kernel: BM x BN output tile, four wavefronts in a
// 2 x 2 grid, each owning a (BM/2) x (BN/2) block of 32x32 MFMA fragments.
//
// LDS stage layout (one stage = one 128-K block):
//   [A: BM x 128 B][W: BN x 128 B][sA: 4 x 64 fp32][sW: 4 x 64 fp32]
// Every load is a 16-B (or 4-B) direct global->LDS DMA; one A/W instruction
// moves eight full 128-B rows, so every request the vector cache sends to L2
// is a whole 128-B line.
//
// Pipeline over K blocks kb (LDS buffer kb % kStages), per wavefront:
//   sub-step 0: MFMAs of K half 0 of block kb, interleaved with the LDS reads
//               of K half 1 of block kb;
//   hand-off:   wait until block kb+1 has landed and this wavefront's reads of
//               block kb are done; barrier (publishes kb+1, frees buffer kb);
//               DMA block kb+kStages into the freed buffer;
//   sub-step 1: MFMAs of K half 1 of block kb, interleaved with the LDS reads
//               of K half 0 (and the scales) of block kb+1.
// So kStages-1 blocks are in flight while one is consumed, and no fragment
// register set is ever copied.
//
// kFuseA (1, 2 or 4; 0 = off): A arrives as bf16 (a.X) and is quantized
// by the kernel, 1x128 groups with UE8M0 scales exactly as the quant kernel
// does it (quant.hip), so the product equals quant + GEMM bit for bit.  A
// stage then holds 16 kFuseA bf16 A rows of 256 B (the caller keeps
// M <= 16 kFuseA; the tile's rows past those are never loaded, and what the
// MFMAs make of them is never stored).  Tile row r sits at LDS row
// p(r) = (r % 4) 4 kFuseA + r / 4 (wavefront w's DMAs bring rows w, w + 4,
// w + 8, ... into LDS rows 4 kFuseA w, +1, ...), and its 16-B chunk c in slot
// c ^ (r & 15), so 16 consecutive tile rows read conflict-free.  Each
// wavefront quantizes the 4 kFuseA rows its own DMAs brought, in place,
// with 16 / kFuseA lanes per row.
template <int BM, int BN, int kStages, bool kUe8m0, bool kGrouped, bool kSplitK, int kWaves, bool kSorted = false,
          int kFuseA = 0, bool kRowW = false, bool kGlu = false>
__global__ __launch_bounds__(64 * kWaves, (kStages * (gemm_a_stage_bytes(BM, kFuseA) + BN * 128) +
                                               kStages * 512 * kWaves <=
                                           80 * 1024)
                                              ? 2
                                              : 1) void
gemm_bs_kernel(const GemmArgs a) {
    static_assert(!(kSorted && (kGrouped || kSplitK)), "the sorted-token layout is its own grouped mode");
    static_assert(!kFuseA || (kUe8m0 && !kGrouped && !kSorted && BM == 64 && kWaves == 4 &&
                              (kFuseA == 1 || kFuseA == 2 || kFuseA == 4)),
                  "in-kernel activation quant: UE8M0, dense, 64-row tiles of four wavefronts, 16/32/64 rows");
    static_assert(kWaves == 4 || kWaves == 8, "2x2 or 2x4 wavefronts");
    static_assert(!kGlu || (kGrouped && BM == 128 && BN == 256 && kWaves == 4),
                  "SiLU*Mul epilogue: the grouped 128x256 tiles (128 gate + 128 up columns, two per wavefront row)");
    static_assert(!kRowW || (kUe8m0 && !kGrouped && !kSorted && !kFuseA && BN <= 64 * kWaves),
                  "packed per-row weight scales: dense UE8M0 tiles, one scale word per tile row and lane");
    constexpr int WM = 2, WN = kWaves / 2;
    constexpr int TM = BM / WM, TN = BN / WN;   // wavefront tile
    constexpr int FM = TM / 32, FN = TN / 32;   // 32x32 fragments per wavefront
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "fragment tiling");
    static_assert(BM <= 64 * kWaves && BM % (16 * kWaves) == 0 && BN % (16 * kWaves) == 0, "DMA tiling");
    // A wave N tile that does not divide (or is not a multiple of) a 128-row
    // weight-scale block (the 96 columns of a 256x192 tile) takes one W scale
    // per 32-column fragment instead of one per wavefront.
    constexpr bool kFragW = !kRowW && 128 % TN != 0 && TN % 128 != 0;
    constexpr bool kPerFragW = kRowW || kFragW;
    static_assert(!kFragW || (kUe8m0 && TN % 32 == 0), "per-fragment weight scales: UE8M0 contract");
    constexpr int kArow = kFuseA ? 2 * kRowB : kRowB;   // LDS bytes of one A row of a stage
    constexpr int kA = gemm_a_stage_bytes(BM, kFuseA), kB = BN * kRowB, kSA = kWaves * 256, kSW = kWaves * 256;
    constexpr int kAW = 4 * (kFuseA ? kFuseA : 1);     // fused A: LDS rows per wavefront
    constexpr int kStage = kA + kB + kSA + kSW;
    static_assert(kStages >= 2 && kStages * kStage <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStage];
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)smem);

    static_assert(!kGrouped || BM == 128, "grouped tiles cover one 128-row block of the contiguous layout");

    int tm, tn, trel = 0, split = 0;
    // MoE tiles walk column groups of a.group_m row tiles dealt over the
    // XCDs (tile_coords_dealt), so an expert's row tiles meet its weight panel
    // in one L2; dense tiles walk groups of 4 row tiles, which the split
    // reduction's tile order also assumes
    if constexpr (kGrouped || kSorted) {
        static_assert(!kSplitK, "MoE layouts run data-parallel");
        if (!tile_coords_dealt(a.tiles_m, a.tiles_n, a.group_m, tm, tn)) return;
    } else {
        tile_coords<4>(a.tiles_m, a.tiles_n, a.tile_base, kSplitK ? a.splits : 1, tm, tn, trel, split);
    }
    const int m0 = tm * BM, n0 = tn * (kGlu ? BN / 2 : BN);   // kGlu: the first gate column
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    // K blocks of this workgroup: [kb0, kb0 + KB)
    const int kb0 = kSplitK ? split * a.kb_per_split : 0;
    const int KB = kSplitK ? min(a.K / kRowB - kb0, a.kb_per_split) : a.K / kRowB;
    const int NB = (a.N + kGroup - 1) / kGroup;

    const uint8_t* Wbase = a.W;
    const float* sWbase = a.sW;
    int expert = 0;
    if constexpr (kGrouped) {
        expert = a.expert_ids[m0];
        if (expert < 0 || expert >= a.E) return;  // padding block: C rows stay unwritten
        Wbase += (int64_t)expert * a.w_estride;
        sWbase += (int64_t)expert * a.sW_estride;
    }
    if constexpr (kSorted) {
        // a tile lies inside one block of block_m rows (BM divides block_m)
        if (m0 >= a.num_post_pad[0]) return;
        expert = a.expert_ids[m0 / a.block_m];
        if (expert < 0 || expert >= a.E) return;
        Wbase += (int64_t)expert * a.w_estride;
        sWbase += (int64_t)expert * a.sW_estride;
    }
    // routed pair of tile row r, or -1 for padding
    auto pair_of = [&](int r) -> int {
        const int R = m0 + r;
        if (R >= a.M) return -1;
        const int t = a.sorted_ids ? a.sorted_ids[R] : (R % a.block_m == 0 ? R / a.block_m : -1);
        return (t >= 0 && t < a.num_valid) ? t : -1;
    };

    const v4i dA = kFuseA  ? make_desc(a.X + (int64_t)m0 * a.ldx, ((int64_t)(a.M - m0 - 1) * a.ldx + a.K) * 2)
                   : kSorted ? make_desc(a.A, a.A_bytes)
                             : make_desc(a.A + (int64_t)m0 * a.lda, (int64_t)(a.M - m0 - 1) * a.lda + a.K);
    const v4i dW = make_desc(Wbase + (int64_t)n0 * a.ldw, (int64_t)(a.N - n0 - 1) * a.ldw + a.K);
    const v4i dSA = make_desc(a.sA, a.sA_bytes);
    const v4i dSW = kRowW ? make_desc(a.sWp, a.sWp_bytes) : make_desc(sWbase, (int64_t)NB * a.sW_ld * 4);

    // DMA lane mapping: one instruction = 8 rows x 128 B starting at row
    // r0 = 8 q; lane i fills slot i % 8 of row r0 + i / 8 with global chunk
    // (i % 8) ^ swz(r0 + i / 8) = (i % 8) ^ ((i >> 4) | 4 (q & 1)).
    // fused bf16 A: kFuseA 4-row DMAs (16 lanes x 16 B per row) per wave
    constexpr int kAInstr = kFuseA ? kFuseA : BM / (8 * kWaves);
    constexpr int kBInstr = BN / (8 * kWaves);   // 8-row DMAs per wave
    static_assert((kFuseA || kAInstr % 2 == 0) && kBInstr % 2 == 0, "even instruction counts keep q & 1 == i & 1");
    const int drow = lane >> 3;
    const int ch_e = ((lane & 7) ^ (lane >> 4)) << 4;
    const int ch_o = ((lane & 7) ^ ((lane >> 4) | 4)) << 4;
    const int a_e = (int)((wave * kAInstr * 8 + drow) * a.lda) + ch_e + kb0 * kRowB;
    const int a_o = a_e - ch_e + ch_o;
    // kGlu: the tile's W rows 128..255 (wavefronts 2 and 3) are the up rows,
    // glu_half - 128 rows further on than the tile's row index says
    const int glu_w = kGlu && wave * kBInstr * 8 >= BN / 2 ? (a.glu_half - BN / 2) * (int)a.ldw : 0;
    const int w_e = (int)((wave * kBInstr * 8 + drow) * a.ldw) + ch_e + kb0 * kRowB + glu_w;
    const int w_o = w_e - ch_e + ch_o;
    // fused A: instruction i of wavefront w fills LDS rows 4 kFuseA w + 4 i + lane / 16
    // with tile row r = w + 16 i + 4 (lane / 16); slot lane % 16 <- global chunk
    // slot ^ (r & 15); this lane's byte offset of its chunk in X
    int xa_off[kFuseA ? kAInstr : 1];
    if constexpr (kFuseA) {
#pragma unroll
        for (int i = 0; i < kAInstr; ++i) {
            const int row = wave + 16 * i + 4 * (lane >> 4);
            xa_off[i] = row * (int)(a.ldx * 2) + (((lane & 15) ^ (row & 15)) << 4) + kb0 * 2 * kRowB;
        }
    }
    // grouped with a.a_pad_zero: bit i set when the row of this lane's A
    // instruction i is not one of the tile expert's rows (its DMA reads zeros;
    // those rows are never stored)
    uint32_t a_dead = 0;
    if constexpr (kGrouped) {
        if (a.a_pad_zero) {
#pragma unroll
            for (int i = 0; i < kAInstr; ++i) {
                const int r = m0 + wave * kAInstr * 8 + i * 8 + drow;
                if (r >= a.M || a.expert_ids[r] != expert) a_dead |= 1u << i;
            }
        }
    }
    // sorted layout: byte offset of each DMA row of this lane's A instructions
    // (gathered rows; padding reads zeros)
    int a_row[kSorted ? kAInstr : 1];
    if constexpr (kSorted) {
#pragma unroll
        for (int i = 0; i < kAInstr; ++i) {
            const int t = pair_of(wave * kAInstr * 8 + i * 8 + drow);
            a_row[i] = t >= 0 ? (t / a.a_row_div) * (int)a.lda + kb0 * kRowB : kOob;
        }
    }
    const int sa_row = wave * 64 + lane;
    int sa_src = -1;    // activation-scale row of this lane's tile row
    if (sa_row < BM) {
        if constexpr (kSorted) {
            const int t = pair_of(sa_row);
            sa_src = t < 0 ? -1 : a.sa_sorted ? m0 + sa_row : t / a.a_row_div;
        } else {
            sa_src = m0 + sa_row < a.M ? m0 + sa_row : -1;
        }
    }
    const bool sa_live = sa_src >= 0;
    const int sa_kstep = sa_live ? (int)(a.sA_sk * 4) : 0;
    const int sa_off0 = sa_live ? (int)((int64_t)sa_src * a.sA_sm * 4) + kb0 * sa_kstep : kOob;
    // W scales of a stage: the tile's 128-row block scales (lane < BN / 128),
    // or with kRowW one packed word per tile row (row wave * 64 + lane): its
    // four K blocks' exponents, word (kb / 4) of the row
    int sw_kstep, sw_off0;
    if constexpr (kRowW) {
        const int r = wave * 64 + lane;
        const bool live = r < BN && n0 + r < a.N;
        sw_kstep = live ? (int)(a.sWp_sk * 4) : 0;
        sw_off0 = live ? (int)((int64_t)(n0 + r) * a.sWp_sn * 4) : kOob;
    } else {
        // the scale blocks the tile's rows touch (a 192-row tile may start mid-block)
        const bool sw_live = kGlu ? lane < 2 : (lane < (((n0 & 127) + BN + 127) >> 7)) & (n0 / 128 + lane < NB);
        sw_kstep = sw_live ? 4 : 0;
        // kGlu: the gate block, then the up block
        const int sw_blk = kGlu ? (lane == 0 ? n0 : a.glu_half + n0) / 128 : n0 / 128 + lane;
        sw_off0 = sw_live ? sw_blk * (int)a.sW_ld * 4 + kb0 * 4 : kOob;
    }
    constexpr int kScaleDma = kFuseA ? 1 : 2;    // scale vectors per stage (no A scales when fused)
    constexpr int kDma = kAInstr + kBInstr + kScaleDma;  // DMA instructions per wave per stage
    // Weight rows stream past L2 (non-temporal) where the weights dominate the
    // traffic: the 128-column dense tiles (chosen only for M <= 128) and the
    // grouped and sorted MoE tiles.  The large dense tiles keep the default,
    // which measures faster where A and W tiles are both re-read from L2.
    constexpr bool kWeightNt = (BN == 128) || kGrouped || kSorted;

    // DMA instruction d (0 <= d < kDma) of K block s -> LDS buffer s % kStages:
    // the two scale vectors, then the A rows, then the W rows.  `live` false
    // turns the load into an out-of-range (zero) read, so the loop never
    // branches around it and every stage issues the same number of loads.
    auto issue_one = [&](int s, bool live, int d) {
        const uint32_t base = lds0 + (s % kStages) * kStage;
        const int k0 = s * kRowB;
        if (!kFuseA && d == 0) {
            dma_b32(dSA, base + kA + kB + wave * 256, live ? sa_off0 + s * sa_kstep : kOob);
        } else if (d == kScaleDma - 1) {
            if constexpr (kRowW)
                dma_b32(dSW, base + kA + kB + kSA + wave * 256, live ? sw_off0 + ((kb0 + s) >> 2) * sw_kstep : kOob);
            else
                dma_b32(dSW, base + kA + kB + kSA + wave * 256, live ? sw_off0 + s * sw_kstep : kOob);
        } else if (d < kScaleDma + kAInstr) {
            const int i = d - kScaleDma;
            int off;
            if constexpr (kFuseA) off = xa_off[i] + s * 2 * kRowB;
            else if constexpr (kSorted) off = a_row[i] + ((i & 1) ? ch_o : ch_e) + k0;
            else off = ((i & 1) ? a_o : a_e) + (int)(i * 8 * a.lda) + k0;
            dma_b128(dA, base + (wave * kAInstr + i) * 1024, live && !((a_dead >> i) & 1u) ? off : kOob);
        } else {
            const int i = d - kScaleDma - kAInstr;
            const uint32_t dst = base + kA + (wave * kBInstr + i) * 1024;
            const int off = live ? ((i & 1) ? w_o : w_e) + (int)(i * 8 * a.ldw) + k0 : kOob;
            if constexpr (kWeightNt) dma_b128_nt(dW, dst, off);
            else dma_b128(dW, dst, off);
        }
    };

    const int nb_local = (wn * TN) / 128;  // this wavefront's weight-scale block within the tile
    // per-lane fragment offsets: row (lane & 31) of a 32-row fragment, chunk
    // c = 4 kk + 2 (lane >> 5) + h for 16-B half h; swz(row) = (lane >> 1) & 7
    const int fs = (lane >> 1) & 7;
    const int frow = (lane & 31) * kRowB;

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    auto stage_ptr = [&](int s) -> const uint8_t* { return smem + (s % kStages) * kStage; };
    // 16-B read q (0 <= q < 2 (FM + FN)) of K half kk: half q % 2 of fragment
    // q / 2, A fragments first
    auto read_half = [&](const uint8_t* st, int kk, int q, v8i (&af)[FM], v8i (&bf)[FN]) {
        const int f = q >> 1, h = q & 1;
        const int c = 4 * kk + 2 * (lane >> 5) + h;
        const uint8_t* tile = f < FM ? st + (wm * TM + f * 32) * kArow : st + kA + (wn * TN + (f - FM) * 32) * kRowB;
        // fused A rows: tile row r at LDS row (r % 4) kAW + r / 4 (256 B each),
        // chunk c in slot c ^ (r & 15); rows past 4 kAW (never stored) alias
        // loaded ones so every read stays inside the stage's A rows
        int off;
        if (kFuseA && f < FM) {
            const int r = wm * TM + f * 32 + (lane & 31);
            off = ((r & 3) * kAW + ((r >> 2) & (kAW - 1))) * kArow + ((c ^ (r & 15)) << 4) -
                  (int)(tile - st);
        } else {
            off = frow + ((c ^ fs) << 4);
        }
        const v4i v = *reinterpret_cast<const v4i*>(tile + off);
        if (f < FM) {
            if (h) af[f].hi = v; else af[f].lo = v;
        } else {
            if (h) bf[f - FM].hi = v; else bf[f - FM].lo = v;
        }
    };
    // raw fp32 scales of a stage: per fragment row (lane & 31) and the
    // wavefront's weight block (converted to E8M0 only when consumed)
    // kRowW: the packed word of each fragment's W row (lane & 31)
    // kFragW: the fp32 block scale (as bits) of each fragment's 32 W rows
    uint32_t swr[kPerFragW ? FN : 1], nswr[kPerFragW ? FN : 1];
    auto read_scales = [&](const uint8_t* st, float (&sa)[FM], float& sw, uint32_t (&wr)[kPerFragW ? FN : 1]) {
        const float* ssa = reinterpret_cast<const float*>(st + kA + kB);
#pragma unroll
        for (int i = 0; i < FM; ++i) sa[i] = ssa[wm * TM + i * 32 + (lane & 31)];
        if constexpr (kRowW) {
            const uint32_t* sww = reinterpret_cast<const uint32_t*>(st + kA + kB + kSA);
#pragma unroll
            for (int j = 0; j < FN; ++j) wr[j] = sww[wn * TN + j * 32 + (lane & 31)];
            sw = 0.f;
        } else if constexpr (kFragW) {
            const uint32_t* ssw = reinterpret_cast<const uint32_t*>(st + kA + kB + kSA + wave * 256);
#pragma unroll
            for (int j = 0; j < FN; ++j) wr[j] = ssw[((n0 & 127) + wn * TN + j * 32) >> 7];
            sw = 0.f;
        } else {
            const float* ssw = reinterpret_cast<const float*>(st + kA + kB + kSA + wave * 256);
            sw = ssw[nb_local];
        }
    };
    v8i fa0[FM], fb0[FN], fa1[FM], fb1[FN];
    float sa[FM], sw = 0.f, nsa[FM], nsw = 0.f;
    int ea[FM], eb = 0, nea[FM], neb = 0;
    // kRowW: E8M0 byte of each fragment's W row for the current (next) block;
    // kFragW: the rounded-up exponent of each fragment's block scale
    int ebr[kPerFragW ? FN : 1], nebr[kPerFragW ? FN : 1];
    auto row_bytes = [&](const uint32_t (&wr)[kPerFragW ? FN : 1], int gkb, int (&e)[kPerFragW ? FN : 1]) {
        if constexpr (kRowW) {
#pragma unroll
            for (int j = 0; j < FN; ++j) e[j] = (int)((wr[j] >> (8 * (gkb & 3))) & 0xFFu);
        } else if constexpr (kFragW) {
#pragma unroll
            for (int j = 0; j < FN; ++j) e[j] = ue8m0_ceil_byte(__uint_as_float(wr[j]));
            (void)gkb;
        }
    };
    // FP32 contract: mantissa product mu = mant(sA) mant(sW) in [1, 4) of the
    // current block per fragment row, and the rescale ratio mu_prev / mu for
    // the block about to start (the exponents go to the MFMA).
    float mu[kUe8m0 ? 1 : FM], ratio[kUe8m0 ? 1 : FM];
    bool rescale = false;
    // Grouped FP32 contract: rows of another expert (padding) are never
    // stored, so their scales, whatever the buffer holds, must not trigger
    // rescales; they keep a mantissa product of 1.
    bool row_live[kGrouped && !kUe8m0 ? FM : 1];
    if constexpr (kGrouped && !kUe8m0) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = m0 + wm * TM + i * 32 + (lane & 31);
            row_live[i] = r < a.M && a.expert_ids[r] == expert;
        }
    }
    // E8M0 bytes of raw scales; FP32 contract: the first block's mantissa
    // products (step < 0), or the ratios to the next block's products, which
    // then become current (their block follows)
    auto convert = [&](const float (&s)[FM], float w, int (&e)[FM], int& f, int step) {
        if constexpr (kUe8m0) {
#pragma unroll
            for (int i = 0; i < FM; ++i) e[i] = ue8m0_ceil_byte(s[i]);
            f = ue8m0_ceil_byte(w);
        } else {
            const float mw = scale_mant(w);
            float m[FM];
            bool diff = false;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                e[i] = scale_exp_byte(s[i]);
                m[i] = scale_mant(s[i]) * mw;
                if constexpr (kGrouped) m[i] = row_live[i] ? m[i] : 1.f;
                diff |= m[i] != mu[i];
            }
            f = scale_exp_byte(w);
            if (step >= 0) {
                // the quotient of two different values in [1, 4) is never 1,
                // so the divisions are needed exactly when a product changed
                rescale = __any(diff);
                if (rescale) {
#pragma unroll
                    for (int i = 0; i < FM; ++i) ratio[i] = mu[i] == m[i] ? 1.f : mu[i] / m[i];
                }
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) mu[i] = m[i];
        }
    };
    // MFMA t (0 <= t < FM FN) of a sub-step.  The product is formed as
    // D^T = W A^T (W fragment as the MFMA's A operand), so accumulator
    // register r of lane l holds output row (l % 32) of fragment i and column
    // 8 (r / 4) + 4 (l / 32) + r % 4 of fragment j: every lane owns runs of
    // four consecutive columns of one row, ready for packed stores.  The
    // block's scales enter as E8M0 operands: eb for the W rows, ea[i] per A row.
    auto mfma_at = [&](int t, const v8i (&fa)[FM], const v8i (&fb)[FN]) {
        const int i = t / FN, j = t % FN;
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], acc[i][j], 0, 0, 0,
                                                                      kPerFragW ? ebr[j] : eb, 0, ea[i]);
    };
    // FP32 contract: bring the running sum to the new block's mantissa base
    // before the block's first MFMA.  One uniform branch around all of it,
    // so the accumulators only leave the MFMA registers when a ratio is not 1.
    auto rescale_all = [&]() {
        if constexpr (!kUe8m0) {
            if (rescale) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] * ratio[i];
            }
        }
    };

    // Each sub-step is laid out as FM*FN issue slots: one MFMA, then this
    // slot's share of the LDS fragment reads and (sub-step 1) of the next
    // stage's DMAs.  sched_barrier keeps the slots in order, so the single
    // texture-address unit of the CU sees a steady trickle of DMAs from each
    // wavefront instead of a burst that stalls the MFMA issue behind it.
    constexpr int kT = FM * FN;           // MFMAs per sub-step
    constexpr int kR = 2 * (FM + FN);     // 16-B fragment reads per sub-step

    // Fused A: the 4 kFuseA rows of a block this wavefront's own DMAs
    // brought (tile rows w, w + 4, ...), quantized in place, 16 / kFuseA lanes
    // per row and 8 kFuseA values per lane: the group absmax (packed 16-bit
    // max of the sign-cleared words, then over the row's lanes by DPP), the
    // UE8M0 scale and the codes exactly as the quant kernel derives them (its
    // general path for a group with an infinity, a NaN or a subnormal scale);
    // fp8 chunk c of row r takes slot c ^ (r & 15) of the row's 256 bytes, the
    // scale the stage's activation-scale slot.  Every lane's loads complete
    // before the first write (the DPP max consumes them all), and no other
    // wavefront reads these rows before the next barrier.
    auto quant_rows = [&](const uint8_t* st_c) {
        if constexpr (kFuseA) {
            typedef uint16_t u16v2 __attribute__((ext_vector_type(2)));
            constexpr int kQ = kFuseA;            // 16-B bf16 chunks per lane
            constexpr int kLanes = 16 / kQ;       // lanes per row
            uint8_t* st = const_cast<uint8_t*>(st_c);
            const int pl = lane / kLanes;         // row of this wave: LDS row 16 w + pl
            const int r = wave + 4 * pl, sr = r & 15;
            const int c0 = (lane % kLanes) * kQ;  // first bf16 chunk of the lane
            uint8_t* row = st + (kAW * wave + pl) * kArow;
            u32x4 v[kQ];
#pragma unroll
            for (int q = 0; q < kQ; ++q) v[q] = *reinterpret_cast<const u32x4*>(row + (((c0 + q) ^ sr) << 4));
            u16v2 m{0, 0};
#pragma unroll
            for (int q = 0; q < kQ; ++q) {
                m = __builtin_elementwise_max(m, __builtin_bit_cast(u16v2, v[q].x & 0x7FFF7FFFu));
                m = __builtin_elementwise_max(m, __builtin_bit_cast(u16v2, v[q].y & 0x7FFF7FFFu));
                m = __builtin_elementwise_max(m, __builtin_bit_cast(u16v2, v[q].z & 0x7FFF7FFFu));
                m = __builtin_elementwise_max(m, __builtin_bit_cast(u16v2, v[q].w & 0x7FFF7FFFu));
            }
            // max over the row's kLanes consecutive lanes (operands are non-negative float bits)
            auto row_max = [](uint32_t x) {
                if constexpr (kLanes == 16) {
                    return row16_max_u32(x);
                } else {
                    uint32_t t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);  // [1,0,3,2]
                    x = x > t ? x : t;
                    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
                    x = x > t ? x : t;
                    if constexpr (kLanes == 8) {
                        t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);  // row_half_mirror
                        x = x > t ? x : t;
                    }
                    return x;
                }
            };
            const uint32_t abits = row_max((uint32_t)(m.x > m.y ? m.x : m.y) << 16);
            float sc = ue8m0_ceil_div448(fmaxf(__uint_as_float(abits), a.eps));
            uint32_t c[2 * kQ];
            if (ue8m0_fast_path(abits, sc)) {
#pragma unroll
                for (int q = 0; q < kQ; ++q) {
                    c[2 * q] = pack4_e4m3_bf16(v[q].x, v[q].y, sc);
                    c[2 * q + 1] = pack4_e4m3_bf16(v[q].z, v[q].w, sc);
                }
            } else {   // uniform over the row's lanes
                float amax = 0.0f;
#pragma unroll
                for (int q = 0; q < kQ; ++q) {
                    amax = fmaxf(amax, fabsf(bf16lo(v[q].x)));
                    amax = fmaxf(amax, fabsf(bf16hi(v[q].x)));
                    amax = fmaxf(amax, fabsf(bf16lo(v[q].y)));
                    amax = fmaxf(amax, fabsf(bf16hi(v[q].y)));
                    amax = fmaxf(amax, fabsf(bf16lo(v[q].z)));
                    amax = fmaxf(amax, fabsf(bf16hi(v[q].z)));
                    amax = fmaxf(amax, fabsf(bf16lo(v[q].w)));
                    amax = fmaxf(amax, fabsf(bf16hi(v[q].w)));
                }
                sc = ue8m0_ceil_div448(fmaxf(__uint_as_float(row_max(__float_as_uint(amax))), a.eps));
#pragma unroll
                for (int q = 0; q < kQ; ++q) {
                    c[2 * q] = pack4_e4m3_ue8m0_general(bf16lo(v[q].x), bf16hi(v[q].x), bf16lo(v[q].y),
                                                        bf16hi(v[q].y), sc);
                    c[2 * q + 1] = pack4_e4m3_ue8m0_general(bf16lo(v[q].z), bf16hi(v[q].z), bf16lo(v[q].w),
                                                            bf16hi(v[q].w), sc);
                }
            }
            // codes of bf16 chunk c0 + q are fp8 bytes [8 (c0 + q), +8): chunk (c0 + q) / 2, half (c0 + q) % 2
            if constexpr (kQ == 1) {
                *reinterpret_cast<uint2*>(row + (((c0 >> 1) ^ sr) << 4) + 8 * (c0 & 1)) = make_uint2(c[0], c[1]);
            } else {
#pragma unroll
                for (int q = 0; q < kQ; q += 2)
                    *reinterpret_cast<u32x4*>(row + ((((c0 + q) >> 1) ^ sr) << 4)) =
                        u32x4{c[2 * q], c[2 * q + 1], c[2 * q + 2], c[2 * q + 3]};
            }
            if (lane % kLanes == 0) reinterpret_cast<float*>(st + kA + kB)[r] = sc;
        } else {
            (void)st_c;
        }
    };

    // MoE tiles: this wavefront computes its A fragments up to the last one
    // holding a row of the tile's expert (nlive of FM); the fragment reads and
    // MFMAs of the fragments past it are left out, so the 32-row fragments of
    // padding at a segment's end cost no matrix-core or LDS time.  Their
    // accumulators stay zero and their rows are never stored, so the output
    // is the same bits.  Dense tiles: FM, a constant (same instructions as
    // without this).  cfg4 (121 of 377 row tiles hold at most 32 rows of
    // their expert), one box, three interleaved rounds: GEMM1 with the
    // SiLU*Mul epilogue 1835-1855 -> 1787-1803 us, plain GEMM1 and the down
    // GEMM unchanged, the experts layer 2942-2951 -> 2920-2946 us.
    int nlive = FM;
    if constexpr (kGrouped) {
        static_assert(!kGrouped || (FM == 2 && TM == 64), "one ballot bit per wavefront row, two A fragments");
        const int r = m0 + wm * TM + lane;
        const uint64_t live = __ballot(r < a.M && a.expert_ids[r] == expert);
        nlive = (live >> 32) ? 2 : live ? 1 : 0;
    }
    auto want = [&](int q) { return !kGrouped || ((q >> 1) < FM ? (q >> 1) < nlive : nlive > 0); };
    // prologue: blocks 0 .. kStages-1 in flight, block 0 published
#pragma unroll
    for (int s = 0; s < kStages; ++s)
#pragma unroll
        for (int d = 0; d < kDma; ++d) issue_one(s, s < KB, d);
    wait_dma_n<(kStages - 1) * kDma>();
    quant_rows(stage_ptr(0));   // fused A: block 0 (the loop quantizes block kb+1 in iteration kb)
    __syncthreads();
    read_scales(stage_ptr(0), sa, sw, swr);
#pragma unroll
    for (int q = 0; q < kR; ++q)
        if (want(q)) read_half(stage_ptr(0), 0, q, fa0, fb0);

    convert(sa, sw, ea, eb, -1);
    row_bytes(swr, kb0, ebr);

    for (int kb = 0; kb < KB; ++kb) {
        const uint8_t* cur = stage_ptr(kb);
        rescale_all();
        // ---- sub-step 0: K half 0 of block kb; read K half 1
#pragma unroll
        for (int t = 0; t < kT; ++t) {
            if (!kGrouped || t / FN < nlive) mfma_at(t, fa0, fb0);
#pragma unroll
            for (int q = t * kR / kT; q < (t + 1) * kR / kT; ++q)
                if (want(q)) read_half(cur, 1, q, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
        }

        // fused A: block kb+1's rows of this wavefront, quantized in place as
        // soon as they have landed (its own DMAs: the activation rows come
        // from L2 ahead of the block's weights, which may still stream in);
        // the hand-off below publishes the codes with the weights
        if constexpr (kFuseA) {
            wait_dma_n<(kStages - 2) * kDma + kBInstr>();
            quant_rows(stage_ptr(kb + 1));
        }

        // ---- hand-off: publish block kb+1, free buffer kb for block kb+kStages
        wait_dma_n<(kStages - 2) * kDma>();
        wait_lds();
        __syncthreads();

        // ---- sub-step 1: K half 1 of block kb; read K half 0 of block kb+1
        // (past the last block this reads a zero-filled buffer, unused) and
        // DMA block kb+kStages into the freed buffer
        const uint8_t* nxt = stage_ptr(kb + 1);
        const int snext = kb + kStages;
        const bool live = snext < KB;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
            if (!kGrouped || t / FN < nlive) mfma_at(t, fa1, fb1);
            if (t == 0) read_scales(nxt, nsa, nsw, nswr);
            // converted scales of block kb+1, half a sub-step after their
            // reads (FP32 contract: none past the last block, whose mantissa
            // products the store needs)
            if (t == kT / 2) {
                if constexpr (kUe8m0) convert(nsa, nsw, nea, neb, kb);
                else if (kb + 1 < KB) convert(nsa, nsw, nea, neb, kb);
                row_bytes(nswr, kb0 + kb + 1, nebr);
            }
#pragma unroll
            for (int q = t * kR / kT; q < (t + 1) * kR / kT; ++q)
                if (want(q)) read_half(nxt, 0, q, fa0, fb0);
#pragma unroll
            for (int d = t * kDma / kT; d < (t + 1) * kDma / kT; ++d) issue_one(snext, live, d);
            __builtin_amdgcn_sched_barrier(0);
        }
        // FP32 contract: the running sum is kept in units of the current
        // block's mantissa product, S_kb = S_{kb-1} mu_{kb-1} / mu_kb + 2^e P_kb
        // (rescale_at applies the ratio as block kb+1 starts), so the true
        // sum after the last block is S mu_last.  Ratios of 1 (power-of-two
        // scales, or equal mantissas) skip the multiplies.
#pragma unroll
        for (int i = 0; i < FM; ++i) ea[i] = nea[i];
        eb = neb;
        if constexpr (kPerFragW) {
#pragma unroll
            for (int j = 0; j < FN; ++j) ebr[j] = nebr[j];
        }
    }
    // the trailing (out-of-range) loads still target this workgroup's LDS
    wait_dma();
    if constexpr (!kUe8m0) {
        bool any = false;
#pragma unroll
        for (int i = 0; i < FM; ++i) any |= mu[i] != 1.f;
        if (__any(any)) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] * mu[i];
        }
    }

    // Epilogue of a tile: fp32 -> bf16 (RNE), written with raw buffer stores
    // whose range ends at the last row of D, so rows past M (and any offset
    // set to kOob) are dropped by the hardware and no store is branched
    // around.  Lanes l and l + 32 hold the two 4-column halves of each
    // 8-column run of a row; one permlane32 swap per dword pair gives each
    // lane a whole 16-B run.  D rows that are not 16-B aligned (or N not a
    // multiple of 8 on a ragged tile) take 2-B element stores instead.
    // Split-K epilogue: the fp32 partial sums, one 16-B store per run of four
    // columns, into this (split, tile)'s BM x BN slab (rows past M dropped by
    // the range).
    auto epilogue_partial = [&]() {
        const int64_t bytes = (int64_t)min(a.M - m0, BM) * BN * 4;
        const __amdgpu_buffer_rsrc_t dP = __builtin_amdgcn_make_buffer_rsrc(
            a.P + ((int64_t)split * a.tile_count + trel) * BM * BN, (short)0, (int)bytes, (int)kRsrcWord3);
        // Slabs that fit the idle LDS stages leave as whole rows: each
        // wavefront parks its fp32 block row-major (16-B chunks rotated by the
        // row index) and stores TN * 4 bytes per row, whole 128-B lines,
        // instead of four 32-B pieces per line (which the L2 fills from memory
        // before merging).  Same slab layout, same values.  One box, HIP
        // events, weights rotated past the MALL: qkv 64 x 10240 x 8192 22.2 ->
        // 20.0 us, o 64 x 8192 x 8192 19.8 -> 17.5 us, 32 rows 6-7% faster.
        // Tiles with few live rows (decode at M < 16) keep the direct
        // stores: they write few lines, and the LDS round trip cost them
        // 0.1-0.5 us.
        constexpr bool kLdsSlab = BM * BN * 4 <= kStages * kStage && (TN == 64 || TN == 32);
        if constexpr (kLdsSlab) if (min(a.M - m0, BM) >= 16) {
            constexpr int kCh = TN / 4;                 // 16-B chunks per wavefront row
            constexpr int kRowB4 = TN * 4;              // bytes per wavefront row
            constexpr int kRowsPer = 64 / kCh;          // rows per store instruction
            uint8_t* reg = smem + wave * (TM * kRowB4);
            __syncthreads();   // every wavefront is past its last stage reads
            const int h = lane >> 5;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int rl = i * 32 + (lane & 31);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const int c = 8 * j + 2 * p + h;   // this lane's 16-B chunk of the row (4 columns)
                        const u32x4 v = {__float_as_uint(acc[i][j][4 * p]), __float_as_uint(acc[i][j][4 * p + 1]),
                                         __float_as_uint(acc[i][j][4 * p + 2]), __float_as_uint(acc[i][j][4 * p + 3])};
                        *reinterpret_cast<u32x4*>(reg + rl * kRowB4 + ((c + rl) % kCh) * 16) = v;
                    }
            }
            wait_lds();
            const int cl = lane % kCh, rsub = lane / kCh;
#pragma unroll
            for (int it = 0; it < TM / kRowsPer; ++it) {
                const int rl = it * kRowsPer + rsub;
                const u32x4 v = *reinterpret_cast<const u32x4*>(reg + rl * kRowB4 + ((cl + rl) % kCh) * 16);
                const int voff = (wm * TM + rl) * BN * 4 + (wn * TN + cl * 4) * 4;
                if (a.flags) __builtin_amdgcn_raw_buffer_store_b128(v, dP, voff, 0, kDeviceCoherent);
                else __builtin_amdgcn_raw_buffer_store_b128(v, dP, voff, 0, 0);
            }
            return;
        }
        const int ncol = wn * TN + 4 * (lane >> 5);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int roff = (wm * TM + i * 32 + (lane & 31)) * BN * 4;
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int voff = roff + (ncol + j * 32 + 8 * p) * 4;
                    const v4i v = {__float_as_int(acc[i][j][4 * p]), __float_as_int(acc[i][j][4 * p + 1]),
                                   __float_as_int(acc[i][j][4 * p + 2]), __float_as_int(acc[i][j][4 * p + 3])};
                    if (a.flags)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), dP, voff, 0,
                                                               kDeviceCoherent);
                    else
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), dP, voff, 0, 0);
                }
        }
    };

    // sorted layout: each fragment row's output row (its pair) and factor
    int out_row[kSorted ? FM : 1];
    if constexpr (kSorted) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            out_row[i] = pair_of(wm * TM + i * 32 + (lane & 31));
            if (a.row_weight) {
                const float f = out_row[i] >= 0 ? a.row_weight[out_row[i]] : 0.f;
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] * f;
            }
        }
    }
    // row byte offset of fragment row i in D (kOob: not stored)
    auto out_off = [&](int i) -> int {
        const int row = wm * TM + i * 32 + (lane & 31);
        if constexpr (kSorted) return out_row[i] >= 0 ? out_row[i] * (int)a.ldd * 2 : kOob;
        else if constexpr (kGrouped)
            return (m0 + row < a.M && a.expert_ids[m0 + row] == expert) ? row * (int)a.ldd * 2 : kOob;
        else return row * (int)a.ldd * 2;
    };

    auto epilogue = [&]() {
        const int64_t bytes = kSorted ? a.D_bytes
                                      : std::min<int64_t>((int64_t)(a.M - m0 - 1) * a.ldd * 2 + (int64_t)a.N * 2,
                                                          (int64_t)BM * a.ldd * 2);
        const __amdgpu_buffer_rsrc_t dD = __builtin_amdgcn_make_buffer_rsrc(
            kSorted ? a.D : a.D + (int64_t)m0 * a.ldd, (short)0, (int)std::min<int64_t>(bytes, 0x7FFFFFFFLL),
            (int)kRsrcWord3);
        const int h = lane >> 5;
        const int ncol = n0 + wn * TN + 8 * h;
        const bool vec = a.vec_store && (n0 + BN <= a.N || a.N % 8 == 0);
        // 256-row dense tiles, the 128-row MoE tiles (and short-K 64/128-row
        // dense tiles, below): the fragments'
        // natural stores write each 128-B line of D as four 32-B pieces (32
        // rows x 32 B per instruction), and the tiles of a wave of workgroups
        // all end at once.  Instead each wavefront parks its bf16 block in the
        // (now idle) LDS stages, row-major with each row's 16-B chunks rotated
        // by the row index (conflict-spreading), reads it back by whole rows
        // and stores full lines, non-temporal (4 rows x 256 B per instruction
        // for 128 columns, 8 x 128 B for 64, 4 x 192 B for 96).  Bit-identical;
        // one box, interleaved runs: q_b M = 4096 167 -> 160 us, gate_up 836 ->
        // 825 us; cfg4 grouped down 1007 -> 935 us, gate_up 1965 -> 1929 us
        // (UE8M0), layer 3165 -> 3112 us.  With the natural partial-line
        // stores the non-temporal hint was much slower (q_b 157 -> 284 us):
        // those pieces must merge in L2.
        constexpr bool kLdsEpi =
            !kSplitK && (TN == 128 || TN == 96 || TN == 64) && BM * BN * 2 <= kStages * kStage;
        // The FP32 contract's 128x256 dense tiles (one workgroup per CU, as
        // 256x256) always stage: gate_up M = 4096 1122 -> 1105 us,
        // 1024 x 7168 x 4096 40 -> 37.4 us.  64- and 128-row dense tiles of
        // at most 128 columns stage their block only for short K (at
        // most 16 blocks) and at least 16 live rows: q_b at M = 128 (12
        // blocks) 13.5 -> 12.7 us, while long-K weight-streaming tiles lost
        // 2-4% (their workgroup's exit waits on the staging while its
        // neighbour on the CU streams) and decode rows write few lines
        static_assert(!kGlu || kLdsEpi, "the SiLU*Mul epilogue runs on the LDS-staged block");
        if (kLdsEpi && (vec || kGlu) &&
            (kGrouped || kSorted || BM == 256 || BN == 256 || (KB <= 16 && min(a.M - m0, BM) >= 16))) {
            constexpr int kCh = TN / 8;                            // 16-B chunks per wavefront row
            constexpr int kRowB2 = TN * 2;                         // bytes per wavefront row
            constexpr int kRowsPer = kCh == 12 ? 4 : 64 / kCh;     // rows per store instruction
            constexpr int kNt = 2;                                 // cache policy: non-temporal
            uint8_t* reg = smem + wave * (TM * kRowB2);
            __syncthreads();   // every wavefront is past its last stage reads (and the DMAs have landed)
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int rl = i * 32 + (lane & 31);
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int p = 0; p < 4; p += 2) {
                        const uint32_t x0 = pack_bf16(acc[i][j][4 * p], acc[i][j][4 * p + 1]);
                        const uint32_t x1 = pack_bf16(acc[i][j][4 * p + 2], acc[i][j][4 * p + 3]);
                        const uint32_t y0 = pack_bf16(acc[i][j][4 * p + 4], acc[i][j][4 * p + 5]);
                        const uint32_t y1 = pack_bf16(acc[i][j][4 * p + 6], acc[i][j][4 * p + 7]);
                        const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
                        const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
                        const int c = 4 * j + p + h;     // this lane's 16-B chunk of the row (8 columns)
                        const u32x4 v = {(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
                        *reinterpret_cast<u32x4*>(reg + rl * kRowB2 + ((c + rl) % kCh) * 16) = v;
                    }
                }
            }
            // grouped: rows of another expert (padding) are not stored
            uint64_t row_mask = ~0ull;
            if constexpr (kGrouped) {
                static_assert(!kGrouped || TM <= 64, "one mask bit per wavefront row");
                // kGlu: the rows of this wavefront's SiLU*Mul pass below
                const int r = m0 + (kGlu ? wave * (BM / 4) : wm * TM) + lane;
                row_mask = __ballot(lane < (kGlu ? BM / 4 : TM) && r < a.M && a.expert_ids[r] == expert);
            }
            wait_lds();
            if constexpr (kGlu) {
                // SiLU*Mul + 1x128 quant: wavefront w takes tile rows [32 w, 32 w + 32),
                // 16 lanes (one 128-column group) per row, four rows per pass;
                // row rt's gate block is wavefront (rt / 64, 0)'s, its up block
                // wavefront (rt / 64, 1)'s, both laid out as stored above
                __syncthreads();   // every wavefront's block is in LDS
                const int sub = lane & 15, rq = lane >> 4;
#pragma unroll
                for (int it = 0; it < BM / 4 / 4; ++it) {
                    const int rt = wave * (BM / 4) + it * 4 + rq;
                    const int r = m0 + rt;
                    if ((row_mask >> (it * 4 + rq)) & 1) {   // uniform over the row's 16 lanes
                        const int bw = rt / TM, rl = rt % TM;
                        const uint8_t* gate = smem + (bw * WN) * (TM * kRowB2) + rl * kRowB2 + ((sub + rl) % kCh) * 16;
                        const u32x4 g = *reinterpret_cast<const u32x4*>(gate);
                        const u32x4 u = *reinterpret_cast<const u32x4*>(gate + TM * kRowB2);
                        const uint32_t w[4] = {silu_mul_pair(a.silu_lut, g.x, u.x), silu_mul_pair(a.silu_lut, g.y, u.y),
                                               silu_mul_pair(a.silu_lut, g.z, u.z), silu_mul_pair(a.silu_lut, g.w, u.w)};
                        uint8_t* q = a.q2 + (int64_t)r * a.ldq2 + n0;
                        const float sc = a.glu_ue8m0 ? quant8_store<true, false>(w, a.glu_eps, sub, q)
                                                     : quant8_store<false, false>(w, a.glu_eps, sub, q);
                        if (sub == 0) a.s2[(int64_t)r * a.s2_sm + (int64_t)(n0 / 128) * a.s2_sg] = sc;
                    }
                }
                return;
            }
            const bool active = lane < kRowsPer * kCh;             // 96 columns: 48 lanes of 64 store
            const int cl = active ? lane % kCh : 0, rsub = active ? lane / kCh : 0;
            const int col = n0 + wn * TN + cl * 8;
            const bool col_ok = active && col < a.N;
#pragma unroll
            for (int it = 0; it < TM / kRowsPer; ++it) {
                const int rl = it * kRowsPer + rsub;
                const u32x4 v = *reinterpret_cast<const u32x4*>(reg + rl * kRowB2 + ((cl + rl) % kCh) * 16);
                int roff;
                if constexpr (kSorted) {
                    // the output row (routed pair) of wavefront row rl, held by
                    // lane rl % 32 for fragment rl / 32 (rl / 32 is it / 8)
                    const int orow = __shfl(out_row[(it * kRowsPer) / 32], rl & 31);
                    roff = orow >= 0 ? orow * (int)a.ldd * 2 : kOob;
                } else if constexpr (kGrouped) {
                    roff = ((row_mask >> rl) & 1ull) ? (wm * TM + rl) * (int)a.ldd * 2 : kOob;
                } else {
                    roff = (wm * TM + rl) * (int)a.ldd * 2;
                }
                const int voff = col_ok && roff != kOob ? roff + col * 2 : kOob;
                __builtin_amdgcn_raw_buffer_store_b128(v, dD, voff, 0, kNt);
            }
        } else if (vec) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int roff = out_off(i);
                const bool ok = roff != kOob;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int p = 0; p < 4; p += 2) {
                        // dwords of runs p (X) and p + 1 (Y): columns 8 p + 4 h + {0..3}
                        const uint32_t x0 = pack_bf16(acc[i][j][4 * p], acc[i][j][4 * p + 1]);
                        const uint32_t x1 = pack_bf16(acc[i][j][4 * p + 2], acc[i][j][4 * p + 3]);
                        const uint32_t y0 = pack_bf16(acc[i][j][4 * p + 4], acc[i][j][4 * p + 5]);
                        const uint32_t y1 = pack_bf16(acc[i][j][4 * p + 6], acc[i][j][4 * p + 7]);
                        // lanes < 32 end with run p (own half, then lane + 32's);
                        // lanes >= 32 with run p + 1 (lane - 32's half, then own)
                        const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
                        const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
                        const int n = ncol + j * 32 + 8 * p;
                        const int voff = (ok && n < a.N) ? roff + n * 2 : kOob;
                        const u32x4 v = {(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
                        __builtin_amdgcn_raw_buffer_store_b128(v, dD, voff, 0, 0);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int roff = out_off(i);
                const bool ok = roff != kOob;
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int n = n0 + wn * TN + j * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                        const int voff = (ok && n < a.N) ? roff + n * 2 : kOob;
                        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16(acc[i][j][r], 0.f) & 0xFFFFu), dD,
                                                              voff, 0, 0);
                    }
            }
        }
    };

    if constexpr (kSplitK) {
        epilogue_partial();
        // the fused sum is only planned for the 64-row tiles (fused_split_sum)
        if constexpr (BM <= 64) if (a.flags) {
            // Fused reduction: every wavefront's (device-coherent) slab stores
            // have completed before its workgroup counts itself in; the
            // workgroup that brings the tile's count to `splits` sums all
            // slabs (its own included, in split order, with device-coherent
            // loads) and leaves the counter at zero.  No workgroup waits for
            // another, so nothing depends on residency.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // also: the main loop's LDS reads are done, smem is free
            unsigned* last = reinterpret_cast<unsigned*>(smem);
            if (threadIdx.x == 0) {
                const unsigned prev =
                    __hip_atomic_fetch_add(a.flags + trel, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const unsigned is_last = prev + 1 == (unsigned)a.splits;
                if (is_last) __hip_atomic_store(a.flags + trel, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *last = is_last;
            }
            __syncthreads();
            if (*last) {
                constexpr int kRuns = BN / 4, kRowStep = 64 * kWaves / kRuns;
                static_assert((64 * kWaves) % kRuns == 0, "whole rows per pass");
                splitk_sum_rows<BM, BN, kDeviceCoherent, (BM + kRowStep - 1) / kRowStep>(
                    a, trel, m0, n0, (int)threadIdx.x / kRuns, min(a.M - m0, BM), kRowStep,
                    ((int)threadIdx.x % kRuns) * 4);
            }
        }
    } else {
        epilogue();
    }
}

// Split-K reduction: D = bf16(sum_s slab[s]) summed in split order
// (deterministic).  One workgroup per 8-row strip of a tile of the split
// launch (blockIdx.x = tile * BM/8 + strip), one float4 run per lane.
template <int BM, int BN>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmArgs a) {
    constexpr int kRuns = BN / 4, kRows = 256 / kRuns;   // rows per pass of the workgroup
    constexpr int kStrips = BM / 8;
    const int trel = blockIdx.x / kStrips, strip = blockIdx.x - trel * kStrips;
    int tm, tn;
    {
        constexpr int kGroupM = 4;
        const int t = a.tile_base + trel;
        const int group = kGroupM * a.tiles_n;
        const int g = t / group;
        const int first_m = g * kGroupM;
        const int gm = min(a.tiles_m - first_m, kGroupM);
        const int w = t - g * group;
        tm = first_m + w % gm;
        tn = w / gm;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    splitk_sum_rows<BM, BN, 0, (8 + kRows - 1) / kRows>(a, trel, m0, n0, strip * 8 + (int)threadIdx.x / kRuns,
                                                        min(strip * 8 + 8, a.M - m0), kRows,
                                                        ((int)threadIdx.x % kRuns) * 4);
}


// Launch plan of a dense GEMM.  Whole waves of tiles run data-parallel in
// one launch; when the last wave would be partly empty, its tiles (the
// "tail") may instead run split-K in a second launch over all workgroup
// slots, followed by the reduction.
struct Schedule {
    int bm = 0, bn = 0, stages = 0;
    int64_t tiles = 0;
    int64_t dp_tiles = 0;         // tiles [0, dp_tiles) data-parallel
    int splits = 1, kb_per_split = 0;  // the tail [dp_tiles, tiles)
    int64_t ws_bytes = 0;         // fp32 slabs of the tail
    bool fused = false;           // the split launch sums the slabs itself
    int fuse_a = 0;               // bf16 activations quantized by the GEMM: rows of four per wavefront (1, 2, 4)
    // 256-row tiles only: the last n192 columns run as 256x192 tiles in a
    // second launch (the first N - n192 as 256x256), so that both launches
    // fill whole waves where 256x256 tiles alone would leave a partial one
    int n192 = 0;
};

// Split-K tails of the 64-row tiles summed by the split launch itself (no
// reduction launch, about 3 us less host time per call): up to 32 rows
// always, up to 48 rows when a tile has at most 4 splits (8 for the 64x64
// tiles, whose slabs are half as wide), up to 64 rows when it also has at
// most 24 K blocks per split.  The summing workgroup reads
// its tile's slabs alone, so more rows, deeper splits or long splits (whose
// workgroups finish far apart) measure slower than the separate reduction
// spread over 8-row strips (64 rows: 1024 x 28672 15.1 -> 17.1 us,
// 8192 x 28672 44.1 -> 46.3 us; 40-64 rows with 3-4 splits of at most 22
// blocks: 10240 x 8192 21.9 -> 21.0 us at 49 rows, 8192 x 8192 19.9 -> 18.5
// us at 49 rows and 20.2 -> 19.9 us at 64, 2048 x 2048 10.9 -> 10.3 us).
constexpr int kFusedReduceRows = 32, kFusedShallowRows = 48, kFusedShallowSplits = 4, kFusedShortKb = 24;
constexpr bool fused_split_sum(int bm, int bn, int64_t M, int splits, int kb_per_split) {
    const int max_splits = bn <= 64 ? 2 * kFusedShallowSplits : kFusedShallowSplits;
    return bm <= 64 && (M <= kFusedReduceRows || (M <= kFusedShallowRows && splits <= max_splits) ||
                        (M <= 64 && splits <= max_splits && kb_per_split <= kFusedShortKb));
}
// Arrival counters of the fused split-K reduction for one launch on `st`, or
// nullptr (then the separate reduction kernel runs); defined in gemm.hip.
unsigned* splitk_flags_for(hipStream_t st, int64_t tail_tiles);

// The 256x256 dense tiles (M > 128, UE8M0), built in their own translation
// unit (gemm_big.hip) without the VGPR-form MFMA option: their 256
// accumulators per lane need the AGPRs.
int launch_gemm_256(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what);
int launch_gemm_256_roww(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what);

template <int BM, int BN, int kStages, bool kUe8m0, bool kGrouped, int kWaves = 4, int kFuseA = 0, bool kRowW = false,
          bool kGlu = false>
static int launch_gemm(GemmArgs a, const Schedule& sc, hipStream_t st, const char* what) {
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = kGlu ? a.glu_half / (BN / 2) : (a.N + BN - 1) / BN;
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    KBN_CHECK_ARG(tiles <= 0x7FFFFFFFLL, "%s: too many tiles", what);
    const int64_t dp = (!kGrouped && a.P && sc.splits > 1) ? sc.dp_tiles : tiles;
    if (dp > 0) {
        a.tile_base = 0;
        a.tile_count = (int)dp;
        a.splits = 1;
        a.kb_per_split = a.K / kRowB;
        if (kGrouped) a.group_m = moe_group_m(a.K);
        const int64_t grid = kGrouped ? moe_dealt_grid(a.tiles_m, a.tiles_n, a.group_m) : dp;
        KBN_CHECK_ARG(grid <= 0x7FFFFFFFLL, "%s: too many tiles", what);
        gemm_bs_kernel<BM, BN, kStages, kUe8m0, kGrouped, false, kWaves, false, kFuseA, kRowW, kGlu>
            <<<dim3((unsigned)grid), dim3(64 * kWaves), 0, st>>>(a);
        KBN_CHECK_LAUNCH(what);
    }
    if (dp < tiles) {
        // the plan must be for this tile shape, and its slabs must fit the workspace
        KBN_CHECK_ARG(sc.bm == BM && sc.bn == BN && sc.tiles == tiles && sc.fuse_a == kFuseA,
                      "%s: split plan does not match the %dx%d tiles", what, BM, BN);
        const int64_t need = (int64_t)sc.splits * (tiles - dp) * BM * BN * 4;
        KBN_CHECK_ARG(need < 0x7FFFFFFFLL, "%s: split slabs span >= 2 GiB", what);
        KBN_CHECK_ARG(sc.splits >= 2 && sc.kb_per_split >= 1 && need <= a.ws_bytes,
                      "%s: workspace of %lld bytes is smaller than the %lld the split plan writes", what,
                      (long long)a.ws_bytes, (long long)need);
        KBN_CHECK_ARG((int64_t)sc.splits * sc.kb_per_split >= a.K / kRowB &&
                          (int64_t)(sc.splits - 1) * sc.kb_per_split < a.K / kRowB,
                      "%s: split plan does not cover K in %d non-empty splits", what, sc.splits);
        a.tile_base = (int)dp;
        a.tile_count = (int)(tiles - dp);
        a.splits = sc.splits;
        a.kb_per_split = sc.kb_per_split;
        const int64_t blocks = (tiles - dp) * sc.splits;
        KBN_CHECK_ARG(blocks <= 0x7FFFFFFFLL, "%s: too many tiles", what);
        // Few rows: the tile's last workgroup sums the slabs (one launch
        // less).  More rows: that sum would run on one workgroup per tile at
        // the end of the launch, so the separate kernel spreads it instead.
        a.flags = (BM <= 64 && sc.fused) ? splitk_flags_for(st, tiles - dp) : nullptr;
        gemm_bs_kernel<BM, BN, kStages, kUe8m0, kGrouped && false, true, kWaves, false, kFuseA, kRowW>
            <<<dim3((unsigned)blocks), dim3(64 * kWaves), 0, st>>>(a);
        KBN_CHECK_LAUNCH(what);
        if (!a.flags) {
            splitk_reduce_kernel<BM, BN><<<dim3((unsigned)((tiles - dp) * (BM / 8))), dim3(256), 0, st>>>(a);
            KBN_CHECK_LAUNCH(what);
        }
    }
    return 0;
}

}  // namespace kbn
