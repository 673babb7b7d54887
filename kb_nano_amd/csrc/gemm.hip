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
//  * FP32 (disable_ue8m0_cast): scales are used as given; each 128-K stage
//    accumulates a fresh partial with plain fp8 MFMA and is promoted into the
//    running sum with one FMA per element and stage.
//
// Dataflow per workgroup (256 lanes = 4 wavefronts, one per SIMD):
//   HBM --buffer_load_dwordx4 ... lds (direct DMA)--> LDS (4 stages x (BM+BN) x 64 B)
//   LDS --ds_read_b128--> VGPR fragments --MFMA 32x32x64--> fp32 accumulators
// Each LDS row is 64 B (one 64-K stage); its four 16-B chunks are XOR-
// swizzled so the rows read by one ds_read_b128 hit distinct banks.  The
// swizzle is applied on the global side of the DMA (lane i of a load
// instruction always writes LDS chunk i), so no extra LDS pass is needed.
// Out-of-range rows read as zero through the buffer descriptor's range check.

#include "kbn_common.h"

namespace kbn {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;           // K per stage == scale block
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dword format (gfx9 family)

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

constexpr int kOob = (int)0x80000000;  // offset beyond any range: reads zero

// LDS row layout.  A stage holds 64 K per row (64 B = four 16-B chunks);
// chunk c of row r lives in slot c ^ ((r >> 2) & 3).  A ds_read_b128 is served
// 16 lanes (256 B, all 64 banks) per cycle; the 16 rows read by 16 lanes span
// four 256-B bank lines (r % 4) with four distinct slots each (r >> 2), so
// fragment reads are conflict-free.
__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// 32 bytes of K (chunks c0, c0+1) of LDS row `r` as one MFMA operand.
__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int r, int c0) {
    const v4i lo = *reinterpret_cast<const v4i*>(tile + r * 64 + ((c0 ^ swz(r)) << 4));
    const v4i hi = *reinterpret_cast<const v4i*>(tile + r * 64 + (((c0 + 1) ^ swz(r)) << 4));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// XCD-aware tile order.  Consecutive workgroup ids are dispatched round-robin
// over the 8 XCDs; give each XCD a contiguous range of the tile sequence so
// the tiles resident on one XCD (and its L2) share A row panels and W panels,
// and walk that sequence in column groups of kGroupM row tiles.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kGroupM = 4;
    const int nblk = gridDim.x;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, i = bid >> 3;
    const int per = nblk >> 3, rem = nblk & 7;
    const int t = xcd * per + (xcd < rem ? xcd : rem) + i;
    const int group = kGroupM * tiles_n;
    const int g = t / group;
    const int first_m = g * kGroupM;
    const int gm = min(tiles_m - first_m, kGroupM);
    const int w = t - g * group;
    tm = first_m + w % gm;
    tn = w / gm;
}

constexpr int kKS = 64;      // K per LDS stage (one 32x32x64 MFMA deep)
constexpr int kStages = 4;   // LDS buffers: three stages in flight while one is read

// Block-scaled GEMM tile kernel.
// LDS stage layout: [A: BM x 64 B][W: BN x 64 B][sA: 64 fp32 per wavefront][sW: 64 fp32 per wavefront]
// Pipeline (stage s = K range [64 s, 64 s + 64), scale block s / 2):
//   prologue: DMA stages 0..3; wait stage 0; fragments of stage 0 -> registers
//   iteration s: wait until stage s+1 landed (s+2, s+3 may still fly) and
//     this wavefront's reads of stage s finished, barrier (publishes s+1 and
//     frees buffer s, whose fragments now sit in registers), DMA stage s+4
//     into it, then the MFMAs of stage s interleaved with the LDS reads of
//     the stage s+1 fragments.  Three stages (96 KB for a 256x256 tile) stay
//     in flight per CU, which is what covers the L2/MALL latency.
template <int BM, int BN, int WM, int WN, bool kUe8m0, bool kGrouped>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_bs_kernel(const GemmArgs a) {
    constexpr int kWaves = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;   // wavefront tile
    constexpr int FM = TM / 32, FN = TN / 32;   // 32x32 fragments per wavefront
    static_assert(kWaves == 4, "four wavefronts");
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "fragment tiling");
    static_assert(BM % 64 == 0 && BN % 64 == 0 && BM <= 256, "DMA tiling");
    static_assert(128 % TN == 0 || TN % 128 == 0, "wave N tile must not straddle a scale block");
    constexpr int kA = BM * kKS, kB = BN * kKS, kSA = kWaves * 256, kSW = kWaves * 256;
    constexpr int kStage = kA + kB + kSA + kSW;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStage];
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)smem);

    int tm, tn;
    tile_coords(a.tiles_m, a.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int KS = a.K / kKS;                    // stages
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

    const v4i dA = make_desc(a.A + (int64_t)m0 * a.lda, (int64_t)(a.M - m0 - 1) * a.lda + a.K);
    const v4i dW = make_desc(Wbase + (int64_t)n0 * a.ldw, (int64_t)(a.N - n0 - 1) * a.ldw + a.K);
    const v4i dSA = make_desc(a.sA, a.sA_bytes);
    const v4i dSW = make_desc(sWbase, (int64_t)NB * a.sW_ld * 4);

    // DMA lane mapping: one instruction = 16 rows x 64 B; lane i fills LDS
    // slot i%4 of row r0 + i/4 with global chunk (i%4) ^ swz(row), and since
    // r0 is a multiple of 16, swz(row) = i/16.
    const int drow = lane >> 2;
    const int dchunk = ((lane & 3) ^ (lane >> 4)) << 4;
    const int a_lane = (int)(drow * a.lda) + dchunk;
    const int w_lane = (int)(drow * a.ldw) + dchunk;
    constexpr int kAInstr = BM / 16 / kWaves, kBInstr = BN / 16 / kWaves;  // 16-row DMAs per wave
    const int a_wave = (int)(wave * kAInstr * 16 * a.lda);
    const int w_wave = (int)(wave * kBInstr * 16 * a.ldw);
    constexpr int kScaleInstr = BM / 64;                              // 64 scale rows per dword DMA
    const int sa_row = wave * 64 + lane;
    const bool sa_live = (wave < kScaleInstr) & (m0 + sa_row < a.M);  // rows past BM land in unused slots
    const int sa_off0 = sa_live ? (int)((int64_t)(m0 + sa_row) * a.sA_sm * 4) : kOob;
    const int sa_kstep = sa_live ? (int)(a.sA_sk * 4) : 0;
    const bool sw_live = (lane < (BN + 127) / 128) & (n0 / 128 + lane < NB);
    const int sw_off0 = sw_live ? (n0 / 128 + lane) * (int)a.sW_ld * 4 : kOob;
    const int sw_kstep = sw_live ? 4 : 0;
    constexpr int kDmaPerStage = kAInstr + kBInstr + 2;  // per wave

    // Stage s -> LDS buffer s % kStages.  `live` false turns every load into
    // an out-of-range (zero) read, so the loop never branches around it.
    auto issue_stage = [&](int s, bool live) {
        const uint32_t base = lds0 + (s % kStages) * kStage;
        const int k0 = s * kKS, kb = s >> 1;
#pragma unroll
        for (int i = 0; i < kAInstr; ++i)
            dma_b128(dA, base + (wave * kAInstr + i) * 16 * 64,
                     live ? a_lane + a_wave + (int)(i * 16 * a.lda) + k0 : kOob);
#pragma unroll
        for (int i = 0; i < kBInstr; ++i)
            dma_b128(dW, base + kA + (wave * kBInstr + i) * 16 * 64,
                     live ? w_lane + w_wave + (int)(i * 16 * a.ldw) + k0 : kOob);
        dma_b32(dSA, base + kA + kB + wave * 256, live ? sa_off0 + kb * sa_kstep : kOob);
        dma_b32(dSW, base + kA + kB + kSA + wave * 256, live ? sw_off0 + kb * sw_kstep : kOob);
    };

    const int nb_local = (wn * TN) / 128;  // this wavefront's weight-scale block within the tile

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    // Fragment / scale register sets for two consecutive stages (ping-pong:
    // the loop below is unrolled by two stages so no set is ever copied).
    v8i fa0[FM], fb0[FN], fa1[FM], fb1[FN];
    float sa0[FM], sa1[FM];
    float sw0 = 0.f, sw1 = 0.f;
    float sa_row_scale[kUe8m0 ? 1 : FM][kUe8m0 ? 1 : 16];
    float swv = 0.f;

    auto stage_ptr = [&](int s) -> const uint8_t* { return smem + (s % kStages) * kStage; };
    auto read_frags = [&](const uint8_t* st, v8i (&af)[FM], v8i (&bf)[FN]) {
        const int c0 = (lane >> 5) * 2;
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = lds_frag(st, wm * TM + i * 32 + (lane & 31), c0);
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[j] = lds_frag(st + kA, wn * TN + j * 32 + (lane & 31), c0);
    };
    // raw fp32 scales of a stage (converted to E8M0 only when consumed, so no
    // LDS wait lands in the middle of the MFMA stream)
    auto read_scales = [&](const uint8_t* st, float (&sa)[FM], float& sw) {
        const float* ssa = reinterpret_cast<const float*>(st + kA + kB);
        const float* ssw = reinterpret_cast<const float*>(st + kA + kB + kSA + wave * 256);
#pragma unroll
        for (int i = 0; i < FM; ++i) sa[i] = ssa[wm * TM + i * 32 + (lane & 31)];
        sw = ssw[nb_local];
    };
    auto read_fp32_scales = [&](const uint8_t* st) {
        // output row of accumulator register r: 8*(r/4) + 4*(lane/32) + r%4
        const float* ssa = reinterpret_cast<const float*>(st + kA + kB);
        const float* ssw = reinterpret_cast<const float*>(st + kA + kB + kSA + wave * 256);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                sa_row_scale[i][r] = ssa[wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
        swv = ssw[nb_local];
    };

    v16f part[kUe8m0 ? 1 : FM][kUe8m0 ? 1 : FN];
    // One stage: publish stage s+1, refill buffer s with stage s+4, then the
    // MFMAs of stage s (operands in fa/fb/sa/sw) interleaved with the LDS reads
    // of stage s+1 into na/nb/nsa/nsw.
    auto stage = [&](int s, v8i (&fa)[FM], v8i (&fb)[FN], float (&sa)[FM], float& sw, v8i (&na)[FM],
                     v8i (&nb)[FN], float (&nsa)[FM], float& nsw) {
        wait_dma_n<2 * kDmaPerStage>();   // stage s+1 landed
        wait_lds();                        // this wavefront's reads of stage s are done
        __syncthreads();
        issue_stage(s + 4, s + 4 < KS);
        const uint8_t* nxt = stage_ptr(s + 1);
        read_scales(nxt, nsa, nsw);
        read_frags(nxt, na, nb);
        if constexpr (kUe8m0) {
            int ea[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) ea[i] = ue8m0_ceil_byte(sa[i]);
            const int eb = ue8m0_ceil_byte(sw);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0, 0,
                                                                                ea[i], 0, eb);
        } else {
            // the promotion at the end of odd stage s+1 uses its block's
            // scales; read them now, while buffer s+1 is guaranteed intact
            if ((s & 1) == 0) read_fp32_scales(nxt);
            const bool first_half = (s & 1) == 0;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fa[i], fb[j], first_half ? v16f{} : part[i][j], 0, 0, 0, 0, 0, 0);
            if (!first_half) {
                // promotion after both halves of the scale block:
                // acc += part * sA[row] * sW[block]
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float f = sa_row_scale[i][r] * swv;
#pragma unroll
                        for (int j = 0; j < FN; ++j) acc[i][j][r] = fmaf(part[i][j][r], f, acc[i][j][r]);
                    }
            }
        }
        // Interleave the stage-s MFMAs with the LDS reads of stage s+1 (two
        // 16-B reads between consecutive MFMAs) so the reads complete under
        // the matrix pipe.
#pragma unroll
        for (int i = 0; i < FM * FN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two LDS reads
        }
    };

    // prologue
    issue_stage(0, true);
    issue_stage(1, KS > 1);
    issue_stage(2, KS > 2);
    issue_stage(3, KS > 3);
    wait_dma_n<3 * kDmaPerStage>();
    __syncthreads();
    read_scales(stage_ptr(0), sa0, sw0);
    read_frags(stage_ptr(0), fa0, fb0);

    // KS is even (K is a multiple of 128)
    for (int s = 0; s < KS; s += 2) {
        stage(s, fa0, fb0, sa0, sw0, fa1, fb1, sa1, sw1);
        stage(s + 1, fa1, fb1, sa1, sw1, fa0, fb0, sa0, sw0);
    }

    // epilogue: fp32 -> bf16 (RNE), masked 2-byte stores
    const int ncol_base = n0 + wn * TN;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= a.M) continue;
            if constexpr (kGrouped) {
                if (a.expert_ids[m] != expert) continue;
            }
            uint16_t* drow = a.D + (int64_t)m * a.ldd;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int n = ncol_base + j * 32 + (lane & 31);
                if (n < a.N) drow[n] = (uint16_t)f32_to_bf16_rne(acc[i][j][r]);
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool kUe8m0, bool kGrouped>
static int launch_gemm(GemmArgs a, hipStream_t st, const char* what) {
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n;
    KBN_CHECK_ARG(blocks <= 0x7FFFFFFFLL, "%s: too many tiles", what);
    gemm_bs_kernel<BM, BN, WM, WN, kUe8m0, kGrouped><<<dim3((unsigned)blocks), dim3(64 * WM * WN), 0, st>>>(a);
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
    KBN_CHECK_ARG(lda * 256 + K < 0x7FFFFFFFLL && ldw * 256 + K < 0x7FFFFFFFLL, "%s: leading dimension too large",
                  what);
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

extern "C" int kbn_fp8_gemm_nt(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                               int64_t sA_stride_k, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                               void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K, int scale_ue8m0,
                               void* stream) {
    const char* what = "fp8_gemm_nt";
    if (int rc = check_common(what, A, lda, W, ldw, D_bf16, ldd, M, N, K)) return rc;
    if (M == 0 || N == 0) return 0;
    KBN_CHECK_ARG(K > 0, "%s: K must be positive", what);
    KBN_CHECK_ARG(sA && sW, "%s: null scale pointer", what);
    KBN_CHECK_ARG(sW_ld >= K / kGroup, "%s: weight-scale row stride %lld < K/128", what, (long long)sW_ld);
    GemmArgs a{};
    a.A = (const uint8_t*)A; a.lda = lda;
    if (int rc = check_scale_ranges(what, M, K, sA_stride_m, sA_stride_k, (N + kGroup - 1) / kGroup, sW_ld))
        return rc;
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
    a.sA_bytes = scale_bytes(M, K / kGroup, sA_stride_m, sA_stride_k);
    a.W = (const uint8_t*)W; a.ldw = ldw; a.w_estride = 0;
    a.sW = sW; a.sW_ld = sW_ld; a.sW_estride = 0;
    a.D = (uint16_t*)D_bf16; a.ldd = ldd;
    a.expert_ids = nullptr;
    a.M = (int)M; a.N = (int)N; a.K = (int)K; a.E = 1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (scale_ue8m0) {
        if (M > 128) return launch_gemm<256, 256, 2, 2, true, false>(a, st, what);
        return launch_gemm<128, 128, 2, 2, true, false>(a, st, what);
    }
    return launch_gemm<128, 128, 2, 2, false, false>(a, st, what);
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
    a.expert_ids = expert_ids;
    KBN_CHECK_ARG(E <= 0x7FFFFFFFLL, "%s: too many experts", what);
    a.M = (int)M_sum; a.N = (int)N; a.K = (int)K; a.E = (int)E;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (scale_ue8m0) return launch_gemm<128, 256, 2, 2, true, true>(a, st, what);
    return launch_gemm<128, 128, 2, 2, false, true>(a, st, what);
}
