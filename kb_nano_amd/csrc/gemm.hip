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
//   HBM --buffer_load_dwordx4 ... lds (direct DMA)--> LDS (2 stages x (BM+BN) x 128 B)
//   LDS --ds_read_b128--> VGPR fragments --MFMA 32x32x64--> fp32 accumulators
// Each LDS row is 128 B (one 128-K stage); its eight 16-B chunks are XOR-
// swizzled by (row & 7) so the 32 rows read by one ds_read_b128 hit distinct
// banks.  The swizzle is applied on the global side of the DMA (lane i of a
// load instruction always writes LDS chunk i), so no extra LDS pass is needed.
// Out-of-range rows read as zero through the buffer descriptor's range check.

#include "kbn_common.h"

namespace kbn {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;           // K per stage == scale block
constexpr int kThreads = 256;      // 4 wavefronts
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dword format (gfx9 family)

struct GemmArgs {
    const uint8_t* A;
    int64_t lda;
    const float* sA;
    int64_t sA_sm, sA_sk;
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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    uint32_t n = bytes <= 0 ? 0u : (bytes >= 0xFFFFFFFFLL ? 0xFFFFFFFFu : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, (int)kRsrcWord3);
}

// One DMA instruction: 64 lanes x 16 B = 8 rows x 128 B into LDS at `lds`
// (wave-uniform).  Lane i fills LDS chunk i: row r0 + i/8, slot i%8, which
// holds global chunk (slot ^ (row & 7)) of that row.
__device__ __forceinline__ void dma_rows8(__amdgpu_buffer_rsrc_t rsrc, int64_t ld, int r0, int k0, uint8_t* lds,
                                          int lane) {
    const int r = r0 + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    const int voff = (int)(r * ld) + k0 + c * 16;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// 32 bytes of K (chunks c0, c0+1) of LDS row `r` as one MFMA operand.
__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int r, int c0) {
    const v4i lo = *reinterpret_cast<const v4i*>(tile + r * 128 + ((c0 ^ (r & 7)) << 4));
    const v4i hi = *reinterpret_cast<const v4i*>(tile + r * 128 + (((c0 + 1) ^ (r & 7)) << 4));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

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

template <int BM, int BN, int WM, int WN, bool kUe8m0, bool kGrouped>
__global__ __launch_bounds__(kThreads, 1) void gemm_bs_kernel(const GemmArgs a) {
    constexpr int TM = BM / WM, TN = BN / WN;   // wavefront tile
    constexpr int FM = TM / 32, FN = TN / 32;   // 32x32 fragments per wavefront
    static_assert(WM * WN == 4, "four wavefronts");
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "fragment tiling");
    static_assert(BM % 32 == 0 && BN % 32 == 0, "DMA covers 8 rows per wave instruction");
    static_assert(128 % TN == 0 || TN % 128 == 0, "wave N tile must not straddle a scale block");
    constexpr int kStageBytes = (BM + BN) * kBK;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStageBytes];

    int tm, tn;
    tile_coords(a.tiles_m, a.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int KB = a.K / kBK;

    const uint8_t* Wbase = a.W;
    const float* sWbase = a.sW;
    int expert = 0;
    if constexpr (kGrouped) {
        expert = a.expert_ids[m0];
        if (expert < 0 || expert >= a.E) return;  // padding block: C rows stay unwritten
        Wbase += (int64_t)expert * a.w_estride;
        sWbase += (int64_t)expert * a.sW_estride;
    }

    const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.A + (int64_t)m0 * a.lda, (int64_t)(a.M - m0 - 1) * a.lda + a.K);
    const __amdgpu_buffer_rsrc_t rW = make_rsrc(Wbase + (int64_t)n0 * a.ldw, (int64_t)(a.N - n0 - 1) * a.ldw + a.K);

    auto issue_stage = [&](int kt, int stage) {
        uint8_t* sa = smem + stage * kStageBytes;
        uint8_t* sb = sa + BM * kBK;
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < BM / 32; ++i) {
            const int r0 = (wave * (BM / 32) + i) * 8;
            dma_rows8(rA, a.lda, r0, k0, sa + r0 * 128, lane);
        }
#pragma unroll
        for (int i = 0; i < BN / 32; ++i) {
            const int r0 = (wave * (BN / 32) + i) * 8;
            dma_rows8(rW, a.ldw, r0, k0, sb + r0 * 128, lane);
        }
    };

    // rows of this lane's A operands and the scale rows they need
    const int arow_base = wm * TM + (lane & 31);
    const int ncol_base = n0 + wn * TN;
    const int64_t sW_row = (int64_t)min(ncol_base / 128, (a.N - 1) / 128) * a.sW_ld;

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    // per-stage scales
    float sa_cur[kUe8m0 ? FM : 1];
    float sw_cur = 0.f;
    auto load_scales_ue8m0 = [&](int kt, float (&sa)[kUe8m0 ? FM : 1], float& sw) {
        if constexpr (kUe8m0) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int m = min(m0 + arow_base + i * 32, a.M - 1);
                sa[i] = a.sA[(int64_t)m * a.sA_sm + (int64_t)kt * a.sA_sk];
            }
            sw = sWbase[sW_row + kt];
        }
    };

    issue_stage(0, 0);
    load_scales_ue8m0(0, sa_cur, sw_cur);

    for (int kt = 0; kt < KB; ++kt) {
        wait_vmem();
        __syncthreads();
        float sa_nxt[kUe8m0 ? FM : 1];
        float sw_nxt = 0.f;
        if (kt + 1 < KB) {
            issue_stage(kt + 1, (kt + 1) & 1);
            load_scales_ue8m0(kt + 1, sa_nxt, sw_nxt);
        }
        const uint8_t* ta = smem + (kt & 1) * kStageBytes;
        const uint8_t* tb = ta + BM * kBK;

        if constexpr (kUe8m0) {
            int ea[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) ea[i] = ue8m0_ceil_byte(sa_cur[i]);
            const int eb = ue8m0_ceil_byte(sw_cur);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int c0 = ks * 4 + (lane >> 5) * 2;
                v8i af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = lds_frag(ta, wm * TM + i * 32 + (lane & 31), c0);
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = lds_frag(tb, wn * TN + j * 32 + (lane & 31), c0);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bf[j], acc[i][j], 0, 0, 0,
                                                                                   ea[i], 0, eb);
            }
        } else {
            v16f part[FM][FN];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int c0 = ks * 4 + (lane >> 5) * 2;
                v8i af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = lds_frag(ta, wm * TM + i * 32 + (lane & 31), c0);
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = lds_frag(tb, wn * TN + j * 32 + (lane & 31), c0);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            af[i], bf[j], ks == 0 ? v16f{} : part[i][j], 0, 0, 0, 0, 0, 0);
            }
            // promotion: acc += part * sA[row] * sW[block]; output row of
            // register r is 8*(r/4) + 4*(lane/32) + r%4 within the fragment
            const float sw = sWbase[sW_row + kt];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = min(m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), a.M - 1);
                    const float f = a.sA[(int64_t)m * a.sA_sm + (int64_t)kt * a.sA_sk] * sw;
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j][r] = fmaf(part[i][j][r], f, acc[i][j][r]);
                }
            }
        }
        if constexpr (kUe8m0) {
            if (kt + 1 < KB) {
#pragma unroll
                for (int i = 0; i < FM; ++i) sa_cur[i] = sa_nxt[i];
                sw_cur = sw_nxt;
            }
        }
    }

    // epilogue: fp32 -> bf16 (RNE), masked 2-byte stores
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
    gemm_bs_kernel<BM, BN, WM, WN, kUe8m0, kGrouped><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(a);
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
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
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
    if (M > 128) return launch_gemm<256, 128, 2, 2, false, false>(a, st, what);
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
    a.sA = sA; a.sA_sm = sA_stride_m; a.sA_sk = sA_stride_k;
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
