// Per-token-group (1x128) FP8 quantization and the fused SiLU*Mul + FP8
// quantization, as persistent gfx950 bandwidth kernels.
//
// Work decomposition (both ops, one kernel template): a 1x128 group is owned
// by 16 lanes of a wavefront, 8 elements (16 bytes of bf16) per lane.  The
// grid is sized to the CU count.  Each of the 8 XCDs owns a contiguous slice
// of rows (a multiple of 32, so every 128-B line of column-major scales is
// written through a single L2), and the XCD's workgroups walk its slice in
// flattened (row, group) order: one pass covers a contiguous range, each
// wavefront loading kUnroll consecutive 1 KB blocks (4 groups) per operand
// before any arithmetic; positions advance by a precomputed quotient and
// remainder, so there is no per-group division.  The absmax of a group is a
// packed 16-bit max over the lane's bf16 magnitudes, then a 4-step DPP max
// over its 16-lane row; with UE8M0 scales the codes come from the packed bf16
// values by the scaled conversion v_cvt_scalef32_pk_fp8_bf16 (no widening to
// fp32, about 3 VALU instructions per element pair fewer), and leave as one
// 8-byte store per lane (non-temporal in the SiLU kernel).
//
// Numerics follow tasks/baseline/L1/fp8_linear.py:195-215 and
// tasks/baseline/L1/silu_mul_quant_fp8.py:51-76:
//   amax = max(max|x|, eps);  s = amax/448 (IEEE divide), rounded up to a
//   power of two for UE8M0;  q = e4m3_rne(clamp(x/s, +-448)).
// x/s is exact when s is a power of two (the scaled conversion, or a multiply
// by 1/s), and a correctly rounded division otherwise.  NaN inputs give the
// code 0xFF (gfx950's NaN) whatever their sign.
//
// SiLU: silu(g) of a bf16 g has only 65,536 possible inputs, so the fused
// kernel reads bf16(silu(g)) (correctly rounded, generated at build time by
// gen_silu_lut.cpp) from a 128 KB table staged in LDS, one table per CU.
// y = bf16(silu * up) is the exact fp32 product rounded once by
// v_cvt_pk_bf16_f32.

#include "kbn_common.h"

#include <algorithm>
#include <mutex>

namespace kbn {

// External linkage: a namespace-scope const is otherwise internal, its
// device symbol stays local in the code object, and the runtime cannot
// resolve it for hipGetSymbolAddress (silu_lut_device below).
extern __device__ const uint16_t kSiluLut[65536];
__device__ const uint16_t kSiluLut[65536] __attribute__((aligned(16))) = {
#include "silu_lut.inc"
};

typedef short s16x2 __attribute__((ext_vector_type(2)));

// Launch shape (tunable at build time; defaults are the measured best on MI355X).
#ifndef KBN_QUANT_PER_CU
#define KBN_QUANT_PER_CU 2
#endif
constexpr int kThreads = 1024;       // 16 wavefronts
// 4-group blocks per wavefront per pass (per operand): the SiLU kernel runs
// one workgroup per CU (its LDS table), so it takes more blocks per pass to
// keep as many bytes in flight (measured at cfg2: 4 -> 129 us, 2 -> 132 us,
// 5..8 -> 136-140 us; the quant kernel is best at 2).  The row-skipping
// mode is best at 4 as well (cfg4 layout: 88 us against 90-92 us at 6 and 8).
template <bool kSilu>
constexpr int kUnrollOf = kSilu ? 4 : 2;
constexpr int kXcds = 8;             // MI355X: workgroups are dealt round-robin to 8 XCDs
constexpr int kLineRows = 32;        // rows sharing one 128-B line of column-major scales

struct QuantArgs {
    const uint16_t* x;      // input rows: bf16 (fp16 or fp32 for the plain quant's kIn)
    int64_t ld_x;           // row stride (elements)
    int64_t up_off;         // SiLU kernel: column offset of the up half
    uint8_t* q;
    int64_t ld_q;
    float* s;
    int64_t s_sm, s_sg;
    int M, G;
    int rows_per_xcd;       // contiguous rows owned by one XCD (multiple of kLineRows)
    int step_q, step_r;     // per-pass stride inside an XCD's rows, as (rows, groups)
    float eps;
    // optional per-row ids (nullptr: every row): rows whose id is negative
    // (the padding rows of the contiguous MoE layout) are neither read nor
    // written
    const int32_t* row_ids;
};

// Position of a lane's group in the (row, group) space.
struct GroupCursor {
    int row, g;
    __device__ __forceinline__ void advance(int q, int r, int G) {
        g += r;
        row += q;
        if (g >= G) {
            g -= G;
            row += 1;
        }
    }
    __device__ __forceinline__ void step4(int G) {  // next block of 4 groups
        g += 4;
        while (g >= G) {
            g -= G;
            row += 1;
        }
    }
};

// Input element types of the plain quant (the reference's Triton kernel loads
// any float input and widens it to fp32, tasks/baseline/L1/fp8_linear.py:197).
enum QuantIn : int { kInBf16 = 0, kInF16 = 1, kInF32 = 2 };

// The 8 values of this lane as fp32 (exact widening): from four words of
// fp16 pairs, or from two 16-B chunks of fp32.
__device__ __forceinline__ void widen_f16(const u32x4& x, float (&v)[8]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 h = __builtin_bit_cast(h2, w[i]);
        v[2 * i] = (float)h.x;
        v[2 * i + 1] = (float)h.y;
    }
}
__device__ __forceinline__ void widen_f32(const u32x4& x0, const u32x4& x1, float (&v)[8]) {
    v[0] = __uint_as_float(x0.x); v[1] = __uint_as_float(x0.y);
    v[2] = __uint_as_float(x0.z); v[3] = __uint_as_float(x0.w);
    v[4] = __uint_as_float(x1.x); v[5] = __uint_as_float(x1.y);
    v[6] = __uint_as_float(x1.z); v[7] = __uint_as_float(x1.w);
}

// Quantize 8 fp32 values of this lane (16 lanes per group), the fp16 and
// fp32 inputs' path: the bf16 general path above on the widened values.
// The absmax ignores NaN (fmaxf), an infinity gives an infinite scale;
// UE8M0 codes are x times the exact reciprocal of the power-of-two scale
// (x / s exactly, but where it falls below fp32's normal range, far under
// e4m3's smallest subnormal, so the code is the same), FP32-contract codes
// the correctly rounded x / s, both converted by the hardware RNE.
template <bool kUe8m0>
__device__ __forceinline__ float quant8f_store(const float (&v)[8], float eps, int sub, uint8_t* __restrict__ qptr) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
    amax = fmaxf(amax, eps);
    const float sc = kUe8m0 ? ue8m0_ceil_div448(amax) : amax / kFp8Max;
    uint32_t lo, hi;
    if constexpr (kUe8m0) {
        lo = pack4_e4m3_ue8m0_general(v[0], v[1], v[2], v[3], sc);
        hi = pack4_e4m3_ue8m0_general(v[4], v[5], v[6], v[7], sc);
    } else {
        lo = pack4_e4m3(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
        hi = pack4_e4m3(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
    }
    *reinterpret_cast<u32x2*>(qptr + sub * 8) = u32x2{lo, hi};
    return sc;
}

// One persistent kernel for both ops.  Each XCD owns a contiguous slice of
// rows (a multiple of 32, so every 128-B line of column-major scales is
// written through one L2 and merges there); inside the slice the XCD's
// workgroups walk the flattened (row, group) space so that one pass covers a
// contiguous range, each wavefront reading kUnroll consecutive blocks of 4
// groups (1 KB of bf16 per operand and block) before any arithmetic.
// kRows: rows whose a.row_ids entry is negative are skipped (no loads, no
// stores); the ids are read one pass ahead.  The rows are then dealt to the
// XCDs in blocks of 32 (block b to XCD b % 8) instead of contiguous slices:
// skipped rows cluster (an expert segment's padding, the layout's unused
// tail), and contiguous slices would leave whole XCDs without work.
template <bool kSilu, bool kUe8m0, bool kRows = false, int kIn = kInBf16>
__global__ __launch_bounds__(kThreads) void group_quant_kernel(const QuantArgs a) {
    static_assert(kIn == kInBf16 || (!kSilu && !kRows), "the SiLU and row-skipping kernels take bf16 input");
    constexpr int kEb = kIn == kInF32 ? 4 : 2;   // input bytes per element
    __shared__ __attribute__((aligned(16))) uint16_t lut[kSilu ? 65536 : 8];
    if constexpr (kSilu) {  // stage the bf16 SiLU table: 8192 x 16 B
        const u32x4* src = reinterpret_cast<const u32x4*>(kSiluLut);
        u32x4* dst = reinterpret_cast<u32x4*>(lut);
#pragma unroll
        for (int i = 0; i < 8192 / kThreads; ++i) dst[threadIdx.x + i * kThreads] = src[threadIdx.x + i * kThreads];
        __syncthreads();
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 15;
    const int xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
    // kRows: the cursor walks XCD-local rows [0, rows_per_xcd); local row lr
    // is global row ((lr / 32) * 8 + xcd) * 32 + lr % 32, valid below a.M
    const int row_begin = kRows ? 0 : xcd * a.rows_per_xcd;
    const int row_end = kRows ? a.rows_per_xcd : min(a.M, row_begin + a.rows_per_xcd);
    auto grow = [&](int lr) { return kRows ? (((lr >> 5) * kXcds + xcd) << 5) + (lr & 31) : lr; };
    constexpr int kUnroll = kUnrollOf<kSilu>;
    const int64_t t0 = ((int64_t)local * (kThreads / 64) + wave) * (4 * kUnroll) + (lane >> 4);
    GroupCursor c{row_begin + (int)(t0 / a.G), (int)(t0 % a.G)};
    // kRows: the row ids of the groups of the next pass, loaded one pass
    // ahead (an id below zero skips the group: no loads, no stores)
    int rid[kRows ? kUnroll : 1];
    if constexpr (kRows) {
        GroupCursor cn = c;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int r = grow(cn.row);
            rid[u] = cn.row < row_end && r < a.M ? a.row_ids[r] : -1;
            cn.step4(a.G);
        }
    }
    while (c.row < row_end) {
        GroupCursor cu[kUnroll];
        cu[0] = c;
#pragma unroll
        for (int u = 1; u < kUnroll; ++u) {
            cu[u] = cu[u - 1];
            cu[u].step4(a.G);
        }
        bool skip[kRows ? kUnroll : 1];   // kRows: this pass's groups of skipped rows
        if constexpr (kRows) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) skip[u] = rid[u] < 0;
        }
        u32x4 xa[kUnroll], xb[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            if (cu[u].row < row_end && !(kRows && skip[kRows ? u : 0])) {
                if constexpr (kIn == kInBf16) {
                    const uint16_t* p = a.x + (int64_t)grow(cu[u].row) * a.ld_x + (int64_t)cu[u].g * kGroup + sub * 8;
                    xa[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
                    if constexpr (kSilu) xb[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + a.up_off));
                } else {
                    // fp16: 16 B, fp32: 32 B (two chunks) per lane
                    const uint8_t* p = reinterpret_cast<const uint8_t*>(a.x) +
                                       ((int64_t)cu[u].row * a.ld_x + (int64_t)cu[u].g * kGroup + sub * 8) * kEb;
                    xa[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
                    if constexpr (kIn == kInF32) xb[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 16));
                }
            }
        c.advance(a.step_q, a.step_r, a.G);
        if constexpr (kRows) {
            GroupCursor cn = c;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int r = grow(cn.row);
                rid[u] = cn.row < row_end && r < a.M ? a.row_ids[r] : -1;
                cn.step4(a.G);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (cu[u].row >= row_end) break;  // uniform over the group's 16 lanes; rows grow with u
            if constexpr (kRows)
                if (skip[u]) continue;        // a skipped row (uniform over the group's lanes)
            if constexpr (kIn != kInBf16) {
                float v[8];
                if constexpr (kIn == kInF16) widen_f16(xa[u], v);
                else widen_f32(xa[u], xb[u], v);
                const int64_t r = cu[u].row;
                const float sc = quant8f_store<kUe8m0>(v, a.eps, sub, a.q + r * a.ld_q + (int64_t)cu[u].g * kGroup);
                if (sub == 0) a.s[r * a.s_sm + (int64_t)cu[u].g * a.s_sg] = sc;
                continue;
            }
            uint32_t w[4];
            if constexpr (kSilu) {
                w[0] = silu_mul_pair(lut, xa[u].x, xb[u].x);
                w[1] = silu_mul_pair(lut, xa[u].y, xb[u].y);
                w[2] = silu_mul_pair(lut, xa[u].z, xb[u].z);
                w[3] = silu_mul_pair(lut, xa[u].w, xb[u].w);
            } else {
                w[0] = xa[u].x; w[1] = xa[u].y; w[2] = xa[u].z; w[3] = xa[u].w;
            }
            const int64_t r = grow(cu[u].row);
            const float sc = quant8_store<kUe8m0, kSilu>(w, a.eps, sub, a.q + r * a.ld_q + (int64_t)cu[u].g * kGroup);
            if (sub == 0) a.s[r * a.s_sm + (int64_t)cu[u].g * a.s_sg] = sc;
        }
    }
}

const uint16_t* silu_lut_device(const char* what) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static const uint16_t* ptr[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        set_error("%s: no current HIP device (or device index >= %d)", what, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(kSiluLut));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            set_error("%s: hipGetSymbolAddress(kSiluLut) failed on device %d: %s", what, dev, hipGetErrorString(e));
            return nullptr;
        }
        ptr[dev] = static_cast<const uint16_t*>(p);
    }
    return ptr[dev];
}

// path 0: the table read directly; path 1: the table at the device address
// that hipGetSymbolAddress gives (the grouped GEMM's SiLU*Mul epilogue reads
// it there)
__global__ void silu_bf16_debug_kernel(const uint16_t* __restrict__ g, uint16_t* __restrict__ out, int64_t n,
                                       const uint16_t* __restrict__ lut, int path) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = path ? lut[g[i]] : kSiluLut[g[i]];
}


// Row slices per XCD (multiples of 32 rows) and the number of workgroups
// per XCD: at most `per_cu` per CU, never more than the slice needs.
static int plan(QuantArgs& a, int per_cu, int unroll) {
    const int slice = (a.M + kXcds - 1) / kXcds;
    a.rows_per_xcd = (slice + kLineRows - 1) / kLineRows * kLineRows;
    const int64_t per_block = (int64_t)(kThreads / 64) * 4 * unroll;  // groups per workgroup pass
    const int64_t need = ((int64_t)a.rows_per_xcd * a.G + per_block - 1) / per_block;
    const int per_xcd = (int)std::max<int64_t>(1, std::min<int64_t>(need, (int64_t)cu_count() / kXcds * per_cu));
    const int64_t stride = (int64_t)per_xcd * per_block;
    a.step_q = (int)(stride / a.G);
    a.step_r = (int)(stride % a.G);
    return per_xcd * kXcds;
}

}  // namespace kbn

using namespace kbn;

static int check_quant_args(const char* what, const void* x, int64_t M, int64_t K, int64_t ld_x, const void* q,
                            int64_t ld_q, const float* s) {
    KBN_CHECK_ARG(M >= 0 && K >= 0, "%s: negative shape M=%lld K=%lld", what, (long long)M, (long long)K);
    KBN_CHECK_ARG(K % kGroup == 0, "%s: K=%lld must be a multiple of 128", what, (long long)K);
    if (M == 0 || K == 0) return 0;
    KBN_CHECK_ARG(x && q && s, "%s: null pointer", what);
    KBN_CHECK_ARG(ld_q >= K, "%s: output row stride smaller than the row", what);
    KBN_CHECK_ARG(aligned16(x) && ld_x % 8 == 0, "%s: input rows must be 16-byte aligned (row stride %% 8 == 0)",
                  what);
    KBN_CHECK_ARG((reinterpret_cast<uintptr_t>(q) & 7u) == 0 && ld_q % 8 == 0,
                  "%s: output rows must be 8-byte aligned", what);
    KBN_CHECK_ARG(M <= 0x3FFFFFFFLL && K / kGroup <= 0x3FFFFFFFLL, "%s: shape too large", what);
    return 0;
}

static int quant_typed(const char* what, const void* x, int x_dtype, int64_t M, int64_t K, int64_t ld_x,
                       void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g, float eps,
                       int use_ue8m0, void* stream) {
    KBN_CHECK_ARG(x_dtype == kInBf16 || x_dtype == kInF16 || x_dtype == kInF32,
                  "%s: input dtype code %d (0 bf16, 1 fp16, 2 fp32)", what, x_dtype);
    if (int rc = check_quant_args(what, x, M, K, ld_x, q_fp8, ld_q, scale)) return rc;
    if (M == 0 || K == 0) return 0;
    KBN_CHECK_ARG(ld_x >= K, "%s: input row stride smaller than K", what);
    QuantArgs a{(const uint16_t*)x, ld_x, 0, (uint8_t*)q_fp8, ld_q, scale, s_stride_m, s_stride_g,
                (int)M, (int)(K / kGroup), 0, 0, 0, eps};
    const int blocks = plan(a, KBN_QUANT_PER_CU, kUnrollOf<false>);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (x_dtype == kInBf16) {
        if (use_ue8m0) group_quant_kernel<false, true><<<blocks, kThreads, 0, st>>>(a);
        else group_quant_kernel<false, false><<<blocks, kThreads, 0, st>>>(a);
    } else if (x_dtype == kInF16) {
        if (use_ue8m0) group_quant_kernel<false, true, false, kInF16><<<blocks, kThreads, 0, st>>>(a);
        else group_quant_kernel<false, false, false, kInF16><<<blocks, kThreads, 0, st>>>(a);
    } else {
        if (use_ue8m0) group_quant_kernel<false, true, false, kInF32><<<blocks, kThreads, 0, st>>>(a);
        else group_quant_kernel<false, false, false, kInF32><<<blocks, kThreads, 0, st>>>(a);
    }
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_per_token_group_quant_fp8(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x,
                                             void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                                             int64_t s_stride_g, float eps, int use_ue8m0, void* stream) {
    return quant_typed("per_token_group_quant_fp8", x_bf16, kInBf16, M, K, ld_x, q_fp8, ld_q, scale, s_stride_m,
                       s_stride_g, eps, use_ue8m0, stream);
}

extern "C" int kbn_per_token_group_quant_fp8_typed(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ld_x,
                                                   void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                                                   int64_t s_stride_g, float eps, int use_ue8m0, void* stream) {
    return quant_typed("per_token_group_quant_fp8_typed", x, x_dtype, M, K, ld_x, q_fp8, ld_q, scale, s_stride_m,
                       s_stride_g, eps, use_ue8m0, stream);
}

extern "C" int kbn_silu_mul_quant_fp8(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in, void* q_fp8,
                                      int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g, float eps,
                                      int use_ue8m0, void* stream) {
    const char* what = "silu_mul_quant_fp8";
    if (int rc = check_quant_args(what, in_bf16, M, N_half, ld_in, q_fp8, ld_q, scale)) return rc;
    if (M == 0 || N_half == 0) return 0;
    KBN_CHECK_ARG(ld_in >= 2 * N_half, "%s: input row stride smaller than 2*N/2", what);
    QuantArgs a{(const uint16_t*)in_bf16, ld_in, N_half, (uint8_t*)q_fp8, ld_q, scale, s_stride_m, s_stride_g,
                (int)M, (int)(N_half / kGroup), 0, 0, 0, eps};
    const int blocks = plan(a, 1, kUnrollOf<true>);  // the LDS table allows one workgroup per CU
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        group_quant_kernel<true, true><<<blocks, kThreads, 0, st>>>(a);
    else
        group_quant_kernel<true, false><<<blocks, kThreads, 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_silu_mul_quant_fp8_rows(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in,
                                           void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                                           int64_t s_stride_g, float eps, int use_ue8m0, const int32_t* row_ids,
                                           void* stream) {
    const char* what = "silu_mul_quant_fp8_rows";
    if (int rc = check_quant_args(what, in_bf16, M, N_half, ld_in, q_fp8, ld_q, scale)) return rc;
    if (M == 0 || N_half == 0) return 0;
    KBN_CHECK_ARG(ld_in >= 2 * N_half, "%s: input row stride smaller than 2*N/2", what);
    KBN_CHECK_ARG(row_ids, "%s: null row ids", what);
    QuantArgs a{(const uint16_t*)in_bf16, ld_in, N_half, (uint8_t*)q_fp8, ld_q, scale, s_stride_m, s_stride_g,
                (int)M, (int)(N_half / kGroup), 0, 0, 0, eps, row_ids};
    const int blocks = plan(a, 1, kUnrollOf<true>);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        group_quant_kernel<true, true, true><<<blocks, kThreads, 0, st>>>(a);
    else
        group_quant_kernel<true, false, true><<<blocks, kThreads, 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_debug_silu_bf16(const uint16_t* g_bf16, uint16_t* out_bf16, int64_t n, int path, void* stream) {
    KBN_CHECK_ARG(n >= 0 && n <= 0x7FFFFFFFLL, "debug_silu_bf16: bad n");
    KBN_CHECK_ARG(path == 0 || path == 1, "debug_silu_bf16: path must be 0 (the table) or 1 (its symbol address)");
    if (n == 0) return 0;
    KBN_CHECK_ARG(g_bf16 && out_bf16, "debug_silu_bf16: null pointer");
    const uint16_t* lut = silu_lut_device("debug_silu_bf16");
    if (!lut) return 1;
    silu_bf16_debug_kernel<<<(unsigned)((n + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        g_bf16, out_bf16, n, lut, path);
    KBN_CHECK_LAUNCH("debug_silu_bf16");
    return 0;
}
