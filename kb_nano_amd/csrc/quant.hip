// Per-token-group (1x128) FP8 quantization and the fused SiLU*Mul + FP8
// quantization, as persistent gfx950 bandwidth kernels.
//
// Work decomposition (both kernels): a 1x128 group is owned by 16 lanes of a
// wavefront, 8 elements (16 bytes of bf16) per lane; one wavefront covers 4
// groups per pass and every lane carries kUnroll groups, all loads issued
// before any arithmetic.  The grid is sized to the CU count and each
// workgroup strides over the flattened (row, group) space; the (row, group)
// position advances by a precomputed quotient/remainder, so there is no
// per-group integer division.  The absmax of a group is a 4-step DPP max over
// its 16-lane row; codes leave as one 8-byte non-temporal store per lane.
//
// Numerics follow tasks/baseline/L1/fp8_linear.py:195-215 and
// tasks/baseline/L1/silu_mul_quant_fp8.py:51-76:
//   amax = max(max|x|, eps);  s = amax/448 (IEEE divide), rounded up to a
//   power of two for UE8M0;  q = e4m3_rne(clamp(x/s, +-448)).
// x/s is an exact multiply by 1/s when s is a power of two, and a correctly
// rounded division otherwise.
//
// SiLU: silu(g) of a bf16 g has only 65,536 possible inputs, so the fused
// kernel reads bf16(silu(g)) (correctly rounded, generated at build time by
// gen_silu_lut.cpp) from a 128 KB table staged in LDS, one table per CU.
// y = bf16(silu * up) is the exact fp32 product rounded once by
// v_cvt_pk_bf16_f32.

#include "kbn_common.h"

#include <algorithm>

namespace kbn {

__device__ const uint16_t kSiluLut[65536] __attribute__((aligned(16))) = {
#include "silu_lut.inc"
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kUnroll = 4;           // groups per lane per pass
constexpr int kQuantThreads = 512;
constexpr int kSiluThreads = 1024;   // one workgroup per CU (the table fills 128 KB of LDS)

// Position of a lane's group in the flattened (row, group) space.
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
};

template <bool kUe8m0>
__device__ __forceinline__ void quant8_store(const float (&v)[8], float eps, int sub, uint8_t* __restrict__ qptr,
                                             float* __restrict__ sptr) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
    amax = fmaxf(amax, eps);
    float sc = amax / kFp8Max;
    uint32_t lo, hi;
    if (kUe8m0) {
        sc = ue8m0_ceil(sc);
        const float inv = pow2_recip(sc);
        lo = pack4_e4m3(clamp_fp8(v[0] * inv), clamp_fp8(v[1] * inv), clamp_fp8(v[2] * inv), clamp_fp8(v[3] * inv));
        hi = pack4_e4m3(clamp_fp8(v[4] * inv), clamp_fp8(v[5] * inv), clamp_fp8(v[6] * inv), clamp_fp8(v[7] * inv));
    } else {
        lo = pack4_e4m3(clamp_fp8(v[0] / sc), clamp_fp8(v[1] / sc), clamp_fp8(v[2] / sc), clamp_fp8(v[3] / sc));
        hi = pack4_e4m3(clamp_fp8(v[4] / sc), clamp_fp8(v[5] / sc), clamp_fp8(v[6] / sc), clamp_fp8(v[7] / sc));
    }
    __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(qptr + sub * 8));
    if (sub == 0) *sptr = sc;
}

struct QuantArgs {
    const uint16_t* x;      // bf16 input rows
    int64_t ld_x;           // row stride (elements)
    int64_t up_off;         // SiLU kernel: column offset of the up half
    uint8_t* q;
    int64_t ld_q;
    float* s;
    int64_t s_sm, s_sg;
    int M, G;
    int step_q, step_r;     // stride over the flattened group space as (rows, groups)
    float eps;
};

template <bool kUe8m0>
__global__ __launch_bounds__(kQuantThreads) void quant_group128_kernel(const QuantArgs a) {
    const int sub = threadIdx.x & 15;
    constexpr int kSlots = kQuantThreads / 16;
    const int64_t gid0 = (int64_t)blockIdx.x * kSlots + (threadIdx.x >> 4);
    GroupCursor c{(int)(gid0 / a.G), (int)(gid0 % a.G)};
    while (c.row < a.M) {
        u32x4 raw[kUnroll];
        GroupCursor cu[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            cu[u] = c;
            if (c.row < a.M)
                raw[u] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(a.x + (int64_t)c.row * a.ld_x + c.g * kGroup + sub * 8));
            c.advance(a.step_q, a.step_r, a.G);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (cu[u].row >= a.M) break;  // uniform over the group's 16 lanes
            const float v[8] = {bf16lo(raw[u].x), bf16hi(raw[u].x), bf16lo(raw[u].y), bf16hi(raw[u].y),
                                bf16lo(raw[u].z), bf16hi(raw[u].z), bf16lo(raw[u].w), bf16hi(raw[u].w)};
            quant8_store<kUe8m0>(v, a.eps, sub, a.q + (int64_t)cu[u].row * a.ld_q + cu[u].g * kGroup,
                                 a.s + (int64_t)cu[u].row * a.s_sm + (int64_t)cu[u].g * a.s_sg);
        }
    }
}

// bf16(silu(g)) * up for the two bf16 values of each word, rounded to bf16
// by v_cvt_pk_bf16_f32 and widened back to fp32.
__device__ __forceinline__ void silu_mul_pair(const uint16_t* __restrict__ lut, uint32_t gw, uint32_t uw, float& y0,
                                              float& y1) {
    const float s0 = __uint_as_float((uint32_t)lut[gw & 0xFFFFu] << 16);
    const float s1 = __uint_as_float((uint32_t)lut[gw >> 16] << 16);
    const bf16x2 p = __builtin_convertvector((f32x2{s0 * bf16lo(uw), s1 * bf16hi(uw)}), bf16x2);
    const uint32_t pw = __builtin_bit_cast(uint32_t, p);
    y0 = bf16lo(pw);
    y1 = bf16hi(pw);
}

template <bool kUe8m0>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_quant_kernel(const QuantArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lut[65536];
    const int sub = threadIdx.x & 15;
    constexpr int kSlots = kSiluThreads / 16;
    const int64_t gid0 = (int64_t)blockIdx.x * kSlots + (threadIdx.x >> 4);
    GroupCursor c{(int)(gid0 / a.G), (int)(gid0 % a.G)};

    {  // stage the table: 8192 x 16 B
        const u32x4* src = reinterpret_cast<const u32x4*>(kSiluLut);
        u32x4* dst = reinterpret_cast<u32x4*>(lut);
#pragma unroll
        for (int i = 0; i < 8192 / kSiluThreads; ++i) dst[threadIdx.x + i * kSiluThreads] = src[threadIdx.x + i * kSiluThreads];
    }
    __syncthreads();

    while (c.row < a.M) {
        u32x4 graw[kUnroll], uraw[kUnroll];
        GroupCursor cu[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            cu[u] = c;
            if (c.row < a.M) {
                const uint16_t* p = a.x + (int64_t)c.row * a.ld_x + c.g * kGroup + sub * 8;
                graw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
                uraw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + a.up_off));
            }
            c.advance(a.step_q, a.step_r, a.G);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (cu[u].row >= a.M) break;
            float v[8];
            silu_mul_pair(lut, graw[u].x, uraw[u].x, v[0], v[1]);
            silu_mul_pair(lut, graw[u].y, uraw[u].y, v[2], v[3]);
            silu_mul_pair(lut, graw[u].z, uraw[u].z, v[4], v[5]);
            silu_mul_pair(lut, graw[u].w, uraw[u].w, v[6], v[7]);
            quant8_store<kUe8m0>(v, a.eps, sub, a.q + (int64_t)cu[u].row * a.ld_q + cu[u].g * kGroup,
                                 a.s + (int64_t)cu[u].row * a.s_sm + (int64_t)cu[u].g * a.s_sg);
        }
    }
}

__global__ void silu_bf16_debug_kernel(const uint16_t* __restrict__ g, uint16_t* __restrict__ out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = kSiluLut[g[i]];
}

// Compute units of the current device (cached per device).
static int cu_count() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// Grid over the flattened group space: at most `per_cu` workgroups per CU,
// never more than the work needs.
static int plan(QuantArgs& a, int threads, int per_cu) {
    const int64_t total = (int64_t)a.M * a.G;
    const int slots = threads / 16;
    const int64_t need = (total + (int64_t)slots * kUnroll - 1) / ((int64_t)slots * kUnroll);
    int blocks = (int)std::min<int64_t>(need, (int64_t)cu_count() * per_cu);
    if (blocks < 1) blocks = 1;
    const int64_t stride = (int64_t)blocks * slots;
    a.step_q = (int)(stride / a.G);
    a.step_r = (int)(stride % a.G);
    return blocks;
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

extern "C" int kbn_per_token_group_quant_fp8(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x,
                                             void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                                             int64_t s_stride_g, float eps, int use_ue8m0, void* stream) {
    const char* what = "per_token_group_quant_fp8";
    if (int rc = check_quant_args(what, x_bf16, M, K, ld_x, q_fp8, ld_q, scale)) return rc;
    if (M == 0 || K == 0) return 0;
    KBN_CHECK_ARG(ld_x >= K, "%s: input row stride smaller than K", what);
    QuantArgs a{(const uint16_t*)x_bf16, ld_x, 0, (uint8_t*)q_fp8, ld_q, scale, s_stride_m, s_stride_g,
                (int)M, (int)(K / kGroup), 0, 0, eps};
    const int blocks = plan(a, kQuantThreads, 4);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        quant_group128_kernel<true><<<blocks, kQuantThreads, 0, st>>>(a);
    else
        quant_group128_kernel<false><<<blocks, kQuantThreads, 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_silu_mul_quant_fp8(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in, void* q_fp8,
                                      int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g, float eps,
                                      int use_ue8m0, void* stream) {
    const char* what = "silu_mul_quant_fp8";
    if (int rc = check_quant_args(what, in_bf16, M, N_half, ld_in, q_fp8, ld_q, scale)) return rc;
    if (M == 0 || N_half == 0) return 0;
    KBN_CHECK_ARG(ld_in >= 2 * N_half, "%s: input row stride smaller than 2*N/2", what);
    QuantArgs a{(const uint16_t*)in_bf16, ld_in, N_half, (uint8_t*)q_fp8, ld_q, scale, s_stride_m, s_stride_g,
                (int)M, (int)(N_half / kGroup), 0, 0, eps};
    const int blocks = plan(a, kSiluThreads, 1);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        silu_mul_quant_kernel<true><<<blocks, kSiluThreads, 0, st>>>(a);
    else
        silu_mul_quant_kernel<false><<<blocks, kSiluThreads, 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_debug_silu_bf16(const uint16_t* g_bf16, uint16_t* out_bf16, int64_t n, void* stream) {
    KBN_CHECK_ARG(n >= 0 && n <= 0x7FFFFFFFLL, "debug_silu_bf16: bad n");
    if (n == 0) return 0;
    KBN_CHECK_ARG(g_bf16 && out_bf16, "debug_silu_bf16: null pointer");
    silu_bf16_debug_kernel<<<(unsigned)((n + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        g_bf16, out_bf16, n);
    KBN_CHECK_LAUNCH("debug_silu_bf16");
    return 0;
}
