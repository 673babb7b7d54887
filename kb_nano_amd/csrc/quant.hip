// Per-token-group (1x128) FP8 quantization and the fused SiLU*Mul + FP8
// quantization, as gfx950 bandwidth kernels.
//
// Work decomposition (both kernels): a 1x128 group is owned by 16 lanes of
// one wavefront, 8 elements (16 bytes of bf16) per lane, so one wavefront
// quantizes four groups per pass with a single 16-byte load per lane per
// operand, a 4-step DPP max over the 16-lane row, and one 8-byte store of
// packed e4m3 codes per lane.  Each block (256 lanes) covers a run of
// consecutive groups of ONE row: grid.x walks rows, grid.y walks runs of
// 16*kRuns groups, so no integer division happens on the device.
//
// Numerics follow tasks/baseline/L1/fp8_linear.py:195-215 and
// tasks/baseline/L1/silu_mul_quant_fp8.py:51-76:
//   amax = max(max|x|, eps);  s = amax/448 (IEEE divide), rounded up to a
//   power of two for UE8M0;  q = e4m3_rne(clamp(x/s, +-448)).
// x/s is an exact multiply by 1/s when s is a power of two, and a
// correctly rounded division otherwise.

#include "kbn_common.h"

namespace kbn {

// ----------------------------------------------------------------- SiLU ---
//
// silu(g) = g / (1 + e^-g) rounded once to bf16 (correctly rounded: the
// value a 50-digit evaluation rounds to).  Fast path in fp32 with an error
// of a few fp32 ulps; whenever the fp32 result sits within kSiluMargin ulps
// of a bf16 rounding midpoint, or g is outside the fast path's range, the
// value is recomputed in double.  All 65,536 bf16 inputs are checked
// against the oracle by the exhaustive GPU test.

constexpr int kSiluMargin = 24;

// Correctly rounded double -> bf16 bits (one rounding, bf16 subnormals kept).
__device__ __noinline__ uint32_t double_to_bf16_bits(double d) {
    uint32_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e);
    int q = e - 8;
    if (q < -133) q = -133;
    double r = rint(ldexp(a, -q));
    float v = (float)ldexp(r, q);  // exact: at most 8 significant bits
    return sign | (__float_as_uint(v) >> 16);
}

__device__ __noinline__ uint32_t silu_bf16_slow(float gf) {
    double g = (double)gf;
    if (fabs(g) < 0x1p-64) {
        // silu(g) = g/2 * (1 + g/2 + ...): only subnormal g can make g/2 a
        // bf16 tie; the exact value then lies above the tie in magnitude
        // for g > 0 and below it for g < 0.
        double half = g * 0.5;
        uint32_t h = double_to_bf16_bits(half);
        if ((double)__uint_as_float(h << 16) == half) return h;
        double qn = 0x1p-133;
        double lo = floor(fabs(half) / qn) * qn;
        return double_to_bf16_bits(copysign(g > 0 ? lo + qn : lo, g));
    }
    return double_to_bf16_bits(g / (1.0 + exp(-g)));
}

__device__ __forceinline__ uint32_t silu_bf16(float g) {
    // e^-g = 2^(-g*log2 e): carry the rounding error of the product and the
    // tail of log2 e into a first-order correction of the exp2 result.
    const float kL2eHi = 1.44269502162933349609375f;
    const float kL2eLo = 1.925963033500011e-08f;
    float t = -g * kL2eHi;
    float terr = fmaf(-g, kL2eHi, -t);
    terr = fmaf(-g, kL2eLo, terr);
    float e = __builtin_amdgcn_exp2f(t);
    e = fmaf(e, terr * 0.693147180559945309f, e);
    float r = g * __builtin_amdgcn_rcpf(1.0f + e);
    uint32_t u = __float_as_uint(r);
    int low = (int)(u & 0xFFFFu) - 0x8000;
    bool slow = (low <= kSiluMargin && low >= -kSiluMargin) || !(g >= -64.0f) ||
                (fabsf(g) < 0x1p-60f && g != 0.0f);
    if (__builtin_expect(slow, 0)) return silu_bf16_slow(g);
    return f32_to_bf16_rne(r);
}

// ---------------------------------------------------------------- kernels ---

template <bool kUe8m0>
__device__ __forceinline__ void quant8_store(const float (&v)[8], float eps, int sub,
                                             uint8_t* __restrict__ qrow, float* __restrict__ sptr) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
    amax = fmaxf(amax, eps);
    float sc = amax / kFp8Max;
    uint32_t lo, hi;
    if (kUe8m0) {
        sc = ue8m0_ceil(sc);
        float inv = pow2_recip(sc);
        lo = pack4_e4m3(clamp_fp8(v[0] * inv), clamp_fp8(v[1] * inv), clamp_fp8(v[2] * inv), clamp_fp8(v[3] * inv));
        hi = pack4_e4m3(clamp_fp8(v[4] * inv), clamp_fp8(v[5] * inv), clamp_fp8(v[6] * inv), clamp_fp8(v[7] * inv));
    } else {
        lo = pack4_e4m3(clamp_fp8(v[0] / sc), clamp_fp8(v[1] / sc), clamp_fp8(v[2] / sc), clamp_fp8(v[3] / sc));
        hi = pack4_e4m3(clamp_fp8(v[4] / sc), clamp_fp8(v[5] / sc), clamp_fp8(v[6] / sc), clamp_fp8(v[7] / sc));
    }
    *reinterpret_cast<uint2*>(qrow + sub * 8) = make_uint2(lo, hi);
    if (sub == 0) *sptr = sc;
}

template <bool kUe8m0, int kRuns>
__global__ __launch_bounds__(256) void quant_group128_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, uint8_t* __restrict__ q, int64_t ld_q,
    float* __restrict__ s, int64_t s_sm, int64_t s_sg, int G, float eps) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & 15;
    const int slot = (threadIdx.x >> 4);  // group slot within the block pass: 0..15
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * ld_x;
    uint8_t* qr = q + row * ld_q;

    u32x4 raw[kRuns];
    int gidx[kRuns];
#pragma unroll
    for (int it = 0; it < kRuns; ++it) {
        gidx[it] = (blockIdx.y * kRuns + it) * 16 + slot;
        if (gidx[it] < G)
            raw[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + gidx[it] * kGroup + sub * 8));
    }
#pragma unroll
    for (int it = 0; it < kRuns; ++it) {
        if (gidx[it] >= G) continue;  // uniform over the 16 lanes of a group
        float v[8] = {bf16lo(raw[it].x), bf16hi(raw[it].x), bf16lo(raw[it].y), bf16hi(raw[it].y),
                      bf16lo(raw[it].z), bf16hi(raw[it].z), bf16lo(raw[it].w), bf16hi(raw[it].w)};
        quant8_store<kUe8m0>(v, eps, sub, qr + gidx[it] * kGroup, s + row * s_sm + gidx[it] * s_sg);
    }
}

template <bool kUe8m0, int kRuns>
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(
    const uint16_t* __restrict__ in, int64_t ld_in, int64_t n_half, uint8_t* __restrict__ q, int64_t ld_q,
    float* __restrict__ s, int64_t s_sm, int64_t s_sg, int G, float eps) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & 15;
    const int slot = (threadIdx.x >> 4);
    const int64_t row = blockIdx.x;
    const uint16_t* gr = in + row * ld_in;
    const uint16_t* ur = gr + n_half;
    uint8_t* qr = q + row * ld_q;

    u32x4 graw[kRuns], uraw[kRuns];
    int gidx[kRuns];
#pragma unroll
    for (int it = 0; it < kRuns; ++it) {
        gidx[it] = (blockIdx.y * kRuns + it) * 16 + slot;
        if (gidx[it] < G) {
            graw[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gr + gidx[it] * kGroup + sub * 8));
            uraw[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ur + gidx[it] * kGroup + sub * 8));
        }
    }
#pragma unroll
    for (int it = 0; it < kRuns; ++it) {
        if (gidx[it] >= G) continue;
        const uint32_t gw[4] = {graw[it].x, graw[it].y, graw[it].z, graw[it].w};
        const uint32_t uw[4] = {uraw[it].x, uraw[it].y, uraw[it].z, uraw[it].w};
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // y = bf16(silu_bf16(g) * u): the product of two bf16 values is
            // exact in fp32 (barring subnormals), then one RNE to bf16.
            float s0 = __uint_as_float(silu_bf16(bf16lo(gw[j])) << 16);
            float s1 = __uint_as_float(silu_bf16(bf16hi(gw[j])) << 16);
            v[2 * j] = __uint_as_float(f32_to_bf16_rne(s0 * bf16lo(uw[j])) << 16);
            v[2 * j + 1] = __uint_as_float(f32_to_bf16_rne(s1 * bf16hi(uw[j])) << 16);
        }
        quant8_store<kUe8m0>(v, eps, sub, qr + gidx[it] * kGroup, s + row * s_sm + gidx[it] * s_sg);
    }
}

__global__ void silu_bf16_debug_kernel(const uint16_t* __restrict__ g, uint16_t* __restrict__ out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (uint16_t)silu_bf16(__uint_as_float((uint32_t)g[i] << 16));
}

template <bool kUe8m0>
static void launch_quant(dim3 grid, hipStream_t st, int runs, const uint16_t* x, int64_t ld_x, uint8_t* q,
                         int64_t ld_q, float* s, int64_t s_sm, int64_t s_sg, int G, float eps) {
    if (runs == 1)
        quant_group128_kernel<kUe8m0, 1><<<grid, 256, 0, st>>>(x, ld_x, q, ld_q, s, s_sm, s_sg, G, eps);
    else
        quant_group128_kernel<kUe8m0, 2><<<grid, 256, 0, st>>>(x, ld_x, q, ld_q, s, s_sm, s_sg, G, eps);
}

template <bool kUe8m0>
static void launch_silu(dim3 grid, hipStream_t st, int runs, const uint16_t* in, int64_t ld_in, int64_t nh,
                        uint8_t* q, int64_t ld_q, float* s, int64_t s_sm, int64_t s_sg, int G, float eps) {
    if (runs == 1)
        silu_mul_quant_kernel<kUe8m0, 1><<<grid, 256, 0, st>>>(in, ld_in, nh, q, ld_q, s, s_sm, s_sg, G, eps);
    else
        silu_mul_quant_kernel<kUe8m0, 2><<<grid, 256, 0, st>>>(in, ld_in, nh, q, ld_q, s, s_sm, s_sg, G, eps);
}

// Groups per row up to 16 use one pass per block; longer rows let each
// lane carry two loads in flight.
static inline int pick_runs(int64_t G) { return G > 16 ? 2 : 1; }

}  // namespace kbn

using namespace kbn;

extern "C" int kbn_per_token_group_quant_fp8(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x,
                                             void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                                             int64_t s_stride_g, float eps, int use_ue8m0, void* stream) {
    KBN_CHECK_ARG(M >= 0 && K >= 0, "per_token_group_quant_fp8: negative shape M=%lld K=%lld", (long long)M,
                  (long long)K);
    KBN_CHECK_ARG(K % kGroup == 0, "per_token_group_quant_fp8: K=%lld must be a multiple of 128", (long long)K);
    if (M == 0 || K == 0) return 0;
    KBN_CHECK_ARG(x_bf16 && q_fp8 && scale, "per_token_group_quant_fp8: null pointer");
    KBN_CHECK_ARG(ld_x >= K && ld_q >= K, "per_token_group_quant_fp8: row stride smaller than K");
    KBN_CHECK_ARG(aligned16(x_bf16) && ld_x % 8 == 0,
                  "per_token_group_quant_fp8: input rows must be 16-byte aligned (ld_x %% 8 == 0)");
    KBN_CHECK_ARG((reinterpret_cast<uintptr_t>(q_fp8) & 7u) == 0 && ld_q % 8 == 0,
                  "per_token_group_quant_fp8: output rows must be 8-byte aligned");
    KBN_CHECK_ARG(M <= 0x7FFFFFFFLL, "per_token_group_quant_fp8: M too large");
    const int64_t G = K / kGroup;
    const int runs = pick_runs(G);
    const int64_t per_block = 16 * runs;
    dim3 grid((unsigned)M, (unsigned)((G + per_block - 1) / per_block));
    KBN_CHECK_ARG(grid.y <= 65535u, "per_token_group_quant_fp8: K too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        launch_quant<true>(grid, st, runs, (const uint16_t*)x_bf16, ld_x, (uint8_t*)q_fp8, ld_q, scale, s_stride_m,
                           s_stride_g, (int)G, eps);
    else
        launch_quant<false>(grid, st, runs, (const uint16_t*)x_bf16, ld_x, (uint8_t*)q_fp8, ld_q, scale, s_stride_m,
                            s_stride_g, (int)G, eps);
    KBN_CHECK_LAUNCH("per_token_group_quant_fp8");
    return 0;
}

extern "C" int kbn_silu_mul_quant_fp8(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in, void* q_fp8,
                                      int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g, float eps,
                                      int use_ue8m0, void* stream) {
    KBN_CHECK_ARG(M >= 0 && N_half >= 0, "silu_mul_quant_fp8: negative shape");
    KBN_CHECK_ARG(N_half % kGroup == 0, "silu_mul_quant_fp8: N/2=%lld must be a multiple of 128",
                  (long long)N_half);
    if (M == 0 || N_half == 0) return 0;
    KBN_CHECK_ARG(in_bf16 && q_fp8 && scale, "silu_mul_quant_fp8: null pointer");
    KBN_CHECK_ARG(ld_in >= 2 * N_half && ld_q >= N_half, "silu_mul_quant_fp8: row stride too small");
    KBN_CHECK_ARG(aligned16(in_bf16) && ld_in % 8 == 0,
                  "silu_mul_quant_fp8: input rows must be 16-byte aligned (ld_in %% 8 == 0)");
    KBN_CHECK_ARG((reinterpret_cast<uintptr_t>(q_fp8) & 7u) == 0 && ld_q % 8 == 0,
                  "silu_mul_quant_fp8: output rows must be 8-byte aligned");
    KBN_CHECK_ARG(M <= 0x7FFFFFFFLL, "silu_mul_quant_fp8: M too large");
    const int64_t G = N_half / kGroup;
    const int runs = pick_runs(G);
    const int64_t per_block = 16 * runs;
    dim3 grid((unsigned)M, (unsigned)((G + per_block - 1) / per_block));
    KBN_CHECK_ARG(grid.y <= 65535u, "silu_mul_quant_fp8: N too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (use_ue8m0)
        launch_silu<true>(grid, st, runs, (const uint16_t*)in_bf16, ld_in, N_half, (uint8_t*)q_fp8, ld_q, scale,
                          s_stride_m, s_stride_g, (int)G, eps);
    else
        launch_silu<false>(grid, st, runs, (const uint16_t*)in_bf16, ld_in, N_half, (uint8_t*)q_fp8, ld_q, scale,
                           s_stride_m, s_stride_g, (int)G, eps);
    KBN_CHECK_LAUNCH("silu_mul_quant_fp8");
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
