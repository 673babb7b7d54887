// Fused RMSNorm (optionally after a residual add) + per-token-group (1x128)
// FP8 quantization with UE8M0 scales: the producer of Fp8Linear's activation
// operand in a decoder layer, without the bf16 round trip of a separate norm.
// Contract of tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-93 and :124-201
// (kb_nano):
//   plain: a = x;  fused add: a = r + x (fp32), r <- bf16(a), base = bf16(a)
//   inv = 1 / sqrt(mean(a^2) + eps);  v = (base * inv) * w   (fp32, unrounded)
//   per 1x128 group: s = ceil_pow2(max(max|v|, 1e-10) / 448); q = e4m3(v / s)
//   fused add also writes x <- bf16(v).
//
// One wavefront per token at a time, four per workgroup; each wavefront walks
// tokens with a grid stride and, for rows up to 8192 (plain) or 4096 (fused)
// columns, loads the next token's row before normalizing the current one, so
// reads overlap stores.  The weight vector is staged in LDS once per
// workgroup.  Lane l owns the 16-byte chunks at c*512 + 8l (c = 0 .. kC-1):
// the whole row stays in registers between the sum of squares and the
// normalize+quant pass, so HBM sees one read of the row and one write of the
// codes.  A 1x128 group is 16 lanes of
// one chunk (lanes 16j .. 16j+15), so its absmax is the same 4-step DPP max as
// the standalone quant kernel.  The sum of squares is fmaf in chunk then
// element order per lane, then an xor butterfly over the 64 lanes (every lane
// ends with the same value); inv uses the correctly rounded sqrt and divide.
#include "kbn_common.h"

namespace kbn {
namespace {

constexpr int kNormWaves = 4;
constexpr float kGroupEps = 1e-10f;   // absmax floor of the scale (rmsnorm_quant.cu:75)

struct NormArgs {
    uint16_t* x;          // [M, H] bf16, row stride ld_x (fused add: overwritten with bf16(v))
    int64_t ld_x;
    const uint16_t* w;    // [H] bf16
    uint16_t* r;          // fused add: [M, H] bf16 residual, row stride ld_r (overwritten with r + x)
    int64_t ld_r;
    uint8_t* q;           // [M, H] fp8, row stride ld_q
    int64_t ld_q;
    float* s;             // scale (m, g) at s[m * s_m + g * s_g]
    int64_t s_m, s_g;
    int M, H;
    float eps;
};

__device__ __forceinline__ float bf16_at(const u32x4& v, int j) {
    const uint32_t word = v[j >> 1];
    return (j & 1) ? bf16hi(word) : bf16lo(word);
}

// Row registers of one token: x (and, fused add, the residual) as 16-byte
// chunks c*512 + 8*lane.
template <int kC, bool kAdd>
struct NormRow {
    u32x4 x[kC];
    u32x4 r[kAdd ? kC : 1];
};

template <int kC, bool kAdd>
__device__ __forceinline__ void load_row(const NormArgs& a, int m, int lane, NormRow<kC, kAdd>& row) {
    const uint16_t* xr = a.x + (int64_t)m * a.ld_x;
    const uint16_t* rr = kAdd ? a.r + (int64_t)m * a.ld_r : nullptr;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
        const int e0 = c * 512 + 8 * lane;
        if ((c + 1) * 512 <= a.H) {   // uniform: the whole chunk is in the row
            row.x[c] = *reinterpret_cast<const u32x4*>(xr + e0);
            if constexpr (kAdd) row.r[c] = *reinterpret_cast<const u32x4*>(rr + e0);
        } else {
            row.x[c] = u32x4{0u, 0u, 0u, 0u};
            if (e0 < a.H) row.x[c] = *reinterpret_cast<const u32x4*>(xr + e0);
            if constexpr (kAdd) {
                row.r[c] = u32x4{0u, 0u, 0u, 0u};
                if (e0 < a.H) row.r[c] = *reinterpret_cast<const u32x4*>(rr + e0);
            }
        }
    }
}

// Clamp to the e4m3 range as the reference does (fminf(fmaxf(v, -448), 448),
// rmsnorm_quant.cu:82): one v_med3_f32, which has the same IEEE minNum/maxNum
// semantics (NaN -> -448).
__device__ __forceinline__ float clamp448(float v) { return __builtin_amdgcn_fmed3f(v, -kFp8Max, kFp8Max); }

// Normalize and quantize one token whose row is in registers; `wl` is the
// weight vector in LDS, chunk-major like the row.
template <int kC, bool kAdd>
__device__ __forceinline__ void norm_row(const NormArgs& a, int m, int lane, NormRow<kC, kAdd>& row,
                                         const u32x4* wl) {
#pragma clang fp contract(off)
    uint16_t* xr = a.x + (int64_t)m * a.ld_x;
    // ---- sum of squares (fused add: of the unrounded sums, whose bf16
    // roundings replace the residual and are what gets normalized)
    float p = 0.f;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
        const int e0 = c * 512 + 8 * lane;
        if (e0 >= a.H) continue;
        u32x4 nr = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float av = bf16_at(row.x[c], j);
            if constexpr (kAdd) {
                av = bf16_at(row.r[c], j) + av;
                nr[j >> 1] |= f32_to_bf16_rne(av) << (16 * (j & 1));
            }
            p = fmaf(av, av, p);
        }
        if constexpr (kAdd) {
            row.r[c] = nr;
            *reinterpret_cast<u32x4*>(a.r + (int64_t)m * a.ld_r + e0) = nr;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) p = p + __shfl_xor(p, d, 64);
    const float inv = 1.0f / sqrtf(p / (float)a.H + a.eps);

    // ---- normalize and quantize, one chunk (4 groups per wavefront) at a time
#pragma unroll
    for (int c = 0; c < kC; ++c) {
        const int e0 = c * 512 + 8 * lane;
        if (c * 512 >= a.H) break;   // uniform: no lane of this chunk is in the row
        const bool full = (c + 1) * 512 <= a.H;   // uniform
        const bool live = full || e0 < a.H;
        const u32x4 wv = wl[c * 64 + lane];
        const u32x4& base = kAdd ? row.r[c] : row.x[c];
        float v[8];
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // lanes past the row hold zeros (loads and weights), so v = 0 there
            v[j] = (bf16_at(base, j) * inv) * bf16_at(wv, j);
            amax = fmaxf(amax, fabsf(v[j]));
        }
        amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
        amax = fmaxf(amax, kGroupEps);
        const float sc = ue8m0_ceil(amax / kFp8Max);
        const float is = pow2_recip(sc);
        if (live) {
            const uint32_t lo = pack4_e4m3(clamp448(v[0] * is), clamp448(v[1] * is), clamp448(v[2] * is),
                                           clamp448(v[3] * is));
            const uint32_t hi = pack4_e4m3(clamp448(v[4] * is), clamp448(v[5] * is), clamp448(v[6] * is),
                                           clamp448(v[7] * is));
            *reinterpret_cast<uint2*>(a.q + (int64_t)m * a.ld_q + e0) = make_uint2(lo, hi);
            if ((lane & 15) == 0) a.s[(int64_t)m * a.s_m + (int64_t)(e0 >> 7) * a.s_g] = sc;
            if constexpr (kAdd) {
                u32x4 o;
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] = f32_to_bf16_rne(v[2 * k]) | (f32_to_bf16_rne(v[2 * k + 1]) << 16);
                *reinterpret_cast<u32x4*>(xr + e0) = o;
            }
        }
    }
}

// Token placement.  Consecutive workgroup ids are dispatched round-robin over
// the 8 XCDs; each XCD instead gets a contiguous range of workgroup slots, and
// slot s owns tokens [s * 4T, (s + 1) * 4T) (T = tokens per wavefront),
// wavefront w of it tokens s*4T + w, + 4, + 8, ...  So the 32 tokens that
// share a 128-byte line of the column-major scales are written from one XCD
// and the line merges in its L2.  With kPrefetch, the next token's row is
// loaded before the current one is normalized, so its reads overlap the
// current stores.
template <int kC, bool kAdd, bool kPrefetch>
__global__ __launch_bounds__(64 * kNormWaves) void rmsnorm_quant_kernel(const NormArgs a, int tpw) {
    __shared__ u32x4 wl[kC * 64];
    for (int i = threadIdx.x; i < kC * 64; i += 64 * kNormWaves) {
        const int e0 = (i >> 6) * 512 + 8 * (i & 63);
        wl[i] = e0 < a.H ? *reinterpret_cast<const u32x4*>(a.w + e0) : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nblk = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
    const int slot = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
    const int first = slot * kNormWaves * tpw + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = min(a.M, (slot + 1) * kNormWaves * tpw);   // exclusive
    int m = first;
    if (m >= last) return;
    if constexpr (kPrefetch) {
        NormRow<kC, kAdd> cur, nxt;
        load_row<kC, kAdd>(a, m, lane, cur);
        for (;;) {
            const int mn = m + kNormWaves;
            if (mn < last) load_row<kC, kAdd>(a, mn, lane, nxt);
            norm_row<kC, kAdd>(a, m, lane, cur, wl);
            if (mn >= last) break;
            m = mn;
            const int mm = m + kNormWaves;
            if (mm < last) load_row<kC, kAdd>(a, mm, lane, cur);
            norm_row<kC, kAdd>(a, m, lane, nxt, wl);
            if (mm >= last) break;
            m = mm;
        }
    } else {
        for (; m < last; m += kNormWaves) {
            NormRow<kC, kAdd> cur;
            load_row<kC, kAdd>(a, m, lane, cur);
            norm_row<kC, kAdd>(a, m, lane, cur, wl);
        }
    }
}

// Wavefronts in the grid: one token each up to two per SIMD; beyond that two
// per SIMD, each walking several tokens with the prefetch.
int norm_waves(int M) {
    const int cap = cu_count() * 8;
    return M <= cap ? M : cap;
}

template <bool kAdd>
int launch_norm(const NormArgs& a, hipStream_t st) {
    const int chunks = (a.H + 511) / 512;
    const int waves = norm_waves(a.M);
    const int tpw = (a.M + waves - 1) / waves;                            // tokens per wavefront
    const int blocks = (a.M + kNormWaves * tpw - 1) / (kNormWaves * tpw);  // every slot owns >= 1 token
    const dim3 grid((unsigned)blocks), block(64 * kNormWaves);
    if (chunks <= 2) rmsnorm_quant_kernel<2, kAdd, true><<<grid, block, 0, st>>>(a, tpw);
    else if (chunks <= 4) rmsnorm_quant_kernel<4, kAdd, true><<<grid, block, 0, st>>>(a, tpw);
    else if (chunks <= 8) rmsnorm_quant_kernel<8, kAdd, true><<<grid, block, 0, st>>>(a, tpw);
    else if (chunks <= 16) rmsnorm_quant_kernel<16, kAdd, !kAdd><<<grid, block, 0, st>>>(a, tpw);
    else {
        if constexpr (kAdd) return 1;
        else rmsnorm_quant_kernel<32, false, false><<<grid, block, 0, st>>>(a, tpw);
    }
    return 0;
}

}  // namespace
}  // namespace kbn

using namespace kbn;

extern "C" int kbn_rmsnorm_fp8_quant(void* x_bf16, int64_t M, int64_t H, int64_t ld_x, const void* w_bf16,
                                     void* residual_bf16, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale,
                                     int64_t s_stride_m, int64_t s_stride_g, float eps, void* stream) {
    const char* what = residual_bf16 ? "fused_add_rmsnorm_fp8_quant" : "rmsnorm_fp8_quant";
    const bool add = residual_bf16 != nullptr;
    const int64_t max_h = add ? 8192 : 16384;
    KBN_CHECK_ARG(M >= 0 && M <= 0x7FFFFFFFLL, "%s: bad M=%lld", what, (long long)M);
    KBN_CHECK_ARG(H > 0 && H % 8 == 0 && H <= max_h, "%s: hidden size %lld must be a positive multiple of 8, "
                  "at most %lld", what, (long long)H, (long long)max_h);
    if (M == 0) return 0;
    KBN_CHECK_ARG(x_bf16 && w_bf16 && q_fp8 && scale, "%s: null pointer", what);
    KBN_CHECK_ARG(aligned16(x_bf16) && aligned16(w_bf16) && ld_x >= H && ld_x % 8 == 0,
                  "%s: input and weight must be 16-byte aligned, input row stride >= H and a multiple of 8", what);
    KBN_CHECK_ARG(ld_q >= H && ld_q % 8 == 0 && (reinterpret_cast<uintptr_t>(q_fp8) & 7u) == 0,
                  "%s: output rows must be 8-byte aligned with a stride >= H", what);
    if (add)
        KBN_CHECK_ARG(aligned16(residual_bf16) && ld_r >= H && ld_r % 8 == 0,
                      "%s: residual must be 16-byte aligned with a row stride >= H and a multiple of 8", what);
    KBN_CHECK_ARG(s_stride_m >= 0 && s_stride_g >= 0, "%s: negative scale stride", what);
    NormArgs a{};
    a.x = static_cast<uint16_t*>(x_bf16);
    a.ld_x = ld_x;
    a.w = static_cast<const uint16_t*>(w_bf16);
    a.r = static_cast<uint16_t*>(residual_bf16);
    a.ld_r = ld_r;
    a.q = static_cast<uint8_t*>(q_fp8);
    a.ld_q = ld_q;
    a.s = scale;
    a.s_m = s_stride_m;
    a.s_g = s_stride_g;
    a.M = (int)M;
    a.H = (int)H;
    a.eps = eps;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (add ? launch_norm<true>(a, st) : launch_norm<false>(a, st)) {
        set_error("%s: no kernel for hidden size %lld", what, (long long)H);
        return 1;
    }
    KBN_CHECK_LAUNCH(what);
    return 0;
}
