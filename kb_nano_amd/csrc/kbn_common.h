// Shared device helpers and host-side error plumbing for the gfx950 FP8
// linear-path kernels.  Only gfx950 (CDNA4) is targeted: fp8 means OCP
// e4m3fn, wavefronts are 64 lanes wide.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <cstring>

namespace kbn {

// --------------------------------------------------------------- errors ---

// Per-thread last-error message returned by kbn_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define KBN_CHECK_ARG(cond, ...)            \
    do {                                    \
        if (!(cond)) {                      \
            ::kbn::set_error(__VA_ARGS__);  \
            return 1;                       \
        }                                   \
    } while (0)

#define KBN_CHECK_LAUNCH(what)                                                    \
    do {                                                                          \
        hipError_t e_ = hipGetLastError();                                        \
        if (e_ != hipSuccess) {                                                   \
            ::kbn::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return 2;                                                             \
        }                                                                         \
    } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (cached per device).
inline int cu_count() {
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

// ------------------------------------------------------------ constants ---

constexpr int kGroup = 128;          // 1x128 activation groups, 128x128 weight blocks
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer descriptor word 3: 32-bit dword format (gfx9 family)
constexpr int kOob = (int)0x80000000;         // buffer offset beyond any range: loads read zero, stores are dropped
constexpr float kFp8Max = 448.0f;    // float8_e4m3fn max finite

// ------------------------------------------------------- device helpers ---

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Smallest power of two >= r for a positive normal float r (exponent bits,
// +1 when any mantissa bit is set): the UE8M0 rounding of the scale.
__device__ __forceinline__ float ue8m0_ceil(float r) {
    uint32_t u = __float_as_uint(r);
    uint32_t e = (u >> 23) & 0xFFu;
    if (u & 0x7FFFFFu) e += 1;
    return __uint_as_float(e << 23);
}

// ue8m0_ceil(amax / 448) without the division.  With amax = m 2^e, m in
// [1, 2): for m <= 1.75 the quotient m/1.75 2^(e-8) lies in (2^(e-9), 2^(e-8)]
// (rounding can at most reach 2^(e-8)), for m > 1.75 in (2^(e-8), 2^(e-7)) (it
// exceeds 2^(e-8) by at least 2^-23/1.75 relative, more than half an ulp), so
// the power of two is 2^(e-8) or 2^(e-7) by a compare of the mantissa with
// 1.75's (0x600000).  Zero, subnormal, tiny (result not normal), infinite and
// NaN amax take the division.
__device__ __forceinline__ float ue8m0_ceil_div448(float amax) {
    const uint32_t u = __float_as_uint(amax);
    const uint32_t e = (u >> 23) & 0xFFu;
    if (e <= 9u || e == 255u) return ue8m0_ceil(amax / kFp8Max);
    return __uint_as_float((e - 8u + ((u & 0x7FFFFFu) > 0x600000u ? 1u : 0u)) << 23);
}

// Biased exponent byte (E8M0) of ue8m0_ceil(r): the per-operand scale
// consumed by the block-scaled MFMA.
__device__ __forceinline__ int ue8m0_ceil_byte(float r) {
    uint32_t u = __float_as_uint(r);
    uint32_t e = (u >> 23) & 0xFFu;
    if (u & 0x7FFFFFu) e += 1;
    return (int)(e > 254u ? 254u : e);
}

// Exact reciprocal of a power of two in the normal range.
__device__ __forceinline__ float pow2_recip(float s) {
    uint32_t e = (__float_as_uint(s) >> 23) & 0xFFu;
    return __uint_as_float((254u - e) << 23);
}

// Max over each row of 16 lanes (DPP quad swaps + row rotates); operands
// are non-negative floats carried as bits, so an unsigned max is a float max.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    uint32_t t;
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    v = v > t ? v : t;
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    v = v > t ? v : t;
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false); // row_ror:4
    v = v > t ? v : t;
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false); // row_ror:8
    v = v > t ? v : t;
    return v;
}

// Pack four floats into four e4m3fn codes with the hardware conversion:
// round to nearest even, |x| in (448, 464] -> 448, larger or NaN -> NaN code.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

// Four e4m3 codes of a/sc, b/sc, c/sc, d/sc for a normal power of two sc,
// by the gfx950 scaled conversion v_cvt_scalef32_pk_fp8_f32: the codes of
// pack4_e4m3(a * (1/sc), ...) (checked on the device against it for 2^21
// fp32 pairs at each of 67 scales from 2^-100 to 2^100, edge cases and e4m3
// rounding ties included), without the four multiplies.
__device__ __forceinline__ uint32_t pack4_e4m3_scaled(float a, float b, float c, float d, float sc) {
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    s16x2 r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s16x2{0, 0}, a, b, sc, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, c, d, sc, true);
    return __builtin_bit_cast(uint32_t, r);
}

// Four e4m3 codes of the bf16 pairs w0, w1 divided by the power of two sc,
// by the gfx950 scaled conversion v_cvt_scalef32_pk_fp8_bf16: for every
// finite bf16 input and every normal power-of-two sc it gives the codes of
// v_cvt_pk_fp8_f32(x * (1/sc)) (round to nearest even; checked exhaustively
// on the device), so no widening to fp32 and no multiply are needed.
__device__ __forceinline__ uint32_t pack4_e4m3_bf16(uint32_t w0, uint32_t w1, float sc) {
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    s16x2 r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(s16x2{0, 0}, __builtin_bit_cast(bf16x2, w0), sc, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2, w1), sc, true);
    return __builtin_bit_cast(uint32_t, r);
}

// UE8M0 quantization of a 1x128 group, shared by the quant kernels and the
// GEMM that quantizes its bf16 activations itself, so both produce the same
// codes and scales:
//  * abits: the group's largest bf16 magnitude as fp32 bits (NaN patterns
//    above infinity's); sc = ue8m0_ceil_div448(max(that, eps));
//  * fast path (finite absmax, normal sc): codes by the scaled conversion;
//  * otherwise the general path: the absmax recomputed ignoring NaN (as the
//    reference's max does), and the codes below.
__device__ __forceinline__ bool ue8m0_fast_path(uint32_t abits, float sc) {
    return abits < 0x7F800000u && (__float_as_uint(sc) >> 23) - 1u < 254u;
}
// General-path codes of four values under a UE8M0 scale: an infinite scale
// (a group holding an infinity) maps finite values to +-0 (codes 0x00 /
// 0x80, x / inf) and the rest to the NaN code; otherwise x times the exact
// reciprocal of the power of two, by the hardware conversion.
__device__ __forceinline__ uint32_t pack4_e4m3_ue8m0_general(float a, float b, float c, float d, float sc) {
    if (sc == __builtin_inff()) {
        auto code = [](float v) -> uint32_t {
            return (fabsf(v) < __builtin_inff()) ? (__float_as_uint(v) >> 24 & 0x80u) : 0xFFu;
        };
        return code(a) | code(b) << 8 | code(c) << 16 | code(d) << 24;
    }
    const float inv = pow2_recip(sc);
    return pack4_e4m3(a * inv, b * inv, c * inv, d * inv);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// SiLU*Mul and the 1x128 group quant of bf16 values, shared by the quant
// kernels (csrc/quant.hip) and the grouped GEMM that applies them to its own
// output (gemm_kernel.h), so both produce the same codes and scales.

// bf16(silu(g)) * up for the two bf16 values of each word: the exact fp32
// products rounded to bf16 by one v_cvt_pk_bf16_f32, returned packed.
__device__ __forceinline__ uint32_t silu_mul_pair(const uint16_t* __restrict__ lut, uint32_t gw, uint32_t uw) {
    const float s0 = __uint_as_float((uint32_t)lut[gw & 0xFFFFu] << 16);
    const float s1 = __uint_as_float((uint32_t)lut[gw >> 16] << 16);
    const bf16x2 p = __builtin_convertvector((f32x2{s0 * bf16lo(uw), s1 * bf16hi(uw)}), bf16x2);
    return __builtin_bit_cast(uint32_t, p);
}

// Largest magnitude of the eight bf16 values in four packed words, as the
// fp32 bit pattern of that bf16 magnitude.  Magnitude bits of bf16 order
// like the values they encode (NaN patterns above infinity), so this is a
// packed 16-bit integer max (v_pk_max_u16) over the sign-cleared words.
__device__ __forceinline__ uint32_t absmax8_bits(const uint32_t (&w)[4]) {
    auto mag = [](uint32_t x) { return __builtin_bit_cast(u16x2, x & 0x7FFF7FFFu); };
    const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(mag(w[0]), mag(w[1])),
                                              __builtin_elementwise_max(mag(w[2]), mag(w[3])));
    const uint32_t lo = m.x, hi = m.y;
    return (lo > hi ? lo : hi) << 16;
}

// The codes (eight per lane, packed) and the group scale (valid in every lane
// of the group) that quant8_store below writes, without the store, for callers
// that write the same codes to several places.  The same steps as
// quant8_store's; kept apart so that the quant kernels' instruction schedule
// is not disturbed (the moe permute test checks the two give the same bits).
template <bool kUe8m0>
__device__ __forceinline__ u32x2 quant8_codes(const uint32_t (&w)[4], float eps, float& sc_out) {
    if constexpr (kUe8m0) {
        const uint32_t abits = row16_max_u32(absmax8_bits(w));
        const float sc = ue8m0_ceil_div448(fmaxf(__uint_as_float(abits), eps));
        // finite absmax and a normal scale (a subnormal one needs eps < 2^-118)
        if (ue8m0_fast_path(abits, sc)) {
            sc_out = sc;
            return u32x2{pack4_e4m3_bf16(w[0], w[1], sc), pack4_e4m3_bf16(w[2], w[3], sc)};
        }
    }
    // general path: the non-UE8M0 contract, and UE8M0 groups with an
    // infinity, a NaN or a subnormal scale (uniform over the group's 16 lanes)
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16lo(w[i]);
        v[2 * i + 1] = bf16hi(w[i]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
    amax = fmaxf(amax, eps);
    float sc = kUe8m0 ? ue8m0_ceil_div448(amax) : amax / kFp8Max;
    // The reference clamps v / sc to [-448, 448] before the cast.  Here that
    // clamp can never act on a finite value: sc >= fl(amax / 448), so
    // |v / sc| <= 448 (1 + 2^-23)^2 < 464, and the hardware conversion rounds
    // to nearest even, which maps (448, 464] to 448 (it only goes to NaN above
    // 464).  NaN stays NaN, as under the reference's torch.clamp.  Dropping the
    // two compares and two selects per element is worth 4% (SiLU) to 14%
    // (quant) of kernel time.
    uint32_t lo, hi;
    if (kUe8m0) {
        // an infinite absmax gives an infinite scale: x / inf is +-0 for
        // finite x (code 0x00 / 0x80) and NaN otherwise, as in the reference
        lo = pack4_e4m3_ue8m0_general(v[0], v[1], v[2], v[3], sc);
        hi = pack4_e4m3_ue8m0_general(v[4], v[5], v[6], v[7], sc);
    } else {
        lo = pack4_e4m3(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
        hi = pack4_e4m3(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
    }
    sc_out = sc;
    return u32x2{lo, hi};
}

// Quantize the 8 bf16 values owned by this lane (four packed words; 16
// lanes per group); returns the group scale (valid in every lane of the
// group).
// Codes leave through L2 (plain stores) for the quant kernel: its consumer,
// the GEMM, reads them next, and at 4096x18432 the cached stores are 7%
// faster than non-temporal ones (40 against 43 us).  The SiLU kernel's
// non-temporal stores measure the same either way and are kept.
//
// UE8M0 scales: the group absmax comes from the packed magnitudes and the
// codes from the scaled conversion of the packed values, so the values are
// never widened to fp32.  A group holding an infinity or a NaN (absmax
// pattern >= infinity's) takes the general path below, where the absmax
// ignores NaN as the reference's max does.
template <bool kUe8m0, bool kNtStore>
__device__ __forceinline__ float quant8_store(const uint32_t (&w)[4], float eps, int sub,
                                              uint8_t* __restrict__ qptr) {
    if constexpr (kUe8m0) {
        const uint32_t abits = row16_max_u32(absmax8_bits(w));
        const float sc = ue8m0_ceil_div448(fmaxf(__uint_as_float(abits), eps));
        // finite absmax and a normal scale (a subnormal one needs eps < 2^-118)
        if (ue8m0_fast_path(abits, sc)) {
            const u32x2 o{pack4_e4m3_bf16(w[0], w[1], sc), pack4_e4m3_bf16(w[2], w[3], sc)};
            if constexpr (kNtStore) __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(qptr + sub * 8));
            else *reinterpret_cast<u32x2*>(qptr + sub * 8) = o;
            return sc;
        }
    }
    // general path: the non-UE8M0 contract, and UE8M0 groups with an
    // infinity, a NaN or a subnormal scale (uniform over the group's 16 lanes)
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16lo(w[i]);
        v[2 * i + 1] = bf16hi(w[i]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
    amax = fmaxf(amax, eps);
    float sc = kUe8m0 ? ue8m0_ceil_div448(amax) : amax / kFp8Max;
    // The reference clamps v / sc to [-448, 448] before the cast.  Here that
    // clamp can never act on a finite value: sc >= fl(amax / 448), so
    // |v / sc| <= 448 (1 + 2^-23)^2 < 464, and the hardware conversion rounds
    // to nearest even, which maps (448, 464] to 448 (it only goes to NaN above
    // 464).  NaN stays NaN, as under the reference's torch.clamp.  Dropping the
    // two compares and two selects per element is worth 4% (SiLU) to 14%
    // (quant) of kernel time.
    uint32_t lo, hi;
    if (kUe8m0) {
        // an infinite absmax gives an infinite scale: x / inf is +-0 for
        // finite x (code 0x00 / 0x80) and NaN otherwise, as in the reference
        lo = pack4_e4m3_ue8m0_general(v[0], v[1], v[2], v[3], sc);
        hi = pack4_e4m3_ue8m0_general(v[4], v[5], v[6], v[7], sc);
    } else {
        lo = pack4_e4m3(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
        hi = pack4_e4m3(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
    }
    if constexpr (kNtStore) __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(qptr + sub * 8));
    else *reinterpret_cast<u32x2*>(qptr + sub * 8) = u32x2{lo, hi};
    return sc;
}

// Device address of the correctly rounded bf16 SiLU table (65,536 entries,
// csrc/quant.hip) on the current device, looked up once per device; nullptr
// with the library error set on failure.
const uint16_t* silu_lut_device(const char* what);

}  // namespace kbn
