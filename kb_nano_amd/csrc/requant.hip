// 128x128 block (re)quantization of weights at load time: the single-pass form
// of postprocess_fp8_weights[_batched] (tasks/baseline/L1/fp8_linear.py:453-554),
// which dequantizes a checkpoint's fp8 block with its fp32 scale and re-quantizes
// it through DeepGEMM's per_block_cast_to_fp8 (DeepGEMM v2.1.1.post3, called at
// fp8_linear.py:497-499 and :543-545):
//   x = fp32(code) * s_in            (or an fp32 master weight)
//   sf = max(max |x| over the block, eps) / 448, rounded up to a power of two
//        under UE8M0 (exponent arithmetic; DeepGEMM writes it 2^ceil(log2 sf))
//   code' = e4m3_rne(x * (1 / sf)),  padding rows / columns of ragged blocks
//           count as zeros and are not written.
// The torch version materializes an fp32 copy of the weight (4 bytes per
// element) and runs ~10 launches per tensor; this is one launch over all
// experts, reading 1 byte and writing 1 byte per element.
//
// One workgroup (256 lanes) per block.  Every load instruction of a wavefront
// covers whole 128-byte block rows: fp8 input, lane t takes the 16 bytes at
// column 16*(t%8) of rows t/8 + 32c (c = 0..3); fp32 input, the float4 at
// column 4*(t%32) of rows t/32 + 8c (c = 0..15).  Block amax: wavefront max,
// then four partials through LDS.  Every lane reads its inputs (and the block
// scale) before the barrier and writes after it, so fp8 codes may be
// requantized in place (w_out == w_in, scales at the same positions).
#include "kbn_common.h"

namespace kbn {
namespace {

struct RequantArgs {
    const void* w_in;       // [E, N, K] fp8 codes (in_f32 = 0) or fp32 (1), contiguous
    int in_f32;
    const float* s_in;      // fp8 input: block scale (e, nb, kb) at s_in[e*s_in_e + nb*s_in_ld + kb]
    int64_t s_in_e, s_in_ld;
    uint8_t* w_out;         // [E, N, K] fp8, contiguous (may alias w_in)
    float* s_out;           // (e, nb, kb) at s_out[e*s_out_e + nb*s_out_ld + kb] (may alias s_in)
    int64_t s_out_e, s_out_ld;
    int N, K, NB, KB;
    int ue8m0;
    float eps;
};

__global__ __launch_bounds__(256) void block_requant_kernel(const RequantArgs a) {
    __shared__ float part[4];
    const int t = threadIdx.x;
    const int64_t bid = blockIdx.x;
    const int kb = (int)(bid % a.KB);
    const int nb = (int)((bid / a.KB) % a.NB);
    const int64_t e = bid / ((int64_t)a.KB * a.NB);
    const int rows = min(128, a.N - nb * 128);
    const int64_t blk = (e * a.N + (int64_t)nb * 128) * a.K + (int64_t)kb * 128;   // element (0, 0)

    float x[64];
    if (a.in_f32) {
        const int r0 = t >> 5, col = (t & 31) * 4;
        const bool col_ok = kb * 128 + col < a.K;
        const float* src = static_cast<const float*>(a.w_in) + blk + col;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const int r = r0 + 8 * c;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (col_ok && r < rows) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (int64_t)r * a.K));
            x[4 * c] = __uint_as_float(v.x); x[4 * c + 1] = __uint_as_float(v.y);
            x[4 * c + 2] = __uint_as_float(v.z); x[4 * c + 3] = __uint_as_float(v.w);
        }
    } else {
        const int r0 = t >> 3, col = (t & 7) * 16;
        const bool col_ok = kb * 128 + col < a.K;
        const float s = a.s_in[e * a.s_in_e + (int64_t)nb * a.s_in_ld + kb];
        const uint8_t* src = static_cast<const uint8_t*>(a.w_in) + blk + col;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int r = r0 + 32 * c;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (col_ok && r < rows) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (int64_t)r * a.K));
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int w = (int)v[d];
                x[16 * c + 4 * d] = __builtin_amdgcn_cvt_f32_fp8(w, 0) * s;
                x[16 * c + 4 * d + 1] = __builtin_amdgcn_cvt_f32_fp8(w, 1) * s;
                x[16 * c + 4 * d + 2] = __builtin_amdgcn_cvt_f32_fp8(w, 2) * s;
                x[16 * c + 4 * d + 3] = __builtin_amdgcn_cvt_f32_fp8(w, 3) * s;
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
    if ((t & 63) == 0) part[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));

    float sf = fmaxf(amax, a.eps) / kFp8Max;
    if (a.ue8m0) sf = ue8m0_ceil(sf);
    const float inv = 1.0f / sf;      // exact for a power of two
    // |x * inv| <= 448 (1 + 2^-23)^2 < 464: the conversion's round to nearest
    // even keeps it at or below 448, as the reference's cast does
    uint8_t* dst = a.w_out + blk;
    if (a.in_f32) {
        const int r0 = t >> 5, col = (t & 31) * 4;
        if (kb * 128 + col < a.K) {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const int r = r0 + 8 * c;
                const int i = 4 * c;
                if (r < rows)
                    *reinterpret_cast<uint32_t*>(dst + (int64_t)r * a.K + col) =
                        pack4_e4m3(x[i] * inv, x[i + 1] * inv, x[i + 2] * inv, x[i + 3] * inv);
            }
        }
    } else {
        const int r0 = t >> 3, col = (t & 7) * 16;
        if (kb * 128 + col < a.K) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int r = r0 + 32 * c;
                u32x4 o;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int i = 16 * c + 4 * d;
                    o[d] = pack4_e4m3(x[i] * inv, x[i + 1] * inv, x[i + 2] * inv, x[i + 3] * inv);
                }
                if (r < rows) *reinterpret_cast<u32x4*>(dst + (int64_t)r * a.K + col) = o;
            }
        }
    }
    if (t == 0) a.s_out[e * a.s_out_e + (int64_t)nb * a.s_out_ld + kb] = sf;
}

}  // namespace
}  // namespace kbn

using namespace kbn;

extern "C" int kbn_fp8_block_requant(const void* w_in, int in_f32, const float* s_in, int64_t s_in_e,
                                     int64_t s_in_ld, int64_t E, int64_t N, int64_t K, void* w_out, float* s_out,
                                     int64_t s_out_e, int64_t s_out_ld, int use_ue8m0, float eps, void* stream) {
    const char* what = "fp8_block_requant";
    KBN_CHECK_ARG(E >= 0 && N >= 0 && K >= 0 && E <= 0x7FFFFFFFLL && N <= 0x7FFFFFFFLL && K <= 0x7FFFFFFFLL,
                  "%s: bad shape", what);
    KBN_CHECK_ARG(K % 16 == 0, "%s: K=%lld must be a multiple of 16", what, (long long)K);
    if (E == 0 || N == 0 || K == 0) return 0;
    const int64_t NB = (N + 127) / 128, KB = (K + 127) / 128;
    KBN_CHECK_ARG(w_in && w_out && s_out && (in_f32 || s_in), "%s: null pointer", what);
    KBN_CHECK_ARG(aligned16(w_in) && aligned16(w_out), "%s: weights must be 16-byte aligned", what);
    KBN_CHECK_ARG(s_out_ld >= KB && s_out_e >= NB * s_out_ld, "%s: output scale strides too small", what);
    if (!in_f32) KBN_CHECK_ARG(s_in_ld >= KB && s_in_e >= NB * s_in_ld, "%s: input scale strides too small", what);
    KBN_CHECK_ARG(eps >= 1e-30f, "%s: eps must be at least 1e-30 (sf = eps/448 stays a normal float)", what);
    // In-place requant is safe only where every block reads exactly the bytes
    // it later writes: fp8 codes over the same layout (w_out == w_in) and
    // scales at the same positions.  fp32 input is 4 bytes per element, so an
    // fp8 output over it would overwrite other blocks' unread inputs.
    const uintptr_t wi = reinterpret_cast<uintptr_t>(w_in), wo = reinterpret_cast<uintptr_t>(w_out);
    const uintptr_t wi_end = wi + (uintptr_t)(E * N * K * (in_f32 ? 4 : 1)), wo_end = wo + (uintptr_t)(E * N * K);
    const bool w_overlap = wi < wo_end && wo < wi_end;
    KBN_CHECK_ARG(!w_overlap || (!in_f32 && wi == wo), "%s: w_out overlaps w_in (%s)", what,
                  in_f32 ? "fp32 input cannot be requantized in place" : "only w_out == w_in is allowed");
    if (!in_f32) {
        const uintptr_t si = reinterpret_cast<uintptr_t>(s_in), so = reinterpret_cast<uintptr_t>(s_out);
        const uintptr_t si_end = si + (uintptr_t)(((E - 1) * s_in_e + (NB - 1) * s_in_ld + KB) * 4);
        const uintptr_t so_end = so + (uintptr_t)(((E - 1) * s_out_e + (NB - 1) * s_out_ld + KB) * 4);
        const bool s_overlap = si < so_end && so < si_end;
        KBN_CHECK_ARG(!s_overlap || (si == so && s_in_e == s_out_e && s_in_ld == s_out_ld),
                      "%s: s_out overlaps s_in with a different layout", what);
    }
    const int64_t blocks = E * NB * KB;
    KBN_CHECK_ARG(blocks <= 0x7FFFFFFFLL, "%s: too many blocks", what);
    RequantArgs a{};
    a.w_in = w_in;
    a.in_f32 = in_f32 != 0;
    a.s_in = s_in;
    a.s_in_e = s_in_e;
    a.s_in_ld = s_in_ld;
    a.w_out = static_cast<uint8_t*>(w_out);
    a.s_out = s_out;
    a.s_out_e = s_out_e;
    a.s_out_ld = s_out_ld;
    a.N = (int)N;
    a.K = (int)K;
    a.NB = (int)NB;
    a.KB = (int)KB;
    a.ue8m0 = use_ue8m0 != 0;
    a.eps = eps;
    block_requant_kernel<<<dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}
