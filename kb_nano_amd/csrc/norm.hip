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
// One workgroup of W wavefronts per token at a time (W = 8 for rows of 4096
// or more columns, else 4).  Chunk c of a row is the 512 elements c*512 ..
// c*512+511 (16 bytes per lane); wavefront w owns chunks c = W*i + w, keeps
// their weights in registers as fp32 for all its tokens, and requests the
// chunks of the token after next as soon as the current ones have been
// summed, so two tokens' reads overlap the normalize, quant and stores.  HBM sees one read of each row and one write
// of the codes.  A 1x128 group is 16 lanes of one chunk, so its absmax is the
// 4-step DPP max of the standalone quant kernel.  Sum of squares: each lane
// applies fmaf over its chunks (increasing c) and their 8 elements, an xor
// butterfly sums the wavefront's 64 lanes, and the W wavefront sums meet in
// LDS, added in wavefront order (((P0 + P1) + P2) + ...); inv uses the
// correctly rounded sqrt and divide.  When the row's sum of squares is finite and the wavefront's
// weights are finite and below 2^100, every normalized value is finite and
// |v / s| <= 448 (1 + 2^-23)^2, where the hardware conversion already gives
// the clamped code, so the clamp is skipped; other rows take it.
#include "kbn_common.h"

#include <algorithm>
#include <type_traits>

namespace kbn {
namespace {

constexpr int kNormMaxWgPerCu = 8;     // bound on the resident workgroups per CU the grid is sized for
constexpr float kGroupEps = 1e-10f;    // absmax floor of the scale (rmsnorm_quant.cu:75)

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
    int s_bytes;          // bytes the scale view spans from s
    int M, H;
    float eps;
};

// Two floats rounded to bf16 (nearest even) and packed, lo in the low half:
// one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}

__device__ __forceinline__ float bf16_at(const u32x4& v, int j) {
    const uint32_t word = v[j >> 1];
    return (j & 1) ? bf16hi(word) : bf16lo(word);
}

// This wavefront's chunks of one token: x (and, fused add, the residual).
template <int kCW, bool kAdd>
struct NormRow {
    u32x4 x[kCW];
    u32x4 r[kAdd ? kCW : 1];
};

// Row descriptor: `bytes` bytes from p; buffer accesses past them read zero
// or are dropped, so no access is branched around and every token issues the
// same memory instructions (which keeps the compiler's counter waits exact).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, (int)kRsrcWord3);
}

// Cache-policy operand of the row loads: non-temporal (each row is read once;
// at H = 7168, M = 4096 this is 20.5 against 22.4 us plain and 55.6 against
// 58.2 us with the residual add).
constexpr int kNtLoad = 2;

template <int kW, int kCW, bool kAdd>
__device__ __forceinline__ void load_row(const NormArgs& a, int m, int wave, int lane, NormRow<kCW, kAdd>& row,
                                         int dep = 0) {
    const __amdgpu_buffer_rsrc_t xr = row_rsrc(a.x + (int64_t)m * a.ld_x, 2 * a.H);
    const __amdgpu_buffer_rsrc_t rr = row_rsrc(kAdd ? a.r + (int64_t)m * a.ld_r : a.x, kAdd ? 2 * a.H : 0);
#pragma unroll
    for (int i = 0; i < kCW; ++i) {
        const int off = 2 * ((kW * i + wave) * 512 + 8 * lane) + dep;   // lanes past the row read zeros
        row.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, kNtLoad);
        if constexpr (kAdd) row.r[i] = __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, kNtLoad);
    }
}

// Clamp to the e4m3 range as the reference does (fminf(fmaxf(v, -448), 448),
// rmsnorm_quant.cu:82): one v_med3_f32, which has the same IEEE minNum/maxNum
// semantics (NaN -> -448).
__device__ __forceinline__ float clamp448(float v) { return __builtin_amdgcn_fmed3f(v, -kFp8Max, kFp8Max); }

// Factor that divides by the power-of-two scale sc exactly: its reciprocal,
// or 0 for an infinite scale (a group whose absmax overflowed), so that
// v * 0 gives v / inf's +-0 for finite v and NaN (clamped to -448) for
// infinite v, as the reference's division does.
__device__ __forceinline__ float inv_scale(float sc) { return sc < __builtin_inff() ? pow2_recip(sc) : 0.f; }

// Normalize and quantize one token.  `wf` holds this wavefront's weights,
// `part` the LDS slots of the W wavefront sums (double-buffered by token
// parity, so one barrier per token suffices), `wok` whether this wavefront's
// weights allow skipping the clamp.
template <int kW, int kCW, bool kAdd, typename Prefetch>
__device__ __forceinline__ void norm_row(const NormArgs& a, int m, int wave, int lane, NormRow<kCW, kAdd>& row,
                                         const float (&wf)[kCW][8], float* part, bool wok, Prefetch prefetch) {
#pragma clang fp contract(off)
    const __amdgpu_buffer_rsrc_t xw = row_rsrc(a.x + (int64_t)m * a.ld_x, kAdd ? 2 * a.H : 0);
    const __amdgpu_buffer_rsrc_t rw = row_rsrc(kAdd ? a.r + (int64_t)m * a.ld_r : a.x, kAdd ? 2 * a.H : 0);
    const __amdgpu_buffer_rsrc_t qw = row_rsrc(a.q + (int64_t)m * a.ld_q, a.H);
    const __amdgpu_buffer_rsrc_t sw = row_rsrc(a.s, a.s_bytes);
    // ---- sum of squares (fused add: of the unrounded sums, whose bf16
    // roundings replace the residual and are what gets normalized); chunks
    // past the row hold zeros and add nothing
    float p = 0.f;
    float base[kCW][8];   // the values to normalize, fp32 (fused add: the bf16-rounded sums)
#pragma unroll
    for (int i = 0; i < kCW; ++i) {
        const int c = kW * i + wave;
        u32x4 nr = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            float a0 = bf16_at(row.x[i], j), a1 = bf16_at(row.x[i], j + 1);
            base[i][j] = a0;
            base[i][j + 1] = a1;
            if constexpr (kAdd) {
                a0 = bf16_at(row.r[i], j) + a0;
                a1 = bf16_at(row.r[i], j + 1) + a1;
                const uint32_t h = pack_bf16_rne(a0, a1);
                nr[j >> 1] = h;
                base[i][j] = __uint_as_float(h << 16);
                base[i][j + 1] = __uint_as_float(h & 0xFFFF0000u);
            }
            p = fmaf(a0, a0, p);
            p = fmaf(a1, a1, p);
        }
        if constexpr (kAdd) __builtin_amdgcn_raw_buffer_store_b128(nr, rw, 2 * (c * 512 + 8 * lane), 0, 0);
    }
    // the next token's loads go out only now that this token's data has
    // arrived, so waiting for it never waits for them: their offsets depend
    // on p through an opaque zero, which no code motion can hoist above p
    int dep;
    asm volatile("v_mov_b32 %0, 0" : "=v"(dep) : "v"(p));
    prefetch(dep);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) p = p + __shfl_xor(p, d, 64);
    if (lane == 0) part[wave] = p;
    __syncthreads();
    p = part[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) p = p + part[w];
    const float inv = 1.0f / sqrtf(p / (float)a.H + a.eps);
    const bool noclamp = wok && p < __builtin_inff();   // uniform per wavefront

    // ---- normalize and quantize, one chunk (4 groups per wavefront) at a time;
    // the clamped and unclamped passes are separate code (a row-level branch,
    // not a per-value select) that only compute; the stores follow the branch,
    // so every path issues the same memory instructions
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 codes[kCW];
    float scl[kCW];
    float vout[kAdd ? kCW : 1][8];
    auto quant_pass = [&](auto clamp_tag) {
        constexpr bool kClamp = decltype(clamp_tag)::value;
#pragma unroll
        for (int i = 0; i < kCW; ++i) {
            float v[8];
            float amax = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // lanes past the row hold zeros (loads and weights), so v = 0 there
                v[j] = (base[i][j] * inv) * wf[i][j];
                amax = fmaxf(amax, fabsf(v[j]));
                if constexpr (kAdd) vout[i][j] = v[j];
            }
            amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
            amax = fmaxf(amax, kGroupEps);
            const float sc = ue8m0_ceil_div448(amax);
            if constexpr (kClamp) {
                const float is = inv_scale(sc);
                float t[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = clamp448(v[j] * is);
                codes[i] = u32x2{pack4_e4m3(t[0], t[1], t[2], t[3]), pack4_e4m3(t[4], t[5], t[6], t[7])};
            } else {
                // finite row: sc is a normal power of two, and the scaled
                // conversion divides by it exactly
                codes[i] = u32x2{pack4_e4m3_scaled(v[0], v[1], v[2], v[3], sc),
                                 pack4_e4m3_scaled(v[4], v[5], v[6], v[7], sc)};
            }
            scl[i] = sc;
        }
    };
    if (noclamp) quant_pass(std::false_type{});
    else quant_pass(std::true_type{});
#pragma unroll
    for (int i = 0; i < kCW; ++i) {
        const int e0 = (kW * i + wave) * 512 + 8 * lane;
        // past the row: dropped by the descriptor ranges
        __builtin_amdgcn_raw_buffer_store_b64(codes[i], qw, e0, 0, 0);
        const bool owner = (lane & 15) == 0 && e0 < a.H;
        __builtin_amdgcn_raw_buffer_store_b32(
            __float_as_uint(scl[i]), sw, owner ? (int)(4 * ((int64_t)m * a.s_m + (int64_t)(e0 >> 7) * a.s_g)) : kOob,
            0, 0);
        if constexpr (kAdd) {
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = pack_bf16_rne(vout[i][2 * k], vout[i][2 * k + 1]);
            __builtin_amdgcn_raw_buffer_store_b128(o, xw, 2 * e0, 0, 0);
        }
    }
}

// Token placement.  Consecutive workgroup ids are dispatched round-robin over
// the 8 XCDs; each XCD instead gets a contiguous range of workgroup slots, and
// slot s owns tokens [s * T, (s + 1) * T) (T tokens per workgroup), so the 32
// tokens that share a 128-byte line of the column-major scales are written
// from one XCD and the line merges in its L2.
template <int kW, int kCW, bool kAdd>
__global__ __launch_bounds__(64 * kW) void rmsnorm_quant_kernel(const NormArgs a, int tpw) {
    __shared__ float part[2][kW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // this wavefront's weights, fp32; lanes past the row hold zeros
    float wf[kCW][8];
    bool wok = true;
#pragma unroll
    for (int i = 0; i < kCW; ++i) {
        const int e0 = (kW * i + wave) * 512 + 8 * lane;
        u32x4 wv = u32x4{0u, 0u, 0u, 0u};
        if (e0 < a.H) wv = *reinterpret_cast<const u32x4*>(a.w + e0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            wf[i][j] = bf16_at(wv, j);
            wok = wok && fabsf(wf[i][j]) <= 0x1p100f;   // false for NaN and infinities
        }
    }
    wok = __all(wok);
    const int nblk = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, per = nblk >> 3, rem = nblk & 7;
    const int slot = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
    int m = slot * tpw;
    const int last = min(a.M, (slot + 1) * tpw);   // exclusive
    if (m >= last) return;                         // uniform over the workgroup
    // ring of three rows: token m + 2 is requested while token m is
    // normalized
    NormRow<kCW, kAdd> b0, b1, b2;
    load_row<kW, kCW, kAdd>(a, m, wave, lane, b0);
    if (m + 1 < last) load_row<kW, kCW, kAdd>(a, m + 1, wave, lane, b1);
    // as many stores as a token issues, all dropped (zero-length range): the
    // loop is entered with memory instructions in flight after the row loads
    // as on its back edge, so the compiler's wait for the first token lets the
    // previous token's stores stay in flight
    {
        const __amdgpu_buffer_rsrc_t none = row_rsrc(a.q, 0);
#pragma unroll
        for (int k = 0; k < kCW * (kAdd ? 4 : 2); ++k)   // distinct offsets, so none is merged away
            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)k, none, kOob + 4 * k, 0, 0);
    }
    for (;;) {
        norm_row<kW, kCW, kAdd>(a, m, wave, lane, b0, wf, part[m & 1], wok, [&](int dep) {
            if (m + 2 < last) load_row<kW, kCW, kAdd>(a, m + 2, wave, lane, b2, dep);
        });
        if (++m >= last) break;
        norm_row<kW, kCW, kAdd>(a, m, wave, lane, b1, wf, part[m & 1], wok, [&](int dep) {
            if (m + 2 < last) load_row<kW, kCW, kAdd>(a, m + 2, wave, lane, b0, dep);
        });
        if (++m >= last) break;
        norm_row<kW, kCW, kAdd>(a, m, wave, lane, b2, wf, part[m & 1], wok, [&](int dep) {
            if (m + 2 < last) load_row<kW, kCW, kAdd>(a, m + 2, wave, lane, b1, dep);
        });
        if (++m >= last) break;
    }
}

// Workgroups of one instantiation resident per CU (from its register use),
// queried once per process.
template <int kW, int kCW, bool kAdd>
int norm_occupancy() {
    static int occ = 0;
    if (occ == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, rmsnorm_quant_kernel<kW, kCW, kAdd>, 64 * kW, 0) !=
                hipSuccess || n <= 0)
            n = 1;
        occ = std::min(n, kNormMaxWgPerCu);
    }
    return occ;
}

// One wave of resident workgroups, each walking an equal share of the tokens.
template <int kW, int kCW, bool kAdd>
void launch_norm_cfg(const NormArgs& a, hipStream_t st) {
    const int64_t cap = (int64_t)cu_count() * norm_occupancy<kW, kCW, kAdd>();
    const int wgs = (int)std::min<int64_t>(a.M, cap);
    const int tpw = (a.M + wgs - 1) / wgs;                    // tokens per workgroup
    const int blocks = (a.M + tpw - 1) / tpw;                 // every slot owns >= 1 token
    rmsnorm_quant_kernel<kW, kCW, kAdd><<<dim3((unsigned)blocks), dim3(64 * kW), 0, st>>>(a, tpw);
}

// Wavefronts per token: 8 from 8 chunks (4096 columns) up, else 4.
template <bool kAdd>
int launch_norm(const NormArgs& a, hipStream_t st) {
    const int chunks = (a.H + 511) / 512;
    if (chunks <= 4) launch_norm_cfg<4, 1, kAdd>(a, st);
    else if (chunks < 8) launch_norm_cfg<4, 2, kAdd>(a, st);
    else if (chunks <= 8) launch_norm_cfg<8, 1, kAdd>(a, st);
    else if (chunks <= 16) launch_norm_cfg<8, 2, kAdd>(a, st);
    else if (chunks <= 32 && !kAdd) launch_norm_cfg<8, 4, false>(a, st);
    else return 1;
    return 0;
}

// ------------------------------------------------------------- general
// Any H (a multiple of 8) and bf16 / fp16 / fp32 rows, as the reference
// dispatches its kernel over the float types (rmsnorm_quant.cu:111) for any
// hidden size.  The same summation order as rmsnorm_quant_kernel: W
// wavefronts, wavefront w owning the 512-element chunks c = w, w + W, ...,
// 8 elements per lane, fmaf in chunk then element order, the xor butterfly,
// the wavefront sums added in order; inv by the correctly rounded sqrt and
// divide.  The row is read twice (the second time mostly from L2) instead of
// held in registers.  Weight and residual share the input's type.  The fused
// add recomputes r + x in the second pass (the same fp32 sum), rounds it to
// the type, stores it to the residual and normalizes it, so no pass reads
// what another wrote.  Codes always take the clamped conversion (equal to
// the unclamped one for finite rows).  One workgroup per token at a time.
constexpr int kNormBf16 = 0, kNormF16 = 1, kNormF32 = 2;   // element type codes

template <int kT>
constexpr int elt_bytes() { return kT == kNormF32 ? 4 : 2; }

// Eight elements at byte offset `off` as fp32 (reads past the range are zeros).
template <int kT>
__device__ __forceinline__ void load8(__amdgpu_buffer_rsrc_t rs, int off, float (&v)[8]) {
    if constexpr (kT == kNormF32) {
        const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNtLoad);
        const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, kNtLoad);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = __uint_as_float(lo[j]);
            v[4 + j] = __uint_as_float(hi[j]);
        }
    } else {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNtLoad);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (kT == kNormBf16) {
                v[2 * j] = bf16lo(w[j]);
                v[2 * j + 1] = bf16hi(w[j]);
            } else {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const uint32_t word = w[j];   // (a vector element is not a bit_cast operand)
                const h2 h = __builtin_bit_cast(h2, word);
                v[2 * j] = (float)h.x;
                v[2 * j + 1] = (float)h.y;
            }
        }
    }
}

// Two fp32 values rounded to the 16-bit type (nearest even), packed.
template <int kT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (kT == kNormBf16) {
        return pack_bf16_rne(lo, hi);
    } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, h2{(_Float16)lo, (_Float16)hi});
    }
}

// v rounded to the type (nearest even), as fp32.
template <int kT>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (kT == kNormBf16) return __uint_as_float(pack_bf16_rne(v, 0.f) << 16);
    else if constexpr (kT == kNormF16) return (float)(_Float16)v;
    else return v;
}

// Eight fp32 values stored in the type at byte offset `off` (dropped past the range).
template <int kT>
__device__ __forceinline__ void store8(__amdgpu_buffer_rsrc_t rs, int off, const float (&v)[8]) {
    if constexpr (kT == kNormF32) {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])}, rs,
            off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])}, rs,
            off + 16, 0, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{pack2<kT>(v[0], v[1]), pack2<kT>(v[2], v[3]), pack2<kT>(v[4], v[5]), pack2<kT>(v[6], v[7])}, rs,
            off, 0, 0);
    }
}

template <int kW, int kT, bool kAdd>
__global__ __launch_bounds__(64 * kW) void rmsnorm_quant_any_kernel(const NormArgs a) {
#pragma clang fp contract(off)
    __shared__ float part[2][kW];
    constexpr int kB = elt_bytes<kT>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int C = (a.H + 511) / 512;
    const int row_bytes = kB * a.H;
    const __amdgpu_buffer_rsrc_t wr = row_rsrc(a.w, row_bytes);
    const __amdgpu_buffer_rsrc_t sw = row_rsrc(a.s, a.s_bytes);
    int parity = 0;
    for (int m = blockIdx.x; m < a.M; m += gridDim.x, parity ^= 1) {
        const uint8_t* xrow = reinterpret_cast<const uint8_t*>(a.x) + (int64_t)m * a.ld_x * kB;
        const uint8_t* rrow = kAdd ? reinterpret_cast<const uint8_t*>(a.r) + (int64_t)m * a.ld_r * kB : xrow;
        const __amdgpu_buffer_rsrc_t xr = row_rsrc(xrow, row_bytes);
        const __amdgpu_buffer_rsrc_t rr = row_rsrc(rrow, kAdd ? row_bytes : 0);
        const __amdgpu_buffer_rsrc_t qw = row_rsrc(a.q + (int64_t)m * a.ld_q, a.H);
        // ---- pass 1: sum of squares of x (fused add: of r + x, unrounded);
        // lanes past the row read zeros and add nothing
        float p = 0.f;
        for (int c = wave; c < C; c += kW) {
            const int off = kB * (c * 512 + 8 * lane);
            float xv[8], rv[8];
            load8<kT>(xr, off, xv);
            if constexpr (kAdd) load8<kT>(rr, off, rv);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float t = kAdd ? rv[j] + xv[j] : xv[j];
                p = fmaf(t, t, p);
            }
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) p = p + __shfl_xor(p, d, 64);
        if (lane == 0) part[parity][wave] = p;
        __syncthreads();   // (the other parity's slots are free: every wavefront has read them)
        p = part[parity][0];
#pragma unroll
        for (int w = 1; w < kW; ++w) p = p + part[parity][w];
        const float inv = 1.0f / sqrtf(p / (float)a.H + a.eps);
        // ---- pass 2: normalize, quantize, store
        for (int c = wave; c < C; c += kW) {
            const int e0 = c * 512 + 8 * lane;
            const int off = kB * e0;
            float xv[8], rv[8], wv[8], base[8], v[8];
            load8<kT>(xr, off, xv);
            if constexpr (kAdd) load8<kT>(rr, off, rv);
            load8<kT>(wr, off, wv);
#pragma unroll
            for (int j = 0; j < 8; ++j) base[j] = kAdd ? round_to<kT>(rv[j] + xv[j]) : xv[j];
            if constexpr (kAdd) store8<kT>(rr, off, base);   // residual <- r + x in the type
            float amax = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] = (base[j] * inv) * wv[j];
                amax = fmaxf(amax, fabsf(v[j]));
            }
            amax = __uint_as_float(row16_max_u32(__float_as_uint(amax)));
            amax = fmaxf(amax, kGroupEps);
            const float sc = ue8m0_ceil_div448(amax);
            const float is = inv_scale(sc);
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = clamp448(v[j] * is);
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            __builtin_amdgcn_raw_buffer_store_b64(
                u32x2{pack4_e4m3(t[0], t[1], t[2], t[3]), pack4_e4m3(t[4], t[5], t[6], t[7])}, qw, e0, 0, 0);
            const bool owner = (lane & 15) == 0 && e0 < a.H;
            __builtin_amdgcn_raw_buffer_store_b32(
                __float_as_uint(sc), sw, owner ? (int)(4 * ((int64_t)m * a.s_m + (int64_t)(e0 >> 7) * a.s_g)) : kOob,
                0, 0);
            if constexpr (kAdd) store8<kT>(xr, off, v);       // input <- normalized row in the type
        }
    }
}

template <int kW, int kT, bool kAdd>
void launch_norm_any_cfg(const NormArgs& a, hipStream_t st) {
    const int blocks = (int)std::min<int64_t>(a.M, (int64_t)cu_count() * 4);
    rmsnorm_quant_any_kernel<kW, kT, kAdd><<<dim3((unsigned)blocks), dim3(64 * kW), 0, st>>>(a);
}

// W = 8 from 8 chunks (H > 3584) up, else 4, as the fast kernel.
template <int kT, bool kAdd>
void launch_norm_any(const NormArgs& a, hipStream_t st) {
    if ((a.H + 511) / 512 >= 8) launch_norm_any_cfg<8, kT, kAdd>(a, st);
    else launch_norm_any_cfg<4, kT, kAdd>(a, st);
}

}  // namespace
}  // namespace kbn

using namespace kbn;

static int rmsnorm_impl(const char* what, void* x, int x_dtype, int64_t M, int64_t H, int64_t ld_x, const void* w,
                        void* residual, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m,
                        int64_t s_stride_g, float eps, void* stream) {
    const bool add = residual != nullptr;
    KBN_CHECK_ARG(x_dtype == kNormBf16 || x_dtype == kNormF16 || x_dtype == kNormF32,
                  "%s: input dtype code %d (0 bf16, 1 fp16, 2 fp32)", what, x_dtype);
    KBN_CHECK_ARG(M >= 0 && M <= 0x7FFFFFFFLL, "%s: bad M=%lld", what, (long long)M);
    KBN_CHECK_ARG(H > 0 && H % 8 == 0 && H * 4 + 1024 < 0x7FFFFFFFLL,
                  "%s: hidden size %lld must be a positive multiple of 8", what, (long long)H);
    if (M == 0) return 0;
    KBN_CHECK_ARG(x && w && q_fp8 && scale, "%s: null pointer", what);
    KBN_CHECK_ARG(aligned16(x) && aligned16(w) && ld_x >= H && ld_x % 8 == 0,
                  "%s: input and weight must be 16-byte aligned, input row stride >= H and a multiple of 8", what);
    KBN_CHECK_ARG(ld_q >= H && ld_q % 8 == 0 && (reinterpret_cast<uintptr_t>(q_fp8) & 7u) == 0,
                  "%s: output rows must be 8-byte aligned with a stride >= H", what);
    KBN_CHECK_ARG((reinterpret_cast<uintptr_t>(scale) & 3u) == 0, "%s: scales must be 4-byte aligned", what);
    if (add)
        KBN_CHECK_ARG(aligned16(residual) && ld_r >= H && ld_r % 8 == 0,
                      "%s: residual must be 16-byte aligned with a row stride >= H and a multiple of 8", what);
    KBN_CHECK_ARG(s_stride_m >= 0 && s_stride_g >= 0, "%s: negative scale stride", what);
    NormArgs a{};
    a.x = static_cast<uint16_t*>(x);
    a.ld_x = ld_x;
    a.w = static_cast<const uint16_t*>(w);
    a.r = static_cast<uint16_t*>(residual);
    a.ld_r = ld_r;
    a.q = static_cast<uint8_t*>(q_fp8);
    a.ld_q = ld_q;
    a.s = scale;
    a.s_m = s_stride_m;
    a.s_g = s_stride_g;
    const int64_t s_bytes = ((M - 1) * s_stride_m + ((H + 127) / 128 - 1) * s_stride_g + 1) * 4;
    KBN_CHECK_ARG(s_bytes < 0x7FFFFFFFLL, "%s: the scales span 2 GiB or more", what);
    a.s_bytes = (int)s_bytes;
    a.M = (int)M;
    a.H = (int)H;
    a.eps = eps;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // bf16 rows of up to 16384 columns (8192 with the add): the register-
    // resident kernel; everything else: the general one (same order)
    const int64_t fast_h = add ? 8192 : 16384;
    if (x_dtype == kNormBf16 && H <= fast_h) {
        if (add ? launch_norm<true>(a, st) : launch_norm<false>(a, st)) {
            set_error("%s: no kernel for hidden size %lld", what, (long long)H);
            return 1;
        }
    } else if (x_dtype == kNormBf16) {
        if (add) launch_norm_any<kNormBf16, true>(a, st);
        else launch_norm_any<kNormBf16, false>(a, st);
    } else if (x_dtype == kNormF16) {
        if (add) launch_norm_any<kNormF16, true>(a, st);
        else launch_norm_any<kNormF16, false>(a, st);
    } else {
        if (add) launch_norm_any<kNormF32, true>(a, st);
        else launch_norm_any<kNormF32, false>(a, st);
    }
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_rmsnorm_fp8_quant(void* x_bf16, int64_t M, int64_t H, int64_t ld_x, const void* w_bf16,
                                     void* residual_bf16, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale,
                                     int64_t s_stride_m, int64_t s_stride_g, float eps, void* stream) {
    return rmsnorm_impl(residual_bf16 ? "fused_add_rmsnorm_fp8_quant" : "rmsnorm_fp8_quant", x_bf16, kNormBf16, M, H,
                        ld_x, w_bf16, residual_bf16, ld_r, q_fp8, ld_q, scale, s_stride_m, s_stride_g, eps, stream);
}

extern "C" int kbn_rmsnorm_fp8_quant_typed(void* x, int x_dtype, int64_t M, int64_t H, int64_t ld_x, const void* w,
                                           void* residual, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale,
                                           int64_t s_stride_m, int64_t s_stride_g, float eps, void* stream) {
    return rmsnorm_impl(residual ? "fused_add_rmsnorm_fp8_quant" : "rmsnorm_fp8_quant", x, x_dtype, M, H, ld_x, w,
                        residual, ld_r, q_fp8, ld_q, scale, s_stride_m, s_stride_g, eps, stream);
}
