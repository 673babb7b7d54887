/*
 * CPU oracle for the block-scaled FP8 linear path.  TEST INFRASTRUCTURE ONLY:
 * it is loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg as the checker.  The product path (kb_nano_amd) never links or calls it.
 *
 * Each routine restates the reference algorithm it cites (paths relative to
 * the kb_nano tree):
 *
 *   orc_e4m3_encode        torch `.to(float8_e4m3fn)` as used after the clamp in
 *                          tasks/reference/L1/fp8_linear.py:63 and
 *                          bench/kernels/scenario_registry.py:178-180
 *                          (round-to-nearest-even, subnormals kept, NaN above 464).
 *   orc_ue8m0_from_ratio   s = 2^ceil(log2(amax/448)) from
 *                          tasks/baseline/L1/fp8_linear.py:203-205 and
 *                          tasks/reference/L1/fp8_linear.py:59-61, derived from the
 *                          exponent bits of the IEEE quotient.
 *   orc_quant_group128     tasks/baseline/L1/fp8_linear.py:181-215 (one 1x128 group:
 *                          absmax, eps clamp, scale, divide, clamp, cast) with the
 *                          stride-addressed scale store of :214-215.
 *   orc_quant_group128_f32 the same on fp32 values: fp16 and fp32 inputs, which
 *                          :197 widens to fp32 (exactly) before the absmax.
 *   orc_silu_bf16          tasks/baseline/L1/silu_mul_quant_fp8.py:57-59, silu rounded
 *                          once to bf16; pinned here as the correctly rounded value
 *                          of g/(1+e^-g) (evaluated in double).
 *   orc_silu_mul_quant     tasks/baseline/L1/silu_mul_quant_fp8.py:48-76 (gate at
 *                          column n, up at n + N/2, y = bf16(silu*up), 1x128 quant,
 *                          scale at s[g*col_stride + m]).
 *   orc_gemm_nt_sample     D[m,n] = sum_kb sA[m,kb]*sW[n/128,kb]*sum_k A[m,k]W[n,k]
 *                          (the fp8_gemm_nt contract at fp8_linear.py:97-110, with
 *                          the weight-scale expansion of
 *                          tasks/reference/L1/fp8_linear.py:26-38); double accumulate.
 *   orc_grouped_gemm_nt_sample
 *                          the contiguous grouped contract of
 *                          tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:136-170:
 *                          row r uses expert expert_ids[r]; rows with -1 are skipped.
 *   orc_rmsnorm_quant      tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-93 and :124-201
 *                          (RMSNorm, optional residual add, UE8M0 1x128 quant of the
 *                          fp32 normalized values), in a fixed fp32 reduction order.
 *   orc_rmsnorm_quant_f32  the same for bf16, fp16 or fp32 rows (the kernel's type
 *                          dispatch, :111), with orc_float_to_f16 / orc_f16_to_float.
 *
 * Everything is plain scalar C99 on the host; no GPU code.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_float(uint16_t h) { return u2f(((uint32_t)h) << 16); }

/* Round a float to bf16 with round-to-nearest-even (NaN kept quiet). */
uint16_t orc_float_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* IEEE binary16: decode, and round a float to it (nearest even; fp16
 * subnormals kept, magnitudes from 65520 up to infinity, NaN kept quiet). */
float orc_f16_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    float v;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) v = ldexpf((float)m, -24);
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return sign ? -v : v;
}

uint16_t orc_float_to_f16(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u | (uint16_t)((a >> 13) & 0x3FFu);
    if (a >= 0x477FF000u) return sign | 0x7C00u;          /* >= 65520: infinity (ties to the even 2^16) */
    if (a < 0x38800000u) {                                /* below 2^-14: multiples of 2^-24 */
        const float t = u2f(a) * 16777216.0f;             /* exact */
        return sign | (uint16_t)nearbyintf(t);            /* round to nearest even; 1024 is 2^-14 */
    }
    uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13));
    const uint32_t rest = a & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1;
    return sign | (uint16_t)h;
}

/* Round a double to bf16 directly (one rounding, RNE), including bf16
 * subnormals and overflow to infinity. */
uint16_t orc_double_to_bf16(double d) {
    if (isnan(d)) return 0x7FC0;
    uint16_t sign = signbit(d) ? 0x8000 : 0;
    double a = fabs(d);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e);             /* a = f * 2^e, f in [0.5, 1) */
    int exp_unbiased = e - 1; /* a in [2^(e-1), 2^e) */
    int q = exp_unbiased - 7; /* quantum: 8 significant bits */
    if (q < -133) q = -133;   /* bf16 subnormal quantum is 2^-133 */
    double scaled = ldexp(a, -q);      /* exact (power-of-two scaling) */
    double r = nearbyint(scaled);      /* default rounding mode: RNE */
    double v = ldexp(r, q);
    if (v >= 0x1p128) return sign | 0x7F80;
    /* v is exactly representable in bf16; convert via float (exact). */
    float fv = (float)v;
    return sign | (uint16_t)(f2u(fv) >> 16);
}

/* fp8 e4m3fn (OCP): bias 7, no infinities, NaN = S.1111.111, max 448. */
uint8_t orc_e4m3_encode(float x) {
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    if (isnan(x)) return sign | 0x7F;
    float a = fabsf(x);
    if (a > 464.0f) return sign | 0x7F;  /* rounds past 448 -> NaN (no inf) */
    if (a < 0x1p-6f) {
        /* subnormal range: value = m * 2^-9, m in [0,8] */
        float m = nearbyintf(a * 512.0f);  /* exact scale, RNE */
        int mi = (int)m;
        if (mi >= 8) return sign | 0x08;   /* rounds up to the min normal */
        return sign | (uint8_t)mi;
    }
    uint32_t au = f2u(a);
    int e = (int)((au >> 23) & 0xFF) - 127; /* -6 .. 8 */
    uint32_t mant = au & 0x7FFFFFu;
    uint32_t keep = mant >> 20;
    uint32_t rest = mant & 0xFFFFFu;
    uint32_t half = 0x80000u;
    if (rest > half || (rest == half && (keep & 1u))) keep += 1;
    if (keep == 8) { keep = 0; e += 1; }
    if (e > 8 || (e == 8 && keep == 7)) return sign | 0x7F; /* cannot happen for a <= 464 except tie */
    return sign | (uint8_t)(((e + 7) << 3) | keep);
}

float orc_e4m3_decode(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 0xF, m = c & 7;
    float v;
    if (e == 0xF && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

/* UE8M0 scale for a positive ratio r = amax/448: the smallest power of two
 * >= r.  Exponent bits of r, plus one when the mantissa is non-zero. */
float orc_ue8m0_from_ratio(float r) {
    uint32_t u = f2u(r);
    uint32_t e = (u >> 23) & 0xFF;
    uint32_t m = u & 0x7FFFFFu;
    if (e == 0) {
        /* subnormal ratio: ceil to a power of two via frexp (exact) */
        if (m == 0) return 0.0f;
        int ex; float f = frexpf(r, &ex);
        return (f == 0.5f) ? r : ldexpf(1.0f, ex);
    }
    if (m) e += 1;
    return u2f(e << 23);
}

static inline float group_scale(float amax, float eps, int use_ue8m0) {
    if (amax < eps) amax = eps;      /* max(absmax, eps); NaN propagates as in fmax? keep simple */
    float r = amax / 448.0f;
    return use_ue8m0 ? orc_ue8m0_from_ratio(r) : r;
}

static inline uint8_t quant_one(float x, float s) {
    float v = x / s;
    if (v > 448.0f) v = 448.0f;
    if (v < -448.0f) v = -448.0f;
    return orc_e4m3_encode(v);
}

/* Per-token-group quantization of a bf16 [M,K] matrix (K % 128 == 0). */
int orc_quant_group128(const uint16_t* x, int64_t M, int64_t K, int64_t ld_x,
                       uint8_t* q, int64_t ld_q, float* s, int64_t s_stride_m,
                       int64_t s_stride_g, float eps, int use_ue8m0) {
    if (K % 128) return 1;
    int64_t G = K / 128;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < G; ++g) {
            const uint16_t* xr = x + m * ld_x + g * 128;
            float v[128];
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) {
                v[i] = orc_bf16_to_float(xr[i]);
                float a = fabsf(v[i]);
                if (a > amax) amax = a;
            }
            float sc = group_scale(amax, eps, use_ue8m0);
            uint8_t* qr = q + m * ld_q + g * 128;
            for (int i = 0; i < 128; ++i) qr[i] = quant_one(v[i], sc);
            s[m * s_stride_m + g * s_stride_g] = sc;
        }
    }
    return 0;
}

/* The same quantization of fp32 values [M,K] (K % 128 == 0): fp16 and fp32
 * inputs, which the reference's kernel widens to fp32 before the absmax
 * (tasks/baseline/L1/fp8_linear.py:197); the widening is exact, so the
 * caller passes the fp32 values. */
int orc_quant_group128_f32(const float* x, int64_t M, int64_t K, int64_t ld_x,
                           uint8_t* q, int64_t ld_q, float* s, int64_t s_stride_m,
                           int64_t s_stride_g, float eps, int use_ue8m0) {
    if (K % 128) return 1;
    int64_t G = K / 128;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < G; ++g) {
            const float* xr = x + m * ld_x + g * 128;
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) {
                float a = fabsf(xr[i]);
                if (a > amax) amax = a;
            }
            float sc = group_scale(amax, eps, use_ue8m0);
            uint8_t* qr = q + m * ld_q + g * 128;
            for (int i = 0; i < 128; ++i) qr[i] = quant_one(xr[i], sc);
            s[m * s_stride_m + g * s_stride_g] = sc;
        }
    }
    return 0;
}

/* silu(g) rounded once to bf16, evaluated in double. */
uint16_t orc_silu_bf16(uint16_t gbits) {
    double g = (double)orc_bf16_to_float(gbits);
    if (isnan(g)) return 0x7FC0;
    double r;
    if (isinf(g)) return orc_double_to_bf16(g > 0 ? g : -0.0);
    if (fabs(g) < 0x1p-64) {
        /* silu(g) = g/2 * (1 + g/2 + O(g^2)): the relative perturbation g/2 is
         * far below double precision, so decide ties explicitly.  g/2 is a
         * bf16 tie only for subnormal g with an odd last bit; the exact value
         * then lies just above the tie in magnitude for g > 0 and just below
         * it for g < 0. */
        double half = g * 0.5;
        uint16_t h = orc_double_to_bf16(half);
        if ((double)orc_bf16_to_float(h) == half) return h;
        double q = 0x1p-133;
        double lo = floor(fabs(half) / q) * q;
        return orc_double_to_bf16(copysign(g > 0 ? lo + q : lo, g));
    }
    r = g / (1.0 + exp(-g));
    return orc_double_to_bf16(r);
}

/* Fused silu(gate)*up + per-token-group quant.  Input bf16 [M, 2*Nh] with row
 * stride ld_in; gate = columns [0,Nh), up = [Nh, 2Nh). */
int orc_silu_mul_quant(const uint16_t* in, int64_t M, int64_t Nh, int64_t ld_in,
                       uint8_t* q, int64_t ld_q, float* s, int64_t s_stride_m,
                       int64_t s_stride_g, float eps, int use_ue8m0) {
    if (Nh % 128) return 1;
    int64_t G = Nh / 128;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* row = in + m * ld_in;
        for (int64_t g = 0; g < G; ++g) {
            float y[128];
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) {
                int64_t n = g * 128 + i;
                uint16_t sb = orc_silu_bf16(row[n]);
                float prod = orc_bf16_to_float(sb) * orc_bf16_to_float(row[n + Nh]); /* exact */
                y[i] = orc_bf16_to_float(orc_float_to_bf16(prod));
                float a = fabsf(y[i]);
                if (a > amax) amax = a;
            }
            float sc = group_scale(amax, eps, use_ue8m0);
            uint8_t* qr = q + m * ld_q + g * 128;
            for (int i = 0; i < 128; ++i) qr[i] = quant_one(y[i], sc);
            s[m * s_stride_m + g * s_stride_g] = sc;
        }
    }
    return 0;
}

static double e4m3_lut[256];
static int e4m3_lut_ready = 0;
static void ensure_lut(void) {
    if (e4m3_lut_ready) return;
    for (int i = 0; i < 256; ++i) e4m3_lut[i] = (double)orc_e4m3_decode((uint8_t)i);
    e4m3_lut_ready = 1;
}

/* Scale transform applied by the GEMM contract: mode 0 uses fp32 scales as
 * given; mode 1 (UE8M0 contract) rounds each scale up to a power of two. */
static inline double gemm_scale(float s, int ue8m0) {
    if (!ue8m0) return (double)s;
    return (double)orc_ue8m0_from_ratio(s);
}

/* Block-scaled NT GEMM evaluated at selected (row, col) pairs of the output
 * grid rows x cols.  out is fp32 [nrows, ncols] holding the double result
 * rounded to float (callers round to bf16 for comparisons). */
int orc_gemm_nt_sample(const uint8_t* A, int64_t lda, const float* sA, int64_t sA_sm, int64_t sA_sk,
                       const uint8_t* W, int64_t ldw, const float* sW, int64_t sW_ld,
                       int64_t M, int64_t N, int64_t K,
                       const int64_t* rows, int64_t nrows, const int64_t* cols, int64_t ncols,
                       double* out, int ue8m0) {
    if (K % 128) return 1;
    ensure_lut();
    int64_t KB = K / 128;
    for (int64_t i = 0; i < nrows; ++i)
        if (rows[i] < 0 || rows[i] >= M) return 2;
    for (int64_t j = 0; j < ncols; ++j)
        if (cols[j] < 0 || cols[j] >= N) return 3;
#pragma omp parallel for schedule(dynamic, 1) if (nrows > 1)
    for (int64_t i = 0; i < nrows; ++i) {
        int64_t m = rows[i];
        for (int64_t j = 0; j < ncols; ++j) {
            int64_t n = cols[j];
            double acc = 0.0;
            for (int64_t kb = 0; kb < KB; ++kb) {
                const uint8_t* a = A + m * lda + kb * 128;
                const uint8_t* w = W + n * ldw + kb * 128;
                double p = 0.0;
                for (int k = 0; k < 128; ++k) p += e4m3_lut[a[k]] * e4m3_lut[w[k]];
                acc += p * gemm_scale(sA[m * sA_sm + kb * sA_sk], ue8m0) *
                       gemm_scale(sW[(n / 128) * sW_ld + kb], ue8m0);
            }
            out[i * ncols + j] = acc;
        }
    }
    return 0;
}

/* Contiguous grouped GEMM at selected rows/cols.  B is [E, N, K] fp8 and
 * sB is [E, ceil(N/128), K/128].  Rows whose expert id is negative yield NaN
 * (the contract leaves them unwritten). */
int orc_grouped_gemm_nt_sample(const uint8_t* A, const float* sA, int64_t sA_sm, int64_t sA_sk,
                               const uint8_t* B, const float* sB, const int32_t* expert_ids,
                               int64_t M_sum, int64_t N, int64_t K, int64_t E,
                               const int64_t* rows, int64_t nrows, const int64_t* cols, int64_t ncols,
                               double* out, int ue8m0) {
    if (K % 128) return 1;
    int64_t NB = (N + 127) / 128, KB = K / 128;
    for (int64_t i = 0; i < nrows; ++i) {
        int64_t r = rows[i];
        if (r < 0 || r >= M_sum) return 2;
        int32_t e = expert_ids[r];
        if (e >= E) return 4;
        if (e < 0) {
            for (int64_t j = 0; j < ncols; ++j) out[i * ncols + j] = NAN;
            continue;
        }
        int rc = orc_gemm_nt_sample(A + r * K, K, sA + r * sA_sm, 0, sA_sk,
                                    B + (int64_t)e * N * K, K, sB + (int64_t)e * NB * KB, KB,
                                    1, N, K, &(int64_t){0}, 1, cols, ncols, out + i * ncols, ue8m0);
        if (rc) return rc;
    }
    return 0;
}

/* Fused RMSNorm + 1x128 FP8 quantization, plain and with residual add
 * (tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-93 and :124-201, module
 * tasks/baseline/L1/rmsnorm_quant.py:27-55):
 *   plain:  a = x;  base = x
 *   fused:  a = fp32(r) + fp32(x) (unrounded);  r <- bf16(a);  base = fp32(bf16(a))
 *   inv  = 1 / sqrt(sum(a^2) / H + eps)
 *   v    = (base * inv) * w            (two fp32 products, not rounded to bf16)
 *   per 128-group: amax = max(max|v|, 1e-10); s = ceil_pow2(amax / 448);
 *   q = e4m3_rne(fminf(fmaxf(v / s, -448), 448)); fused: x <- bf16(v)
 * The reference sums in whatever order its thread layout gives and takes
 * rsqrtf; this restatement fixes the order the gfx950 kernel uses, so the
 * kernel can be checked bit for bit: W groups of 64 lanes (W = 8 when the row
 * has at least 8 chunks of 512, i.e. H > 3584, else 4); lane l of group w
 * owns the 8-element chunks starting at c*512 + 8l for c = w, w+W, w+2W, ...,
 * accumulates a*a with fmaf in chunk then element order; each group's 64
 * partials are combined by the xor butterfly p[l] + p[l ^ d] for d = 32, 16,
 * ..., 1, and the group sums in group order, ((P0 + P1) + P2) + ... .  inv
 * uses the correctly rounded sqrt and divide.  r == NULL selects the plain
 * variant.
 * H % 8 == 0; scale (m, g) at s[m*s_m + g*s_g] for g < ceil(H/128). */
int orc_rmsnorm_quant(uint16_t* x, int64_t M, int64_t H, int64_t ld_x, const uint16_t* w, uint16_t* r,
                      int64_t ld_r, uint8_t* q, int64_t ld_q, float* s, int64_t s_m, int64_t s_g, float eps) {
    if (H <= 0 || H % 8) return 1;
    const int64_t G = (H + 127) / 128, C = (H + 511) / 512;
    int bad = 0;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        float* base = (float*)malloc((size_t)H * sizeof(float));
        if (!base) { bad = 1; continue; }
        uint16_t* xr = x + m * ld_x;
        uint16_t* rr = r ? r + m * ld_r : NULL;
        const int W = C >= 8 ? 8 : 4;
        float P[8];
        for (int wv = 0; wv < W; ++wv) {
        float part[64];
        for (int l = 0; l < 64; ++l) {
            float p = 0.0f;
            for (int64_t c = wv; c < C; c += W) {
                const int64_t e0 = c * 512 + 8 * l;
                if (e0 >= H) continue;
                for (int j = 0; j < 8; ++j) {
                    const int64_t e = e0 + j;
                    const float xv = orc_bf16_to_float(xr[e]);
                    float a = xv;
                    if (rr) {
                        a = orc_bf16_to_float(rr[e]) + xv;
                        rr[e] = orc_float_to_bf16(a);
                        base[e] = orc_bf16_to_float(rr[e]);
                    } else {
                        base[e] = xv;
                    }
                    p = fmaf(a, a, p);
                }
            }
            part[l] = p;
        }
        for (int d = 32; d >= 1; d >>= 1) {
            float t[64];
            for (int l = 0; l < 64; ++l) t[l] = part[l] + part[l ^ d];
            memcpy(part, t, sizeof(t));
        }
        P[wv] = part[0];
        }
        float ptot = P[0];
        for (int wv = 1; wv < W; ++wv) ptot = ptot + P[wv];
        const float mean = ptot / (float)H;
        const float inv = 1.0f / sqrtf(mean + eps);
        for (int64_t g = 0; g < G; ++g) {
            const int64_t e1 = (g + 1) * 128 < H ? (g + 1) * 128 : H;
            float amax = 0.0f;
            for (int64_t e = g * 128; e < e1; ++e) {
                const float v = (base[e] * inv) * orc_bf16_to_float(w[e]);
                const float av = fabsf(v);
                if (av > amax) amax = av;
            }
            const float sc = group_scale(amax, 1e-10f, 1);
            for (int64_t e = g * 128; e < e1; ++e) {
                const float v = (base[e] * inv) * orc_bf16_to_float(w[e]);
                /* the reference clamps with fminf(fmaxf(.)) (rmsnorm_quant.cu:82):
                 * a NaN quotient becomes -448 */
                q[m * ld_q + e] = orc_e4m3_encode(fminf(fmaxf(v / sc, -448.0f), 448.0f));
                if (rr) xr[e] = orc_float_to_bf16(v);
            }
            s[m * s_m + g * s_g] = sc;
        }
        free(base);
    }
    return bad ? 2 : 0;
}

/* v rounded to bf16 (rnd 0) or fp16 (rnd 1) and back; fp32 (rnd 2) as is. */
static inline float round_type(float v, int rnd) {
    if (rnd == 0) return orc_bf16_to_float(orc_float_to_bf16(v));
    if (rnd == 1) return orc_f16_to_float(orc_float_to_f16(v));
    return v;
}

/* orc_rmsnorm_quant for rows of bf16, fp16 or fp32 (rnd 0 / 1 / 2; the
 * reference dispatches its kernel over the float types,
 * rmsnorm_quant.cu:111): x, w and r hold the fp32 values of the type's
 * numbers; the residual sum and the normalized row written back are rounded
 * to the type.  The same fixed summation order as orc_rmsnorm_quant. */
int orc_rmsnorm_quant_f32(float* x, int64_t M, int64_t H, int64_t ld_x, const float* w, float* r,
                          int64_t ld_r, uint8_t* q, int64_t ld_q, float* s, int64_t s_m, int64_t s_g, float eps,
                          int rnd) {
    if (H <= 0 || H % 8 || rnd < 0 || rnd > 2) return 1;
    const int64_t G = (H + 127) / 128, C = (H + 511) / 512;
    int bad = 0;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        float* base = (float*)malloc((size_t)H * sizeof(float));
        if (!base) { bad = 1; continue; }
        float* xr = x + m * ld_x;
        float* rr = r ? r + m * ld_r : NULL;
        const int W = C >= 8 ? 8 : 4;
        float P[8];
        for (int wv = 0; wv < W; ++wv) {
            float part[64];
            for (int l = 0; l < 64; ++l) {
                float p = 0.0f;
                for (int64_t c = wv; c < C; c += W) {
                    const int64_t e0 = c * 512 + 8 * l;
                    if (e0 >= H) continue;
                    for (int j = 0; j < 8; ++j) {
                        const int64_t e = e0 + j;
                        float a = xr[e];
                        if (rr) {
                            a = rr[e] + xr[e];
                            rr[e] = round_type(a, rnd);
                            base[e] = rr[e];
                        } else {
                            base[e] = a;
                        }
                        p = fmaf(a, a, p);
                    }
                }
                part[l] = p;
            }
            for (int d = 32; d >= 1; d >>= 1) {
                float t[64];
                for (int l = 0; l < 64; ++l) t[l] = part[l] + part[l ^ d];
                memcpy(part, t, sizeof(t));
            }
            P[wv] = part[0];
        }
        float ptot = P[0];
        for (int wv = 1; wv < W; ++wv) ptot = ptot + P[wv];
        const float inv = 1.0f / sqrtf(ptot / (float)H + eps);
        for (int64_t g = 0; g < G; ++g) {
            const int64_t e1 = (g + 1) * 128 < H ? (g + 1) * 128 : H;
            float amax = 0.0f;
            for (int64_t e = g * 128; e < e1; ++e) {
                const float v = (base[e] * inv) * w[e];
                const float av = fabsf(v);
                if (av > amax) amax = av;
            }
            const float sc = group_scale(amax, 1e-10f, 1);
            for (int64_t e = g * 128; e < e1; ++e) {
                const float v = (base[e] * inv) * w[e];
                q[m * ld_q + e] = orc_e4m3_encode(fminf(fmaxf(v / sc, -448.0f), 448.0f));
                if (rr) xr[e] = round_type(v, rnd);
            }
            s[m * s_m + g * s_g] = sc;
        }
        free(base);
    }
    return bad ? 2 : 0;
}
