/*
 * kbn_fp8.h -- C-ABI of libkbn_fp8.so, the MI355X (gfx950) implementation of
 * kb_nano's block-scaled FP8 linear path.
 *
 * Conventions for every entry point:
 *   - Plain device pointers and sizes; bf16 and fp8 buffers are passed as
 *     void* (bf16 = 16-bit bfloat16 bit patterns, fp8 = OCP float8_e4m3fn).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Calls are
 *     asynchronous on that stream; they never allocate, free or synchronise,
 *     so they may be captured into HIP graphs and may run concurrently on
 *     different streams.  The caller owns every buffer.
 *   - Return 0 on success.  A non-zero code means the arguments were
 *     rejected (1) or the launch failed (2); kbn_last_error() then holds a
 *     message (thread-local).  Nothing is launched when arguments are rejected.
 *   - Strides are in elements of the buffer's type.
 *
 * Paths cited below are relative to the kb_nano tree.
 */
#ifndef KBN_FP8_H
#define KBN_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char* kbn_last_error(void);

/* ABI revision of this header (1). */
int kbn_abi_version(void);

/* gcnArchName of a HIP device into buf (e.g. "gfx950:sramecc+:xnack-"). */
int kbn_device_arch(int device, char* buf, int len);

/*
 * Per-token-group (1x128) FP8 quantization.
 * Replaces _per_token_group_quant_fp8 / op kb_nano_fp8::per_token_group_quant_fp8
 * (tasks/baseline/L1/fp8_linear.py:157-178, :234-279; kernel :181-215).
 *   x       bf16 [M, K], row stride ld_x (multiple of 8, 16-byte aligned), K % 128 == 0
 *   q       fp8  [M, K], row stride ld_q (multiple of 8)
 *   scale   fp32 [M, K/128]; element (m, g) at scale[m*s_stride_m + g*s_stride_g]
 *           (row-major: (K/128, 1); column-major: (1, M))
 *   For each group: amax = max(max|x|, eps); s = amax/448, rounded up to a
 *   power of two when use_ue8m0; q = e4m3_rne(clamp(x/s, -448, 448)).
 */
int kbn_per_token_group_quant_fp8(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x,
                                  void* q_fp8, int64_t ld_q, float* scale,
                                  int64_t s_stride_m, int64_t s_stride_g,
                                  float eps, int use_ue8m0, void* stream);

/*
 * The same quantization of fp16 or fp32 rows (and bf16): the reference's
 * kernel loads any float input and widens it to fp32 before the group
 * absmax (tasks/baseline/L1/fp8_linear.py:197), which is exact for these
 * types, so each group's codes and scale are those of the fp32 values.
 *   x_dtype 0 bf16, 1 fp16, 2 fp32; x rows 16-byte aligned, ld_x % 8 == 0
 *   (elements); every other argument as kbn_per_token_group_quant_fp8.
 */
int kbn_per_token_group_quant_fp8_typed(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ld_x,
                                        void* q_fp8, int64_t ld_q, float* scale,
                                        int64_t s_stride_m, int64_t s_stride_g,
                                        float eps, int use_ue8m0, void* stream);

/*
 * Fused SiLU*Mul + per-token-group FP8 quantization.
 * Replaces the Triton kernel _silu_mul_per_token_group_quant_fp8_colmajor and
 * SiluMulQuantFp8.forward (tasks/baseline/L1/silu_mul_quant_fp8.py:23-76, :87-143).
 *   in      bf16 [M, 2*N_half] = [gate | up], row stride ld_in (multiple of 8)
 *   q       fp8  [M, N_half], row stride ld_q;  N_half % 128 == 0
 *   scale   fp32 [M, N_half/128] at scale[m*s_stride_m + g*s_stride_g]
 *   y = bf16(bf16(silu(gate)) * up) with silu correctly rounded to bf16,
 *   then quantized per 1x128 group as above.
 */
int kbn_silu_mul_quant_fp8(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in,
                           void* q_fp8, int64_t ld_q, float* scale,
                           int64_t s_stride_m, int64_t s_stride_g,
                           float eps, int use_ue8m0, void* stream);

/*
 * kbn_silu_mul_quant_fp8 over the rows whose id is not negative: rows r with
 * row_ids[r] < 0 are neither read nor written (int32 row_ids[M], device
 * memory).  No counterpart in the reference: FusedExperts (fused_experts.py:
 * 246-283) runs SiLU*Mul+quant over all M_sum rows of the contiguous layout,
 * whose padding rows (expert id -1) GEMM1 never wrote and GEMM2 never reads;
 * with the expert ids as row ids those rows cost no traffic.
 */
int kbn_silu_mul_quant_fp8_rows(const void* in_bf16, int64_t M, int64_t N_half, int64_t ld_in,
                                void* q_fp8, int64_t ld_q, float* scale,
                                int64_t s_stride_m, int64_t s_stride_g,
                                float eps, int use_ue8m0, const int32_t* row_ids, void* stream);

/*
 * Block-scaled FP8 GEMM, "NT" (both operands K-contiguous).
 * Replaces op kb_nano_fp8::fp8_gemm_nt -> deep_gemm.fp8_gemm_nt
 * (tasks/baseline/L1/fp8_linear.py:89-118).
 *   A    fp8 [M, K] row stride lda;  sA fp32 [M, K/128] at sA[m*sA_stride_m + kb*sA_stride_k]
 *   W    fp8 [N, K] row stride ldw;  sW fp32 [ceil(N/128), K/128] row stride sW_ld
 *   D    bf16 [M, N] row stride ldd (written)
 *   D[m,n] = bf16_rne( sum_kb sA[m,kb] * sW[n/128,kb] * sum_{k in kb} A[m,k] * W[n,k] ), fp32 accumulate.
 *   scale_ue8m0 != 0: every scale is first rounded up to a power of two (the
 *   UE8M0 contract, DeepGEMM's disable_ue8m0_cast=False); 0: scales used as given.
 *   K % 128 == 0; A/W rows 16-byte aligned (lda, ldw multiples of 16).
 */
int kbn_fp8_gemm_nt(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m, int64_t sA_stride_k,
                    const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                    void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K,
                    int scale_ue8m0, void* stream);

/*
 * kbn_fp8_gemm_nt with a caller-provided workspace: shapes whose tile grid
 * would leave CUs idle (small M, or few N tiles) split K across workgroups,
 * write fp32 partial sums into `workspace` and sum them in a fixed order (so
 * results are deterministic and equal for any split count up to fp32
 * summation order): for few rows (M <= 32; up to 64 with short, shallow
 * splits) the last workgroup of each tile does it in
 * the same launch, using per-tile arrival counters the library keeps in a
 * static device array per stream (per capturing stream under capture,
 * streams forked into one capture included); otherwise, or
 * when those run out, a second launch on the same stream does it.
 * kbn_fp8_gemm_nt_workspace_bytes returns the bytes this needs for a shape on
 * the current device (0: no split, workspace unused).  A null or smaller
 * workspace runs the unsplit kernel.  The workspace must be 16-byte aligned
 * and must not be used by another call that may run concurrently.
 * No counterpart in the reference (DeepGEMM allocates internally); this is
 * the entry point the Python op kb_nano_fp8::fp8_gemm_nt calls, with a
 * workspace from the PyTorch caching allocator.
 */
int64_t kbn_fp8_gemm_nt_workspace_bytes(int64_t M, int64_t N, int64_t K, int scale_ue8m0);
int kbn_fp8_gemm_nt_ws(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m, int64_t sA_stride_k,
                       const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                       void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K,
                       int scale_ue8m0, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * kbn_fp8_gemm_nt_ws with DeepGEMM's packed per-row UE8M0 weight scales, the
 * layout transform_sf_into_required_layout gives postprocess_fp8_weights
 * (tasks/baseline/L1/fp8_linear.py:501-510) and the layout of the
 * reference's own fp8_linear benchmark scenarios (weight_scale_inv int32
 * [N, ceil(K/512)], bench/kernels/benchmark_scenarios/small/
 * shape_registry.yaml:18719-18737).
 *   sW_packed  int32 [N, ceil(K/512)] at sW_packed[n*sWp_stride_n + i*sWp_stride_k]
 *              (any strides, e.g. DeepGEMM's MN-major (1, aligned N)); byte j
 *              (little-endian) of word (n, i) is the E8M0 exponent e of weight
 *              row n for K block 4i + j, i.e. the scale 2^(e-127)
 *   D[m,n] = bf16_rne( sum_kb ue8m0(sA[m,kb]) * 2^(e(n,kb)-127) * sum_{k in kb} A[m,k] * W[n,k] )
 * The exponents go to the block-scaled MFMA per lane (one weight row per
 * lane), so with the exponents of 128x128 block scales repeated on every row
 * of their block the result is kbn_fp8_gemm_nt_ws's with those block scales
 * (scale_ue8m0 = 1), bit for bit.  Workspace as kbn_fp8_gemm_nt_ws's, sized by
 * kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1).
 */
int kbn_fp8_gemm_nt_packed_ws(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m, int64_t sA_stride_k,
                              const void* W, int64_t ldw, const int32_t* sW_packed, int64_t sWp_stride_n,
                              int64_t sWp_stride_k, void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K,
                              void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fp8Linear.forward's quant + GEMM in one call (tasks/baseline/L1/
 * fp8_linear.py:436-445: per_token_group_quant_fp8 into column-major scales,
 * then fp8_gemm_nt): kbn_per_token_group_quant_fp8(x -> q, scale; eps,
 * quant_ue8m0), then kbn_fp8_gemm_nt_ws(q, scale, W, sW -> D; scale_ue8m0,
 * workspace), launched on `stream` in that order.  The arguments of both
 * are checked before either launches.  One host crossing instead of two,
 * for the eager decode path where the launch path, not the GPU, sets the
 * time per layer.
 */
int kbn_fp8_linear_forward(const void* x_bf16, int64_t M, int64_t K, int64_t ld_x,
                           void* q_fp8, int64_t ld_q, float* scale, int64_t s_stride_m, int64_t s_stride_g,
                           float eps, int quant_ue8m0, const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                           void* D_bf16, int64_t ldd, int64_t N, int scale_ue8m0,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Block-scaled GEMM over bf16 activations, M <= 64, the activation quant done
 * inside the GEMM kernel.  Replaces op kb_nano_fp8::flashinfer_blockscale_gemm
 * (tasks/baseline/L1/fp8_linear.py:126-153), the bf16-input GEMM that
 * Fp8Linear.forward takes for M < 32 (:398-417; FlashInfer's SM90 kernel,
 * which quantizes its input itself).
 *   x  bf16 [M, K] row stride ld_x (elements, 16-byte aligned rows)
 *   W, sW, D as kbn_fp8_gemm_nt; eps as kbn_per_token_group_quant_fp8
 * Every 1x128 group of x is quantized exactly as kbn_per_token_group_quant_fp8
 * does with use_ue8m0 = 1 (same codes, same power-of-two scales), and the
 * product is the UE8M0 contract of kbn_fp8_gemm_nt: D equals that quant
 * followed by kbn_fp8_gemm_nt_ws bit for bit.  No fp8 copy of x is written.
 * M > 64 is rejected (code 1).  The workspace is as kbn_fp8_gemm_nt_ws's
 * (split-K slabs; kbn_fp8_gemm_bf16a_workspace_bytes, 0 if none is needed;
 * a smaller workspace runs the shape without split).
 */
int64_t kbn_fp8_gemm_bf16a_workspace_bytes(int64_t M, int64_t N, int64_t K);
/* 1 when kbn_fp8_gemm_bf16a is expected to be faster on the current device
 * than kbn_fp8_linear_forward (quant + GEMM) for this shape, else 0 (also for
 * shapes kbn_fp8_gemm_bf16a rejects).  Fp8Linear.forward routes by it. */
int kbn_fp8_gemm_bf16a_preferred(int64_t M, int64_t N, int64_t K);
int kbn_fp8_gemm_bf16a(const void* x_bf16, int64_t ld_x, float eps, const void* W, int64_t ldw,
                       const float* sW, int64_t sW_ld, void* D_bf16, int64_t ldd,
                       int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * kbn_fp8_gemm_nt_ws without any allocation by the caller: the split-K slabs
 * go to a device array the library holds per GPU (`scratch`, of
 * kbn_fp8_gemm_nt_noalloc_scratch_bytes() = 64 MiB, kept until the process
 * ends), so results are those of kbn_fp8_gemm_nt_ws with a large enough
 * workspace, bit for bit.  A shape whose split plan needs more than the
 * scratch is rejected (code 1); on a 256-CU MI355X no plan does.  Every call
 * on one GPU uses the same scratch, so calls that may overlap on one GPU
 * (other streams, forked branches of a graph) race: serialise them.
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).
 */
int64_t kbn_fp8_gemm_nt_noalloc_scratch_bytes(void);
int kbn_fp8_gemm_nt_noalloc(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m, int64_t sA_stride_k,
                            const void* W, int64_t ldw, const float* sW, int64_t sW_ld,
                            void* D_bf16, int64_t ldd, int64_t M, int64_t N, int64_t K,
                            int scale_ue8m0, void* stream);

/*
 * Contiguous-layout grouped FP8 GEMM (MoE experts).
 * Replaces op kb_nano_fp8_moe::m_grouped_gemm_nt_contiguous ->
 * deep_gemm.m_grouped_fp8_gemm_nt_contiguous
 * (tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:100-133; free function
 * tasks/baseline/L1/moe_grouped_gemm.py:71-83).
 *   A   fp8 [M_sum, K] row stride lda; sA fp32 [M_sum, K/128] (strides as above)
 *   B   fp8 [E, N, K] contiguous;      sB fp32 [E, ceil(N/128), K/128] contiguous
 *   C   bf16 [M_sum, N] row stride ldc; expert_ids int32 [M_sum]
 *   Rows are taken in 128-row blocks (M_sum % 128 == 0).  A block whose first
 *   row has id e in [0, E) computes C[r] = A[r] x B[e]^T (block-scaled as in
 *   kbn_fp8_gemm_nt) for its rows with id e; rows with any other id (-1 =
 *   padding) and blocks whose first id is outside [0, E) are not written.
 *   scale_ue8m0 = !disable_ue8m0_cast.
 */
int kbn_fp8_grouped_gemm_nt_contiguous(const void* A, int64_t lda, const float* sA,
                                       int64_t sA_stride_m, int64_t sA_stride_k,
                                       const void* B, const float* sB, void* C_bf16, int64_t ldc,
                                       const int32_t* expert_ids, int64_t M_sum, int64_t N, int64_t K,
                                       int64_t E, int scale_ue8m0, void* stream);

/*
 * The contiguous grouped GEMM of the experts' gate/up projection with the
 * SiLU*Mul + 1x128 FP8 quant of its output in the same launch: what
 * kbn_fp8_grouped_gemm_nt_contiguous into C [M_sum, N2] followed by
 * kbn_silu_mul_quant_fp8_rows(C, row ids = expert_ids) writes, without C.
 * Replaces, inside FusedExperts._forward_deep_gemm, the GEMM1 call and the
 * SiLU*Mul+quant call that reads its output (tasks/baseline/L2/
 * fused_experts.py:264-274; tasks/baseline/L1/silu_mul_quant_fp8.py:23-76).
 *   A, sA, B, sB, expert_ids, M_sum, K, E, scale_ue8m0   as the grouped GEMM, B [E, N2, K]
 *   N2 % 256 == 0: B's rows [0, N2/2) are the gate, [N2/2, N2) the up rows
 *   q        fp8 [M_sum, N2/2], row stride ldq (multiple of 8)
 *   q_scale  fp32 (r, g) at q_scale[r*qs_stride_m + g*qs_stride_g]
 *   For every row r with an expert id in [0, E): h = bf16 GEMM row, y =
 *   bf16(bf16(silu(h[:N2/2])) * h[N2/2:]), then the 1x128 quant of y with
 *   absmax floor eps, UE8M0 scales when q_ue8m0.  Other rows are not written.
 */
int kbn_fp8_grouped_gemm_silu_quant(const void* A, int64_t lda, const float* sA, int64_t sA_stride_m,
                                    int64_t sA_stride_k, const void* B, const float* sB, const int32_t* expert_ids,
                                    int64_t M_sum, int64_t N2, int64_t K, int64_t E, int scale_ue8m0,
                                    void* q_fp8, int64_t ldq, float* q_scale, int64_t qs_stride_m,
                                    int64_t qs_stride_g, float eps, int q_ue8m0, void* stream);

/*
 * Workspace bytes of kbn_moe_permute_contiguous for num_pairs = M * top_k
 * routed pairs and num_experts experts; -1 if num_experts is outside
 * [1, 1024] or num_pairs outside [0, 2^31).  (The reference's torch ops
 * allocate their temporaries themselves; this ABI takes them from the caller.)
 */
int64_t kbn_moe_permute_workspace_bytes(int64_t num_pairs, int64_t num_experts);

/*
 * Contiguous-layout MoE permute.
 * Replaces _deepgemm_permute (tasks/baseline/L2/fused_experts.py:42-116).
 *   topk_ids    int32 (ids_bytes 4) or int64 (8) [M, top_k], contiguous
 *   x           [M, row_bytes] rows (any element type, e.g. fp8 [M, K]),
 *               row stride ld_x_bytes; 16-byte aligned, row_bytes % 16 == 0
 *   x_scale     fp32 [M, scale_cols] at x_scale[m*s_stride_m + c*s_stride_c]
 *   M_sum       must equal roundup(M*top_k + E*(alignment-1), alignment)
 *               (_compute_aligned_M, fused_experts.py:32-39)
 *   x_perm      [M_sum, row_bytes] contiguous; scale_perm fp32 [M_sum, scale_cols]
 *               at scale_perm[r*sp_stride_m + c*sp_stride_c], row-major (the
 *               reference's) or column-major (coalesced per-K-block loads in
 *               the grouped GEMM)
 *   expert_ids  int32 [M_sum];  inv_perm int32 [M, top_k]
 *   Expert e owns rows [off[e], off[e] + roundup(count[e], alignment)), with
 *   off the exclusive prefix sum of the rounded counts.  Its first count[e]
 *   rows hold its (token, slot) pairs in (token, slot) order and carry id e;
 *   the rest are padding with id -1, as are rows past the last segment.
 *   inv_perm[m, j] is the row of pair (m, j).  A pair whose id is outside
 *   [0, E) is dropped (inv_perm -1); the reference fails on it in scatter_add.
 *   zero_padding = 1 zeroes the padding rows of x_perm and scale_perm (the
 *   reference's torch.zeros); 0 leaves them unwritten, which is enough for
 *   kbn_fp8_grouped_gemm_nt_contiguous (it never writes padding rows of C).
 *   workspace   >= kbn_moe_permute_workspace_bytes(M*top_k, E), 16-byte aligned
 */
int kbn_moe_permute_contiguous(const void* topk_ids, int ids_bytes, int64_t M, int64_t top_k,
                               int64_t num_experts, int64_t alignment,
                               const void* x, int64_t ld_x_bytes, int64_t row_bytes,
                               const float* x_scale, int64_t s_stride_m, int64_t s_stride_c,
                               int64_t scale_cols, int64_t M_sum, void* x_perm, float* scale_perm,
                               int64_t sp_stride_m, int64_t sp_stride_c,
                               int32_t* expert_ids, int32_t* inv_perm, int zero_padding,
                               void* workspace, int64_t workspace_bytes, void* stream);

/*
 * kbn_moe_permute_contiguous with the 1x128 FP8 quant of the rows folded in
 * (no counterpart in one reference call: it replaces FusedExperts'
 * per_token_group_quant_fp8 of the hidden states followed by
 * _deepgemm_permute, tasks/baseline/L2/fused_experts.py:257-262).
 *   x_bf16   bf16 [M, K] (row stride ld_x elements, 16-byte aligned rows),
 *            K % 128 == 0; top_k <= 64
 *   x_perm / scale_perm / expert_ids / inv_perm / workspace as in
 *            kbn_moe_permute_contiguous (row_bytes = K, scale_cols = K/128)
 *   Each token's row is quantized once, as kbn_per_token_group_quant_fp8
 *   does (absmax floor eps, UE8M0 scales when use_ue8m0), and its codes and
 *   scales go to every routed pair's row: the bytes that quant followed by
 *   kbn_moe_permute_contiguous writes.
 */
int kbn_moe_permute_quant_contiguous(const void* topk_ids, int ids_bytes, int64_t M, int64_t top_k,
                                     int64_t num_experts, int64_t alignment, const void* x_bf16, int64_t ld_x,
                                     int64_t K, float eps, int use_ue8m0, int64_t M_sum, void* x_perm,
                                     float* scale_perm, int64_t sp_stride_m, int64_t sp_stride_c,
                                     int32_t* expert_ids, int32_t* inv_perm, int zero_padding, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/*
 * Unpermute and top-k weighted reduction.
 * Replaces _deepgemm_unpermute_and_reduce (tasks/baseline/L2/fused_experts.py:119-136).
 *   y         bf16 [M_sum, H] (the second grouped GEMM's output), row stride ld_y
 *   inv_perm  int32 [M, top_k];  topk_weights [M, top_k] fp32 (weights_bf16 0)
 *             or bf16 (1), contiguous
 *   out       bf16 [M, H], row stride ld_out;  H % 8 == 0, 16-byte aligned rows
 *   out[m, h] = bf16_rne(sum over j = 0..top_k-1, in slot order, in fp32, of
 *   y[inv_perm[m, j], h] * w[m, j]); each product rounds to fp32 (fp32
 *   weights) or to bf16 (bf16 weights), as torch's product does.  Slots whose
 *   inv_perm is outside [0, M_sum) contribute nothing.
 */
int kbn_moe_unpermute_reduce(const void* y_bf16, int64_t M_sum, int64_t H, int64_t ld_y,
                             const int32_t* inv_perm, int64_t M, int64_t top_k,
                             const void* topk_weights, int weights_bf16,
                             void* out_bf16, int64_t ld_out, void* stream);

/*
 * Fused RMSNorm (+ residual add) + per-token-group (1x128) FP8 quantization.
 * Replaces ops kb_nano_norm::rmsnorm_fp8_quant and
 * kb_nano_norm::fused_add_rmsnorm_fp8_quant (tasks/baseline/L1/rmsnorm_quant.py:27-55;
 * kernels tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-93, :124-201).
 *   x         bf16 [M, H], row stride ld_x; w bf16 [H]; 16-byte aligned, H % 8 == 0
 *   residual  NULL: plain RMSNorm of x.  Otherwise bf16 [M, H], row stride
 *             ld_r: residual <- bf16(residual + x), the norm is taken of the
 *             fp32 sums, and x <- bf16(normalized row).  Any H (multiple of 8):
 *             rows of up to 16384 (8192 with the add) are held in registers,
 *             longer ones read twice, in the same summation order.
 *   q         fp8 [M, H], row stride ld_q (multiple of 8)
 *   scale     fp32 (m, g) at scale[m*s_stride_m + g*s_stride_g], g < ceil(H/128)
 *             (the reference's column-major buffer: (1, M))
 *   inv = 1/sqrt(mean(a^2) + eps) over the row; v = (a_bf16 * inv) * w in fp32;
 *   each 1x128 group (the last one partial when H % 128 != 0) gets the UE8M0
 *   scale ceil_pow2(max(max|v|, 1e-10) / 448) and codes e4m3_rne(v / scale).
 *   The sum of squares is fp32 in a fixed order, inv uses the correctly
 *   rounded sqrt and divide (the reference: its thread layout's order, rsqrtf).
 */
int kbn_rmsnorm_fp8_quant(void* x_bf16, int64_t M, int64_t H, int64_t ld_x, const void* w_bf16,
                          void* residual_bf16, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale,
                          int64_t s_stride_m, int64_t s_stride_g, float eps, void* stream);

/*
 * The same for bf16, fp16 or fp32 rows: the reference dispatches its kernels
 * over the float types (tasks/baseline/L1/csrc/rmsnorm_quant.cu:111).
 *   x_dtype   0 bf16, 1 fp16, 2 fp32; x, w and residual all of that type
 *   The residual sum and the normalized row written back are rounded to the
 *   type (nearest even); every other argument as kbn_rmsnorm_fp8_quant.
 */
int kbn_rmsnorm_fp8_quant_typed(void* x, int x_dtype, int64_t M, int64_t H, int64_t ld_x, const void* w,
                                void* residual, int64_t ld_r, void* q_fp8, int64_t ld_q, float* scale,
                                int64_t s_stride_m, int64_t s_stride_g, float eps, void* stream);

/*
 * Sorted-token MoE layout: moe_align_block_size.
 * Replaces _C.moe_align_block_size (tasks/baseline/L1/csrc/moe_align.cu:28-383,
 * bound by tasks/baseline/L1/moe_align.py:92 and
 * tasks/baseline/L2/vllm_fused_experts.py:66-97).
 *   topk_ids  [numel] int32 (ids_bytes 4) or int64 (8), flattened (token, slot)
 *   Expert e's pairs fill slots [cumsum[e], cumsum[e] + count_e) in (token,
 *   slot) order (the reference's atomic placement allows any order inside an
 *   expert); segments are padded to block_size and every other slot of
 *   sorted_token_ids holds numel.  expert_ids[b] is the owner of block b for
 *   b < *num_tokens_post_pad / block_size (later entries are not written).
 *   Pairs with ids outside [0, E) are not placed.  cumsum [E + 1] may be NULL.
 *   sorted_len >= numel + min(numel, E) * (block_size - 1) and
 *   expert_len * block_size >= that bound (the reference's buffer sizes).
 *   workspace >= kbn_moe_permute_workspace_bytes(numel, E), 16-byte aligned.
 */
int kbn_moe_align_block_size(const void* topk_ids, int ids_bytes, int64_t numel, int64_t num_experts,
                             int64_t block_size, int32_t* sorted_token_ids, int64_t sorted_len,
                             int32_t* expert_ids, int64_t expert_len, int32_t* num_tokens_post_pad,
                             int32_t* cumsum, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Sorted-token fused-MoE FP8 GEMM with 128x128 block scales.
 * Replaces MoeGroupedGemm / _fused_moe_kernel (tasks/baseline/L1/moe_grouped_gemm.py:86-189,
 * :298-382) on its use_fp8_w8a8 + block_shape [128, 128] path.
 *   Row R < EM of the padded grid holds pair t = sorted_token_ids[R] (t >= num_valid:
 *   padding), or with sorted_token_ids NULL (the reference's naive block
 *   assignment) pair R / block_m on the first row of each block.  Block b =
 *   R / block_m uses expert expert_ids[b]; blocks at or past
 *   *num_tokens_post_padded are skipped.
 *   A  fp8 [rows_A, K] (row stride lda) with fp32 scales sA (strides in
 *      elements); pair t reads row t / top_k.
 *   B  fp8 [E, N, K], sB fp32 [E, ceil(N/128), K/128], both contiguous.
 *   C  bf16 [num_valid, ldc]: row t = sum_kb sA[t/top_k, kb] sB[e, n/128, kb]
 *      (A.B^T of block kb), times topk_weights[t] (fp32) when that is not NULL.
 *   Scales are taken as given.  K % 128 == 0, block_m a multiple of 64.
 *   workspace: NULL, or kbn_fp8_fused_moe_gemm_workspace_bytes(EM, K) bytes,
 *   16-byte aligned (see below).
 */
int kbn_fp8_fused_moe_gemm(const void* A, int64_t lda, int64_t rows_A, const float* sA, int64_t sA_stride_m,
                           int64_t sA_stride_k, const void* B, const float* sB, void* C_bf16, int64_t ldc,
                           const int32_t* sorted_token_ids, const int32_t* expert_ids,
                           const int32_t* num_tokens_post_padded, int64_t EM, int64_t block_m,
                           int64_t num_valid, int64_t top_k, const float* topk_weights, int64_t N, int64_t K,
                           int64_t E, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Workspace of kbn_fp8_fused_moe_gemm (EM * K/128 fp32, -1 for bad sizes).
 * With it, a first launch gathers the activation scales into sorted-row
 * order so the GEMM reads them coalesced (about 8% faster at DeepSeek-V3
 * sizes); with workspace NULL each row's scales are read where they lie.
 */
int64_t kbn_fp8_fused_moe_gemm_workspace_bytes(int64_t EM, int64_t K);

/*
 * Top-k sum of the experts' output rows.
 * Replaces _C.moe_sum (tasks/baseline/L1/csrc/moe_sum.cu:8-63, bound by
 * tasks/baseline/L1/moe_sum.py:43).
 *   x    bf16, row (m, j) at x + (m * top_k + j) * ld_x, H columns
 *   out  bf16 [M, H], row stride ld_out
 *   top_k <= 4: x accumulates in bf16 from 0, rounding after every add (the
 *   reference kernel's scalar_t accumulator).  top_k > 4 (and 1): the
 *   reference's at::sum_out: four fp32 accumulators taking slots j % 4,
 *   combined ((a0 + a1) + a2) + a3, one rounding to bf16.
 */
int kbn_moe_sum(const void* x_bf16, int64_t M, int64_t top_k, int64_t H, int64_t ld_x, void* out_bf16,
                int64_t ld_out, void* stream);

/*
 * 128x128 block (re)quantization of weights, one launch over [E, N, K].
 * Replaces postprocess_fp8_weights[_batched] (tasks/baseline/L1/fp8_linear.py:453-554)
 * and the DeepGEMM per_block_cast_to_fp8 it calls (:497-499, :543-545).
 *   w_in    [E, N, K] contiguous: fp8 codes (in_f32 = 0), dequantized with the
 *           block scale s_in[e*s_in_e + nb*s_in_ld + kb], or fp32 values (1)
 *   w_out   fp8 [E, N, K] contiguous, s_out[e*s_out_e + nb*s_out_ld + kb].
 *           In-place requant of fp8 codes: w_out == w_in and s_out == s_in
 *           with equal strides.  Any other overlap (and every overlap of
 *           fp32 input) is rejected.  K % 16 == 0, 16-byte aligned weights.
 *   Per block: sf = max(max|x|, eps) / 448, rounded up to a power of two when
 *   use_ue8m0; codes = e4m3_rne(x * (1/sf)); ragged blocks pad with zeros.
 */
int kbn_fp8_block_requant(const void* w_in, int in_f32, const float* s_in, int64_t s_in_e, int64_t s_in_ld,
                          int64_t E, int64_t N, int64_t K, void* w_out, float* s_out,
                          int64_t s_out_e, int64_t s_out_ld, int use_ue8m0, float eps, void* stream);

/*
 * Split-K arrival counters (no counterpart in the reference; DeepGEMM has no
 * split-K).  The small-M split launches of the 64-row tiles sum their fp32
 * slabs themselves, counting arrivals in a region of a library-held device
 * array: one region per eager stream and per (capture, stream) pair, kept
 * for the life of the process (a captured graph replays with its region).
 * When a device's regions are all taken, later launches on new streams or
 * captures run the separate reduction kernel instead: same results, one
 * launch more; the first such launch also prints one line on stderr.
 *   regions_used   regions in use on the busiest device
 *   regions_total  regions per device (1024)
 *   fallbacks      split launches that found no free region
 * Any pointer may be NULL.  Host bookkeeping only: callable without a GPU.
 */
int kbn_splitk_counter_stats(int64_t* regions_used, int64_t* regions_total, int64_t* fallbacks);

/*
 * Test hook (no counterpart in the reference): the region bookkeeping above
 * on a private table, without a GPU.  n_keys distinct eager streams of one
 * device ask for a region, then the first asks again: out_region[i] gets
 * stream i's region (-1: none left), out_region[n_keys] the repeated
 * stream's; *out_fallbacks the table's fallback count.  1 <= n_keys <= 4096.
 */
int kbn_debug_splitk_regions(int64_t n_keys, int32_t* out_region, int64_t* out_fallbacks);

/*
 * Test hook (no counterpart in the reference): the tile plan the GEMM entry
 * points would launch for an M x N x K call with a workspace, without a GPU
 * (a device with 256 CUs is assumed when none is present).  bf16a != 0 asks
 * for kbn_fp8_gemm_bf16a's plan (M <= 64), else kbn_fp8_gemm_nt_ws's with
 * scale_ue8m0.  out[0..8] = tile rows, tile columns, LDS stages, tiles,
 * data-parallel tiles, K splits of the rest, K blocks per split, whether the
 * split launch sums its own slabs (1) or a reduction launch follows (0), and
 * workspace bytes.
 */
int kbn_debug_gemm_plan(int64_t M, int64_t N, int64_t K, int scale_ue8m0, int bf16a, int64_t* out);

/*
 * Test hook (no counterpart in the reference): the kernels' bf16 SiLU
 * applied elementwise to n bf16 bit patterns, for exhaustive checking.
 * path 0 reads the table as the SiLU*Mul + quant kernels do; path 1 reads it
 * at the device address hipGetSymbolAddress gives, as the grouped GEMM's
 * SiLU*Mul epilogue (kbn_fp8_grouped_gemm_silu_quant) does.
 */
int kbn_debug_silu_bf16(const uint16_t* g_bf16, uint16_t* out_bf16, int64_t n, int path, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KBN_FP8_H */
