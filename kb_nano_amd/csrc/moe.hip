// Contiguous-layout MoE glue around the grouped FP8 GEMM: the permute that
// scatters routed (token, slot) rows into expert-contiguous, alignment-padded
// segments, and the weighted unpermute-and-reduce of the second GEMM's rows.
// Same layout contract as tasks/baseline/L2/fused_experts.py:32-136
// (kb_nano), which builds it from ~40 torch ops (scatter_add, argsort,
// searchsorted, index_put, gather, broadcast multiply, sum).
//
// Permute, three launches on one stream:
//   count  one wavefront per chunk of pairs: each pair's rank among the
//          chunk's earlier pairs routed to the same expert (wave-level
//          multi-split over the bits of the expert id, no atomics), and the
//          chunk's per-expert histogram;
//   scan   one workgroup: per expert, exclusive prefix of the histograms over
//          chunks (the expert's count before each chunk) and the total; then
//          the exclusive scan of the aligned totals = segment offsets;
//   place  one wavefront per pair: destination row = offset[e] + prefix of
//          its chunk + rank, copy of the token's row and scale row; and one
//          wavefront per 4 destination rows: expert id (or -1) and, when
//          asked, zeros for padding rows.
// Ranks follow (token, slot) order inside each expert, as the reference's
// stable argsort does, so the layout is index-identical to the reference.
//
// The same count and scan also build the sorted-token layout of
// moe_align_block_size (tasks/baseline/L1/csrc/moe_align.cu:28-383, the
// sgl-kernel source vLLM uses): a third launch writes each pair's index into
// its slot, fills the rest of the buffer with the sentinel numel, and
// writes the owner expert of every block.  The reference places pairs with
// atomics, so its order inside an expert varies from run to run; here it is
// the (token, slot) order, one of the orders the reference can produce.
//
// moe_sum (tasks/baseline/L1/csrc/moe_sum.cu:8-63) sums the top-k output rows
// of each token: for top_k <= 4 in bf16, rounding after every add as the
// reference kernel's bf16 accumulator does; otherwise through the reference's
// at::sum_out, whose fp32 order on this GPU is four round-robin accumulators
// combined left to right (measured against torch.sum), then one rounding.
#include "kbn_common.h"

#include <algorithm>

namespace kbn {
namespace {

constexpr int kMaxExperts = 1024;
// 64-pair steps per batch of a counting wavefront: 512-pair chunks (64 chunks
// for 32,768 pairs) took the whole permute to 81.3 us against 86.1 us with
// 1024-pair chunks and 82.2 us with 256-pair ones
constexpr int kCountIters = 8;
constexpr int kChunkUnit = 64 * kCountIters;    // chunk sizes are multiples of this
constexpr int kMaxChunks = 256;                 // bound on the scan's walk
// wavefronts per place workgroup: the 32,768-pair, 7168-byte-row permute took
// 93 / 81.5 / 76.5 / 78 us with 2 / 4 / 8 / 16
constexpr int kPlaceWaves = 8;
constexpr int kPadRowsPerWave = 4;

struct PermuteArgs {
    const void* ids;        // [n] int32 or int64 expert ids, (token, slot) order
    int ids64;
    int n;                  // routed pairs, M * top_k
    int top_k;
    int E;
    int bits;               // bits needed for an id in [0, E)
    int align;
    int chunk;              // pairs per counting chunk (multiple of kChunkUnit)
    int nchunks;
    int* hist;              // [nchunks][E] counts, then exclusive prefix over chunks
    int* rank;              // [n]
    int* counts;            // [E]
    int* offsets;           // [E + 1]
    const uint8_t* x;       // [M, row_bytes] rows, stride ld_x bytes
    int64_t ld_x;
    int row_bytes;          // multiple of 16
    const float* xs;        // scale (m, c) at xs[m * xs_m + c * xs_c]
    int64_t xs_m, xs_c;
    int scale_cols;
    uint8_t* xp;            // [M_sum, row_bytes]
    float* sp;              // scale (r, c) at sp[r * sp_m + c * sp_c]
    int64_t sp_m, sp_c;
    int32_t* expert_ids;    // [M_sum]
    int32_t* inv_perm;      // [n]
    int M_sum;
    int zero_padding;
    int place_blocks;       // blocks [0, place_blocks) copy pairs, the rest fill rows
    float eps;              // quantizing permute: the 1x128 quant's absmax floor
    // moe_align_block_size
    int32_t* sorted_ids;    // [sorted_len]: pair index per slot, numel elsewhere
    int sorted_len;
    int32_t* post_pad;      // [1]: total padded slots
    int32_t* cumsum_out;    // [E + 1] segment offsets, or nullptr
};

// Expert id of pair i, or -1 when it lies outside [0, E).
__device__ __forceinline__ int load_id(const PermuteArgs& a, int i) {
    const int64_t v = a.ids64 ? reinterpret_cast<const int64_t*>(a.ids)[i] : reinterpret_cast<const int32_t*>(a.ids)[i];
    return (v >= 0 && v < a.E) ? (int)v : -1;
}

__global__ __launch_bounds__(64) void moe_count_kernel(const PermuteArgs a) {
    __shared__ int cnt[kMaxExperts];
    const int lane = threadIdx.x;
    for (int e = lane; e < a.E; e += 64) cnt[e] = 0;
    __syncthreads();
    const int c = blockIdx.x;
    const int begin = c * a.chunk;
    const int end = min(begin + a.chunk, a.n);
    const uint64_t below = (1ull << lane) - 1ull;
    for (int blk = begin; blk < end; blk += kChunkUnit) {
        int ev[kCountIters];
#pragma unroll
        for (int t = 0; t < kCountIters; ++t) {
            const int i = blk + t * 64 + lane;
            ev[t] = i < end ? load_id(a, i) : -1;
        }
#pragma unroll
        for (int t = 0; t < kCountIters; ++t) {
            const int e = ev[t];
            const bool ok = e >= 0;
            // lanes holding the same id: intersect, bit by bit, the ballots
            // of lanes that agree with this lane's bit
            uint64_t peers = __ballot(ok);
            for (int b = 0; b < a.bits; ++b) {
                const bool bit = (e >> b) & 1;
                const uint64_t m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            const int seen = ok ? cnt[e] : 0;
            if (ok) {
                const int i = blk + t * 64 + lane;
                a.rank[i] = seen + __popcll(peers & below);
                if ((peers & below) == 0) cnt[e] = seen + __popcll(peers);   // lowest peer lane
            }
            __syncthreads();
        }
    }
    for (int e = lane; e < a.E; e += 64) a.hist[(int64_t)c * a.E + e] = cnt[e];
}

__global__ __launch_bounds__(1024) void moe_scan_kernel(const PermuteArgs a) {
    __shared__ int wsum[16];
    const int e = threadIdx.x;
    const int lane = e & 63, wave = e >> 6;
    int total = 0;
    if (e < a.E) {
        int* h = a.hist + e;
        int c = 0;
        for (; c + 8 <= a.nchunks; c += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = h[(int64_t)(c + u) * a.E];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                h[(int64_t)(c + u) * a.E] = total;
                total += v[u];
            }
        }
        for (; c < a.nchunks; ++c) {
            const int v = h[(int64_t)c * a.E];
            h[(int64_t)c * a.E] = total;
            total += v;
        }
        a.counts[e] = total;
    }
    const int seg = e < a.E ? (total + a.align - 1) / a.align * a.align : 0;
    int v = seg;   // inclusive scan within the wavefront
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    if (wave == 0) {
        int w = lane < 16 ? wsum[lane] : 0;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const int t = __shfl_up(w, d, 64);
            if (lane >= d) w += t;
        }
        if (lane < 16) wsum[lane] = w;
    }
    __syncthreads();
    const int excl = v - seg + (wave > 0 ? wsum[wave - 1] : 0);
    if (e < a.E) a.offsets[e] = excl;
    if (e == a.E - 1) a.offsets[a.E] = excl + seg;
}

// Copy (or zero, src == nullptr) `bytes` (multiple of 16) with one wavefront.
__device__ __forceinline__ void wave_row(const uint8_t* src, uint8_t* dst, int bytes, int lane) {
    const int nv = bytes >> 4;
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    u32x4* d = reinterpret_cast<u32x4*>(dst);
    for (int v0 = lane; v0 < nv; v0 += 64 * 4) {
        u32x4 t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int w = v0 + u * 64;
            t[u] = u32x4{0u, 0u, 0u, 0u};
            if (src && w < nv) t[u] = s[w];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int w = v0 + u * 64;
            if (w < nv) __builtin_nontemporal_store(t[u], d + w);
        }
    }
}

// Quantizing permute (kQuant 1: UE8M0 scales, 2: fp32 scales): a.x holds
// bf16 rows [M, K] (stride ld_x bytes), and kQuantWaves wavefronts per token
// (taking turns over steps of kQuantPasses x 4 groups) quantize its row 1x128 once
// (quant8_codes: the codes and scales of per-token-group quant) and write the
// codes and the scale of each group to the destination rows of all the
// token's routed pairs.  At cfg4 (4096 tokens x 7168, top-8) one wavefront
// per token took 73 us against 78 / 82 us with two / four.
constexpr int kQuantWaves = 1;
constexpr int kQuantPasses = 2;
template <int kQuant>
__device__ __forceinline__ void place_quant_token(const PermuteArgs& a, int t, int part, int lane) {
    int dest = -1;
    if (lane < a.top_k) {   // top_k <= 64, checked on the host
        const int i = t * a.top_k + lane;
        const int e = load_id(a, i);
        if (e >= 0) dest = a.offsets[e] + a.hist[(int64_t)(i / a.chunk) * a.E + e] + a.rank[i];
        if (part == 0) a.inv_perm[i] = dest;
    }
    const uint8_t* xrow = a.x + (int64_t)t * a.ld_x;
    const int G = a.scale_cols, sub = lane & 15, gq = lane >> 4;
    for (int g0 = 4 * kQuantPasses * part; g0 < G; g0 += 4 * kQuantPasses * kQuantWaves) {
        // kQuantPasses x 4 groups per step, 16 lanes per group
        u32x4 v[kQuantPasses];
#pragma unroll
        for (int u = 0; u < kQuantPasses; ++u) {
            const int g = g0 + 4 * u + gq;
            v[u] = g < G ? *reinterpret_cast<const u32x4*>(xrow + (int64_t)g * 256 + sub * 16) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kQuantPasses; ++u) {
            const int g = g0 + 4 * u + gq;
            const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            float sc;
            const u32x2 o = quant8_codes<kQuant == 1>(w, a.eps, sc);   // every lane of the 16-lane group
            if (g < G) {
                for (int j = 0; j < a.top_k; ++j) {
                    const int d = __builtin_amdgcn_readlane(dest, j);
                    if (d < 0) continue;
                    __builtin_nontemporal_store(
                        o, reinterpret_cast<u32x2*>(a.xp + (int64_t)d * a.row_bytes + (int64_t)g * 128 + sub * 8));
                    if (sub == 0) a.sp[(int64_t)d * a.sp_m + (int64_t)g * a.sp_c] = sc;
                }
            }
        }
    }
}

template <int kQuant>
__global__ __launch_bounds__(64 * kPlaceWaves) void moe_place_kernel(const PermuteArgs a) {
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_cnt[kMaxExperts];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    if (kQuant && (int)blockIdx.x < a.place_blocks) {
        // kQuantWaves wavefronts per token
        const int tw = (int)blockIdx.x * kPlaceWaves + wave;
        const int t = tw / kQuantWaves;
        if (t < a.n / a.top_k) place_quant_token<kQuant>(a, t, tw % kQuantWaves, lane);
        return;
    }
    if (!kQuant && (int)blockIdx.x < a.place_blocks) {
        // one routed pair per wavefront
        const int i = (int)blockIdx.x * kPlaceWaves + wave;
        if (i >= a.n) return;
        const int e = load_id(a, i);
        if (e < 0) {
            if (lane == 0) a.inv_perm[i] = -1;
            return;
        }
        const int dest = a.offsets[e] + a.hist[(int64_t)(i / a.chunk) * a.E + e] + a.rank[i];
        if (lane == 0) a.inv_perm[i] = dest;
        const int t = i / a.top_k;
        wave_row(a.x + (int64_t)t * a.ld_x, a.xp + (int64_t)dest * a.row_bytes, a.row_bytes, lane);
        for (int g = lane; g < a.scale_cols; g += 64)
            a.sp[(int64_t)dest * a.sp_m + (int64_t)g * a.sp_c] = a.xs[(int64_t)t * a.xs_m + (int64_t)g * a.xs_c];
        return;
    }

    // destination rows: owner expert and padding
    for (int j = threadIdx.x; j <= a.E; j += 64 * kPlaceWaves) {
        s_off[j] = a.offsets[j];
        if (j < a.E) s_cnt[j] = a.counts[j];
    }
    __syncthreads();
    const int r0 = (((int)blockIdx.x - a.place_blocks) * kPlaceWaves + wave) * kPadRowsPerWave;
    for (int rr = 0; rr < kPadRowsPerWave; ++rr) {
        const int r = r0 + rr;
        if (r >= a.M_sum) break;
        // last e in [0, E] with offsets[e] <= r (searchsorted right, minus one)
        int lo = 0, hi = a.E;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_off[mid] <= r) lo = mid;
            else hi = mid - 1;
        }
        const bool valid = lo < a.E && r - s_off[lo] < s_cnt[lo];
        if (lane == 0) a.expert_ids[r] = valid ? lo : -1;
        if (!valid && a.zero_padding) {
            wave_row(nullptr, a.xp + (int64_t)r * a.row_bytes, a.row_bytes, lane);
            for (int g = lane; g < a.scale_cols; g += 64) a.sp[(int64_t)r * a.sp_m + (int64_t)g * a.sp_c] = 0.f;
        }
    }
}

// moe_align_block_size placement.  Blocks [0, place_blocks): one thread per
// pair writes its index into its slot.  The remaining blocks: one thread per
// slot of the buffer writes the sentinel into slots no pair owns and, at the
// first slot of each block below the total, the block's expert.
constexpr int kAlignThreads = 256;

__global__ __launch_bounds__(kAlignThreads) void moe_align_place_kernel(const PermuteArgs a) {
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_cnt[kMaxExperts];
    if ((int)blockIdx.x < a.place_blocks) {
        const int i = (int)blockIdx.x * kAlignThreads + (int)threadIdx.x;
        if (i >= a.n) return;
        const int e = load_id(a, i);
        if (e < 0) return;
        a.sorted_ids[a.offsets[e] + a.hist[(int64_t)(i / a.chunk) * a.E + e] + a.rank[i]] = i;
        return;
    }
    for (int j = threadIdx.x; j <= a.E; j += kAlignThreads) {
        s_off[j] = a.offsets[j];
        if (j < a.E) s_cnt[j] = a.counts[j];
    }
    __syncthreads();
    const int total = s_off[a.E];
    const int r = ((int)blockIdx.x - a.place_blocks) * kAlignThreads + (int)threadIdx.x;
    if (r == 0) {
        a.post_pad[0] = total;
        if (a.cumsum_out)
            for (int j = 0; j <= a.E; ++j) a.cumsum_out[j] = s_off[j];
    }
    if (r >= a.sorted_len) return;
    int lo = 0, hi = a.E;   // last e in [0, E] with offsets[e] <= r
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= r) lo = mid;
        else hi = mid - 1;
    }
    const bool valid = lo < a.E && r - s_off[lo] < s_cnt[lo];
    if (!valid) a.sorted_ids[r] = a.n;
    if (r < total && r % a.align == 0) a.expert_ids[r / a.align] = lo;
}

// ----------------------------------------------------------------- moe_sum ---

constexpr int kSumThreads = 128;   // 8 bf16 columns per thread

struct MoeSumArgs {
    const uint16_t* x;       // row (m, j) at x + (m * top_k + j) * ld_x
    int64_t ld_x;
    int top_k;
    int H;
    uint16_t* out;           // [M, H], row stride ld_out
    int64_t ld_out;
    int col_blocks;
    int vec;                 // rows allow 16-B accesses
};

__device__ __forceinline__ float bf16_round(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(((u >> 16) | 0x40u) << 16);
    return __uint_as_float(((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16) << 16);
}

// out[m, c] for the 8 columns c0 .. c0+7 of token m, v(j, q) the bf16 value
// of slot j, column c0 + q.
template <typename Load>
__device__ __forceinline__ void topk_sum8(int top_k, Load v, float (&r)[8]) {
#pragma clang fp contract(off)
    if (top_k <= 4) {
#pragma unroll
        for (int q = 0; q < 8; ++q) r[q] = 0.f;
        for (int j = 0; j < top_k; ++j) {
            float x[8];
            v(j, x);
#pragma unroll
            for (int q = 0; q < 8; ++q) r[q] = bf16_round(r[q] + x[q]);
        }
        return;
    }
    float acc[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j) v(j, acc[j]);
    for (int j = 4; j < top_k; ++j) {
        float x[8];
        v(j, x);
        float (&t)[8] = acc[j & 3];
#pragma unroll
        for (int q = 0; q < 8; ++q) t[q] = t[q] + x[q];
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = bf16_round(((acc[0][q] + acc[1][q]) + acc[2][q]) + acc[3][q]);
}

__global__ __launch_bounds__(kSumThreads) void moe_sum_kernel(const MoeSumArgs a) {
    const int m = (int)blockIdx.x / a.col_blocks;
    const int cb = (int)blockIdx.x - m * a.col_blocks;
    const int c0 = (cb * kSumThreads + (int)threadIdx.x) * 8;
    if (c0 >= a.H) return;
    const uint16_t* row0 = a.x + (int64_t)m * a.top_k * a.ld_x + c0;
    uint16_t* o = a.out + (int64_t)m * a.ld_out + c0;
    const int nc = min(8, a.H - c0);
    float r[8];
    if (a.vec && nc == 8) {
        topk_sum8(a.top_k, [&](int j, float (&x)[8]) {
            const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row0 + (int64_t)j * a.ld_x));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                x[2 * q] = bf16lo(w[q]);
                x[2 * q + 1] = bf16hi(w[q]);
            }
        }, r);
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            w[q] = (__float_as_uint(r[2 * q]) >> 16) | (__float_as_uint(r[2 * q + 1]) & 0xFFFF0000u);
        *reinterpret_cast<u32x4*>(o) = w;
        return;
    }
    topk_sum8(a.top_k, [&](int j, float (&x)[8]) {
#pragma unroll
        for (int q = 0; q < 8; ++q)
            x[q] = q < nc ? __uint_as_float((uint32_t)row0[(int64_t)j * a.ld_x + q] << 16) : 0.f;
    }, r);
    for (int q = 0; q < nc; ++q) o[q] = (uint16_t)(__float_as_uint(r[q]) >> 16);
}

// ------------------------------------------------------------ unpermute ---

constexpr int kUnpermThreads = 128;   // 8 bf16 columns per thread

struct UnpermuteArgs {
    const uint16_t* y;       // [M_sum, H] bf16, row stride ld_y
    int64_t ld_y;
    int M_sum;
    int H;
    const int32_t* inv;      // [M, top_k]
    int top_k;
    const void* w;           // [M, top_k] fp32 or bf16
    int w_bf16;
    uint16_t* out;           // [M, H] bf16, row stride ld_out
    int64_t ld_out;
    int col_blocks;          // blocks per token
};

// bf16 bits of f, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// out[m, h] = bf16(sum over j = 0..top_k-1 of p_j), p_j = y[inv[m, j], h] * w[m, j]
// rounded to fp32 (fp32 weights) or bf16 (bf16 weights), summed in fp32 in
// slot order; no fused multiply-add, so every product and sum rounds once.
__global__ __launch_bounds__(kUnpermThreads) void moe_unpermute_kernel(const UnpermuteArgs a) {
#pragma clang fp contract(off)
    const int m = (int)blockIdx.x / a.col_blocks;
    const int cb = (int)blockIdx.x - m * a.col_blocks;
    const int c8 = cb * kUnpermThreads + (int)threadIdx.x;
    if (c8 * 8 >= a.H) return;
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.f;
    const int32_t* inv = a.inv + (int64_t)m * a.top_k;
    for (int j0 = 0; j0 < a.top_k; j0 += 4) {
        u32x4 v[4];
        float wt[4];
        bool use[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + u;
            use[u] = false;
            wt[u] = 0.f;
            v[u] = u32x4{0u, 0u, 0u, 0u};
            if (j < a.top_k) {
                const int r = inv[j];
                use[u] = r >= 0 && r < a.M_sum;
                const int64_t wi = (int64_t)m * a.top_k + j;
                wt[u] = a.w_bf16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.w)[wi] << 16)
                                 : reinterpret_cast<const float*>(a.w)[wi];
                if (use[u])
                    v[u] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(a.y + (int64_t)r * a.ld_y + (int64_t)c8 * 8));
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (!use[u]) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float p0 = bf16lo(v[u][q]) * wt[u];
                float p1 = bf16hi(v[u][q]) * wt[u];
                if (a.w_bf16) {
                    p0 = __uint_as_float(bf16_rne(p0) << 16);
                    p1 = __uint_as_float(bf16_rne(p1) << 16);
                }
                acc[2 * q] = acc[2 * q] + p0;
                acc[2 * q + 1] = acc[2 * q + 1] + p1;
            }
        }
    }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = bf16_rne(acc[2 * q]) | (bf16_rne(acc[2 * q + 1]) << 16);
    *reinterpret_cast<u32x4*>(a.out + (int64_t)m * a.ld_out + (int64_t)c8 * 8) = o;
}

// ------------------------------------------------------------- planning ---

struct PermutePlan {
    int chunk, nchunks;
    int64_t hist_off, rank_off, counts_off, offsets_off, bytes;
};

int64_t align16(int64_t v) { return (v + 15) & ~int64_t(15); }

PermutePlan permute_plan(int64_t n, int64_t E) {
    PermutePlan p{};
    const int64_t units = (n + kChunkUnit - 1) / kChunkUnit;
    const int64_t per = units <= kMaxChunks ? 1 : (units + kMaxChunks - 1) / kMaxChunks;
    p.chunk = (int)(per * kChunkUnit);
    p.nchunks = (int)((n + p.chunk - 1) / p.chunk);
    p.hist_off = 0;
    p.rank_off = align16((int64_t)p.nchunks * E * 4);
    p.counts_off = p.rank_off + align16(n * 4);
    p.offsets_off = p.counts_off + align16(E * 4);
    p.bytes = p.offsets_off + align16((E + 1) * 4);
    return p;
}

int64_t aligned_rows(int64_t M, int64_t k, int64_t E, int64_t align) {
    const int64_t t = M * k + E * (align - 1);
    return (t + align - 1) / align * align;
}

}  // namespace
}  // namespace kbn

using namespace kbn;

extern "C" int64_t kbn_moe_permute_workspace_bytes(int64_t num_pairs, int64_t num_experts) {
    if (num_pairs < 0 || num_pairs > 0x7FFFFFFFLL || num_experts < 1 || num_experts > kMaxExperts) return -1;
    return permute_plan(num_pairs, num_experts).bytes;
}

// The contiguous permute; quant 0: copy rows of x (row_bytes each) and their
// scales; quant 1 / 2: x holds bf16 rows of row_bytes elements, quantized
// 1x128 on the way (UE8M0 / fp32 scales, absmax floor eps).
static int permute_impl(const char* what, const void* topk_ids, int ids_bytes, int64_t M, int64_t top_k,
                        int64_t num_experts, int64_t alignment, const void* x, int64_t ld_x_bytes, int64_t row_bytes,
                        const float* x_scale, int64_t s_stride_m, int64_t s_stride_c, int64_t scale_cols,
                        int64_t M_sum, void* x_perm, float* scale_perm, int64_t sp_stride_m, int64_t sp_stride_c,
                        int32_t* expert_ids, int32_t* inv_perm, int zero_padding, void* workspace,
                        int64_t workspace_bytes, void* stream, int quant, float eps) {
    KBN_CHECK_ARG(ids_bytes == 4 || ids_bytes == 8, "%s: ids_bytes must be 4 or 8, got %d", what, ids_bytes);
    KBN_CHECK_ARG(M >= 0 && top_k >= 1 && M * top_k <= 0x7FFFFFFFLL, "%s: bad M=%lld top_k=%lld", what,
                  (long long)M, (long long)top_k);
    KBN_CHECK_ARG(num_experts >= 1 && num_experts <= kMaxExperts, "%s: num_experts=%lld outside [1, %d]", what,
                  (long long)num_experts, kMaxExperts);
    KBN_CHECK_ARG(alignment >= 1 && alignment <= (1 << 16), "%s: bad alignment %lld", what, (long long)alignment);
    const int64_t n = M * top_k;
    const int64_t want = aligned_rows(M, top_k, num_experts, alignment);
    KBN_CHECK_ARG(M_sum == want, "%s: M_sum=%lld, expected roundup(M*top_k + E*(alignment-1), alignment)=%lld", what,
                  (long long)M_sum, (long long)want);
    KBN_CHECK_ARG(M_sum <= 0x7FFFFFFFLL, "%s: M_sum=%lld too large", what, (long long)M_sum);
    KBN_CHECK_ARG(row_bytes >= 0 && row_bytes % 16 == 0 && row_bytes <= 0x7FFFFFFFLL,
                  "%s: row_bytes=%lld must be a multiple of 16", what, (long long)row_bytes);
    KBN_CHECK_ARG(scale_cols >= 0 && scale_cols <= 0x7FFFFFFFLL, "%s: bad scale_cols", what);
    KBN_CHECK_ARG(expert_ids, "%s: null expert_ids", what);
    if (n > 0) {
        KBN_CHECK_ARG(topk_ids && inv_perm, "%s: null topk_ids or inv_perm", what);
        if (row_bytes > 0)
            KBN_CHECK_ARG(x && aligned16(x) && ld_x_bytes >= row_bytes && ld_x_bytes % 16 == 0,
                          "%s: x must be 16-byte aligned with a row stride (%lld B) >= row_bytes and a multiple of 16",
                          what, (long long)ld_x_bytes);
        if (scale_cols > 0 && !quant) KBN_CHECK_ARG(x_scale, "%s: null x_scale", what);
    }
    if (row_bytes > 0) KBN_CHECK_ARG(x_perm && aligned16(x_perm), "%s: x_perm must be 16-byte aligned", what);
    if (scale_cols > 0) {
        KBN_CHECK_ARG(scale_perm, "%s: null scale_perm", what);
        // the rows x columns of scale_perm must not overlap: row-major, column-major or any
        // other layout whose strides separate them
        const bool rowmaj = sp_stride_c == 1 && sp_stride_m >= scale_cols;
        const bool colmaj = sp_stride_m == 1 && sp_stride_c >= M_sum;
        KBN_CHECK_ARG(rowmaj || colmaj, "%s: scale_perm strides (%lld, %lld) must be row-major (s_m >= %lld, 1) "
                      "or column-major (1, s_c >= %lld)", what, (long long)sp_stride_m, (long long)sp_stride_c,
                      (long long)scale_cols, (long long)M_sum);
    }
    const PermutePlan plan = permute_plan(n, num_experts);
    KBN_CHECK_ARG(workspace && aligned16(workspace) && workspace_bytes >= plan.bytes,
                  "%s: workspace of %lld bytes (16-byte aligned) needed, got %lld", what, (long long)plan.bytes,
                  (long long)workspace_bytes);

    PermuteArgs a{};
    a.ids = topk_ids;
    a.ids64 = ids_bytes == 8;
    a.n = (int)n;
    a.top_k = (int)top_k;
    a.E = (int)num_experts;
    int bits = 0;
    while ((1LL << bits) < num_experts) ++bits;
    a.bits = bits;
    a.align = (int)alignment;
    a.chunk = plan.chunk;
    a.nchunks = plan.nchunks;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    a.hist = reinterpret_cast<int*>(ws + plan.hist_off);
    a.rank = reinterpret_cast<int*>(ws + plan.rank_off);
    a.counts = reinterpret_cast<int*>(ws + plan.counts_off);
    a.offsets = reinterpret_cast<int*>(ws + plan.offsets_off);
    a.x = static_cast<const uint8_t*>(x);
    a.ld_x = ld_x_bytes;
    a.row_bytes = (int)row_bytes;
    a.xs = x_scale;
    a.xs_m = s_stride_m;
    a.xs_c = s_stride_c;
    a.scale_cols = (int)scale_cols;
    a.xp = static_cast<uint8_t*>(x_perm);
    a.sp = scale_perm;
    a.sp_m = sp_stride_m;
    a.sp_c = sp_stride_c;
    a.expert_ids = expert_ids;
    a.inv_perm = inv_perm;
    a.M_sum = (int)M_sum;
    a.zero_padding = zero_padding != 0;
    a.eps = eps;
    // a wavefront per routed pair (copy), kQuantWaves per token (quantizing)
    a.place_blocks = (int)(((quant ? M * kQuantWaves : n) + kPlaceWaves - 1) / kPlaceWaves);
    const int64_t pad_blocks = (M_sum + kPlaceWaves * kPadRowsPerWave - 1) / (kPlaceWaves * kPadRowsPerWave);

    hipStream_t st = static_cast<hipStream_t>(stream);
    if (a.nchunks > 0) {
        moe_count_kernel<<<dim3(a.nchunks), dim3(64), 0, st>>>(a);
        KBN_CHECK_LAUNCH(what);
    }
    moe_scan_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    const int64_t blocks = a.place_blocks + pad_blocks;
    if (blocks > 0) {
        if (quant == 1) moe_place_kernel<1><<<dim3((unsigned)blocks), dim3(64 * kPlaceWaves), 0, st>>>(a);
        else if (quant == 2) moe_place_kernel<2><<<dim3((unsigned)blocks), dim3(64 * kPlaceWaves), 0, st>>>(a);
        else moe_place_kernel<0><<<dim3((unsigned)blocks), dim3(64 * kPlaceWaves), 0, st>>>(a);
        KBN_CHECK_LAUNCH(what);
    }
    return 0;
}

extern "C" int kbn_moe_permute_contiguous(const void* topk_ids, int ids_bytes, int64_t M, int64_t top_k,
                                          int64_t num_experts, int64_t alignment, const void* x, int64_t ld_x_bytes,
                                          int64_t row_bytes, const float* x_scale, int64_t s_stride_m,
                                          int64_t s_stride_c, int64_t scale_cols, int64_t M_sum, void* x_perm,
                                          float* scale_perm, int64_t sp_stride_m, int64_t sp_stride_c,
                                          int32_t* expert_ids, int32_t* inv_perm,
                                          int zero_padding, void* workspace, int64_t workspace_bytes, void* stream) {
    return permute_impl("moe_permute_contiguous", topk_ids, ids_bytes, M, top_k, num_experts, alignment, x,
                        ld_x_bytes, row_bytes, x_scale, s_stride_m, s_stride_c, scale_cols, M_sum, x_perm,
                        scale_perm, sp_stride_m, sp_stride_c, expert_ids, inv_perm, zero_padding, workspace,
                        workspace_bytes, stream, 0, 0.0f);
}

extern "C" int kbn_moe_permute_quant_contiguous(const void* topk_ids, int ids_bytes, int64_t M, int64_t top_k,
                                                int64_t num_experts, int64_t alignment, const void* x_bf16,
                                                int64_t ld_x, int64_t K, float eps, int use_ue8m0, int64_t M_sum,
                                                void* x_perm, float* scale_perm, int64_t sp_stride_m,
                                                int64_t sp_stride_c, int32_t* expert_ids, int32_t* inv_perm,
                                                int zero_padding, void* workspace, int64_t workspace_bytes,
                                                void* stream) {
    const char* what = "moe_permute_quant_contiguous";
    KBN_CHECK_ARG(K >= 0 && K % kGroup == 0 && K <= 0x3FFFFFFFLL, "%s: K=%lld must be a multiple of 128", what,
                  (long long)K);
    KBN_CHECK_ARG(top_k >= 1 && top_k <= 64, "%s: top_k=%lld outside [1, 64]", what, (long long)top_k);
    KBN_CHECK_ARG(ld_x >= K && ld_x <= 0x3FFFFFFFLL, "%s: ld_x=%lld < K", what, (long long)ld_x);
    KBN_CHECK_ARG(M == 0 || (x_bf16 && aligned16(x_bf16) && ld_x % 8 == 0),
                  "%s: x rows must be 16-byte aligned", what);
    return permute_impl(what, topk_ids, ids_bytes, M, top_k, num_experts, alignment, x_bf16, ld_x * 2, K, nullptr, 0,
                        0, K / kGroup, M_sum, x_perm, scale_perm, sp_stride_m, sp_stride_c, expert_ids, inv_perm,
                        zero_padding, workspace, workspace_bytes, stream, use_ue8m0 ? 1 : 2, eps);
}

extern "C" int kbn_moe_align_block_size(const void* topk_ids, int ids_bytes, int64_t numel, int64_t num_experts,
                                        int64_t block_size, int32_t* sorted_token_ids, int64_t sorted_len,
                                        int32_t* expert_ids, int64_t expert_len, int32_t* num_tokens_post_pad,
                                        int32_t* cumsum, void* workspace, int64_t workspace_bytes, void* stream) {
    const char* what = "moe_align_block_size";
    KBN_CHECK_ARG(ids_bytes == 4 || ids_bytes == 8, "%s: ids_bytes must be 4 or 8, got %d", what, ids_bytes);
    KBN_CHECK_ARG(numel >= 0 && numel <= 0x3FFFFFFFLL, "%s: bad numel=%lld", what, (long long)numel);
    KBN_CHECK_ARG(num_experts >= 1 && num_experts <= kMaxExperts, "%s: num_experts=%lld outside [1, %d]", what,
                  (long long)num_experts, kMaxExperts);
    KBN_CHECK_ARG(block_size >= 1 && block_size <= (1 << 16), "%s: bad block_size %lld", what, (long long)block_size);
    // the padded total never exceeds numel + min(numel, E) * (block_size - 1)
    const int64_t bound = numel + std::min(numel, num_experts) * (block_size - 1);
    KBN_CHECK_ARG(sorted_len >= bound && sorted_len <= 0x7FFFFFFFLL,
                  "%s: sorted_token_ids holds %lld slots, the layout may need %lld", what, (long long)sorted_len,
                  (long long)bound);
    KBN_CHECK_ARG(expert_len * block_size >= bound, "%s: expert_ids holds %lld blocks, the layout may need %lld", what,
                  (long long)expert_len, (long long)((bound + block_size - 1) / block_size));
    KBN_CHECK_ARG(sorted_token_ids && expert_ids && num_tokens_post_pad, "%s: null output", what);
    if (numel > 0) KBN_CHECK_ARG(topk_ids, "%s: null topk_ids", what);
    const PermutePlan plan = permute_plan(numel, num_experts);
    KBN_CHECK_ARG(workspace && aligned16(workspace) && workspace_bytes >= plan.bytes,
                  "%s: workspace of %lld bytes (16-byte aligned) needed, got %lld", what, (long long)plan.bytes,
                  (long long)workspace_bytes);
    PermuteArgs a{};
    a.ids = topk_ids;
    a.ids64 = ids_bytes == 8;
    a.n = (int)numel;
    a.top_k = 1;
    a.E = (int)num_experts;
    int bits = 0;
    while ((1LL << bits) < num_experts) ++bits;
    a.bits = bits;
    a.align = (int)block_size;
    a.chunk = plan.chunk;
    a.nchunks = plan.nchunks;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    a.hist = reinterpret_cast<int*>(ws + plan.hist_off);
    a.rank = reinterpret_cast<int*>(ws + plan.rank_off);
    a.counts = reinterpret_cast<int*>(ws + plan.counts_off);
    a.offsets = reinterpret_cast<int*>(ws + plan.offsets_off);
    a.expert_ids = expert_ids;
    a.sorted_ids = sorted_token_ids;
    a.sorted_len = (int)sorted_len;
    a.post_pad = num_tokens_post_pad;
    a.cumsum_out = cumsum;
    a.place_blocks = (int)((numel + kAlignThreads - 1) / kAlignThreads);
    const int64_t fill_blocks = (sorted_len + kAlignThreads - 1) / kAlignThreads;

    hipStream_t st = static_cast<hipStream_t>(stream);
    if (a.nchunks > 0) {
        moe_count_kernel<<<dim3(a.nchunks), dim3(64), 0, st>>>(a);
        KBN_CHECK_LAUNCH(what);
    }
    moe_scan_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    moe_align_place_kernel<<<dim3((unsigned)(a.place_blocks + std::max<int64_t>(fill_blocks, 1))),
                             dim3(kAlignThreads), 0, st>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_moe_sum(const void* x_bf16, int64_t M, int64_t top_k, int64_t H, int64_t ld_x, void* out_bf16,
                           int64_t ld_out, void* stream) {
    const char* what = "moe_sum";
    KBN_CHECK_ARG(M >= 0 && top_k >= 1 && M * top_k <= 0x7FFFFFFFLL, "%s: bad M=%lld top_k=%lld", what,
                  (long long)M, (long long)top_k);
    KBN_CHECK_ARG(H >= 0 && H <= 0x7FFFFFFFLL && ld_x >= H && ld_out >= H, "%s: bad H or row strides", what);
    if (M == 0 || H == 0) return 0;
    KBN_CHECK_ARG(x_bf16 && out_bf16, "%s: null pointer", what);
    MoeSumArgs a{};
    a.x = static_cast<const uint16_t*>(x_bf16);
    a.ld_x = ld_x;
    a.top_k = (int)top_k;
    a.H = (int)H;
    a.out = static_cast<uint16_t*>(out_bf16);
    a.ld_out = ld_out;
    a.vec = aligned16(x_bf16) && aligned16(out_bf16) && ld_x % 8 == 0 && ld_out % 8 == 0;
    a.col_blocks = (int)(((H + 7) / 8 + kSumThreads - 1) / kSumThreads);
    const int64_t blocks = M * a.col_blocks;
    KBN_CHECK_ARG(blocks <= 0x7FFFFFFFLL, "%s: M*H too large", what);
    moe_sum_kernel<<<dim3((unsigned)blocks), dim3(kSumThreads), 0, static_cast<hipStream_t>(stream)>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}

extern "C" int kbn_moe_unpermute_reduce(const void* y_bf16, int64_t M_sum, int64_t H, int64_t ld_y,
                                        const int32_t* inv_perm, int64_t M, int64_t top_k, const void* topk_weights,
                                        int weights_bf16, void* out_bf16, int64_t ld_out, void* stream) {
    const char* what = "moe_unpermute_reduce";
    KBN_CHECK_ARG(M >= 0 && top_k >= 1 && M * top_k <= 0x7FFFFFFFLL, "%s: bad M=%lld top_k=%lld", what,
                  (long long)M, (long long)top_k);
    KBN_CHECK_ARG(M_sum >= 0 && M_sum <= 0x7FFFFFFFLL, "%s: bad M_sum=%lld", what, (long long)M_sum);
    KBN_CHECK_ARG(H >= 0 && H % 8 == 0 && H <= 0x7FFFFFFFLL, "%s: H=%lld must be a multiple of 8", what,
                  (long long)H);
    if (M == 0 || H == 0) return 0;
    KBN_CHECK_ARG(inv_perm && topk_weights, "%s: null inv_perm or topk_weights", what);
    KBN_CHECK_ARG(out_bf16 && aligned16(out_bf16) && ld_out >= H && ld_out % 8 == 0,
                  "%s: out must be 16-byte aligned with a row stride >= H and a multiple of 8", what);
    KBN_CHECK_ARG(M_sum == 0 || (y_bf16 && aligned16(y_bf16) && ld_y >= H && ld_y % 8 == 0),
                  "%s: y must be 16-byte aligned with a row stride >= H and a multiple of 8", what);
    UnpermuteArgs a{};
    a.y = static_cast<const uint16_t*>(y_bf16);
    a.ld_y = ld_y;
    a.M_sum = (int)M_sum;
    a.H = (int)H;
    a.inv = inv_perm;
    a.top_k = (int)top_k;
    a.w = topk_weights;
    a.w_bf16 = weights_bf16 != 0;
    a.out = static_cast<uint16_t*>(out_bf16);
    a.ld_out = ld_out;
    a.col_blocks = (int)((H / 8 + kUnpermThreads - 1) / kUnpermThreads);
    const int64_t blocks = M * a.col_blocks;
    KBN_CHECK_ARG(blocks <= 0x7FFFFFFFLL, "%s: M*H too large", what);
    moe_unpermute_kernel<<<dim3((unsigned)blocks), dim3(kUnpermThreads), 0, static_cast<hipStream_t>(stream)>>>(a);
    KBN_CHECK_LAUNCH(what);
    return 0;
}
