// The 256x256 dense GEMM tiles (M > 128, UE8M0 contract; kernels in
// gemm_kernel.h).  Built without the VGPR-form MFMA option that gemm.hip
// uses: each wavefront holds 128x128 fp32 accumulators (256 per lane), which
// need the AGPRs; forced into VGPRs they cost 5-7% at M = 4096.
#include "gemm_kernel.h"

namespace kbn {

// A mixed plan (sc.n192 > 0): columns [0, N - n192) as 256x256 tiles, the
// rest as 256x192 tiles in a second launch on the same stream, with W, its
// scales and D offset to the second part (N - n192 is a multiple of 256, so
// the scale rows stay whole 128-row blocks).
template <bool kRowW>
static int launch_mixed(const GemmArgs& a, const Schedule& sc, hipStream_t st, const char* what) {
    const int n256 = a.N - sc.n192;
    const int64_t tm = (a.M + 255) / 256;
    KBN_CHECK_ARG(n256 >= 0 && n256 % 256 == 0 && sc.n192 % 192 == 0 && sc.splits == 1,
                  "%s: mixed 256/192 plan does not match N", what);
    if (n256 > 0) {
        GemmArgs a1 = a;
        a1.N = n256;
        Schedule s1 = sc;
        s1.n192 = 0;
        s1.tiles = s1.dp_tiles = tm * (n256 / 256);
        if (int rc = launch_gemm<256, 256, 2, true, false, 4, 0, kRowW>(a1, s1, st, what)) return rc;
    }
    GemmArgs a2 = a;
    a2.N = sc.n192;
    a2.W += (int64_t)n256 * a.ldw;
    a2.D += n256;
    a2.vec_store = a.vec_store && (n256 % 8 == 0);
    if constexpr (kRowW) {
        a2.sWp += (int64_t)n256 * a.sWp_sn;
        a2.sWp_bytes -= (int64_t)n256 * a.sWp_sn * 4;
    } else {
        a2.sW += (int64_t)(n256 / 128) * a.sW_ld;
    }
    Schedule s2 = sc;
    s2.bn = 192;
    s2.n192 = 0;
    s2.tiles = s2.dp_tiles = tm * (sc.n192 / 192);
    return launch_gemm<256, 192, 2, true, false, 4, 0, kRowW>(a2, s2, st, what);
}

int launch_gemm_256(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    if (sc.n192 > 0) return launch_mixed<false>(a, sc, st, what);
    // two wavefronts per SIMD when K is short enough that the per-tile fill
    // and epilogue matter (q_b_proj, K = 1536)
    if (K <= 2048) return launch_gemm<256, 256, 2, true, false, 8>(a, sc, st, what);
    return launch_gemm<256, 256, 2, true, false>(a, sc, st, what);
}

// The same tiles with packed per-row UE8M0 weight scales (GemmArgs::sWp).
int launch_gemm_256_roww(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    if (sc.n192 > 0) return launch_mixed<true>(a, sc, st, what);
    if (K <= 2048) return launch_gemm<256, 256, 2, true, false, 8, 0, true>(a, sc, st, what);
    return launch_gemm<256, 256, 2, true, false, 4, 0, true>(a, sc, st, what);
}

}  // namespace kbn
