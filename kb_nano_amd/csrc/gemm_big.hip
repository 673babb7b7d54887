// The 256x256 dense GEMM tiles (M > 128, UE8M0 contract; kernels in
// gemm_kernel.h).  Built without the VGPR-form MFMA option that gemm.hip
// uses: each wavefront holds 128x128 fp32 accumulators (256 per lane), which
// need the AGPRs; forced into VGPRs they cost 5-7% at M = 4096.
#include "gemm_kernel.h"

namespace kbn {

int launch_gemm_256(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    // two wavefronts per SIMD when K is short enough that the per-tile fill
    // and epilogue matter (q_b_proj, K = 1536)
    if (K <= 2048) return launch_gemm<256, 256, 2, true, false, 8>(a, sc, st, what);
    return launch_gemm<256, 256, 2, true, false>(a, sc, st, what);
}

// The same tiles with packed per-row UE8M0 weight scales (GemmArgs::sWp).
int launch_gemm_256_roww(const GemmArgs& a, const Schedule& sc, int64_t K, hipStream_t st, const char* what) {
    if (K <= 2048) return launch_gemm<256, 256, 2, true, false, 8, 0, true>(a, sc, st, what);
    return launch_gemm<256, 256, 2, true, false, 4, 0, true>(a, sc, st, what);
}

}  // namespace kbn
