"""kernel_swapper candidate for target ``fp8_grouped_gemm_contiguous`` (class
``Fp8GroupedGemmContiguous``); copy to ``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.fp8_grouped_gemm_contiguous import Fp8GroupedGemmContiguous  # noqa: F401
