"""kernel_swapper candidate for target ``moe_grouped_gemm`` (class
``MoeGroupedGemm``, with the module's free functions); copy to
``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.moe_grouped_gemm import (  # noqa: F401
    MoeGroupedGemm,
    _valid_deep_gemm,
    get_triton_config,
    m_grouped_fp8_gemm_nt_contiguous,
)
