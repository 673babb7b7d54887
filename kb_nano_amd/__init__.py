"""kb_nano_amd: kb_nano's block-scaled FP8 linear path, native to MI355X (gfx950).

Four operators, each a drop-in for its kb_nano L1 counterpart:

  * ``PerTokenGroupQuantFp8``   1x128 activation quant with UE8M0 scales
  * ``SiluMulQuantFp8``         fused SiLU*Mul + 1x128 FP8 quant
  * ``Fp8Linear``               128x128 block-scaled FP8 GEMM, fp32 accumulate, bf16 out
  * ``Fp8GroupedGemmContiguous``  its contiguous-layout MoE grouped variant

and ``FusedExperts``, the MoE experts layer that chains them (quant, permute,
grouped GEMM, SiLU*Mul+quant, grouped GEMM, weighted unpermute), its
sorted-token counterpart ``VllmFusedExperts`` (``MoeAlign``,
``MoeGroupedGemm``, ``MoeSum``), plus the
fused ``RMSNormFP8Quant`` / ``FusedAddRMSNormFP8Quant`` that produce the
quantized activations of a decoder layer's first linear.

The compute runs in hand-written gfx950 HIP kernels (``csrc/``) behind the
C-ABI of ``libkbn_fp8.so`` (declared in ``include/kbn_fp8.h``); this package
is the PyTorch-side host layer.
"""
from .fp8_grouped_gemm_contiguous import Fp8GroupedGemmContiguous
from .fused_experts import FusedExperts
from .fp8_linear import (
    Fp8Linear,
    PerTokenGroupQuantFp8,
    _alloc_colmajor_scale,
    _Fp8PrefillBufs,
    postprocess_fp8_weights,
    postprocess_fp8_weights_batched,
)
from .moe_align import MoeAlign
from .moe_grouped_gemm import MoeGroupedGemm, m_grouped_fp8_gemm_nt_contiguous
from .moe_sum import MoeSum
from .rmsnorm_quant import FusedAddRMSNormFP8Quant, RMSNormFP8Quant
from .silu_mul_quant_fp8 import SiluMulQuantFp8
from .vllm_fused_experts import VllmFusedExperts
from .weight_path import postprocess_model_fp8_weights, warmup_fp8_linear

__all__ = [
    "Fp8Linear",
    "PerTokenGroupQuantFp8",
    "SiluMulQuantFp8",
    "Fp8GroupedGemmContiguous",
    "FusedExperts",
    "VllmFusedExperts",
    "MoeAlign",
    "MoeGroupedGemm",
    "MoeSum",
    "RMSNormFP8Quant",
    "FusedAddRMSNormFP8Quant",
    "postprocess_model_fp8_weights",
    "warmup_fp8_linear",
    "m_grouped_fp8_gemm_nt_contiguous",
    "postprocess_fp8_weights",
    "postprocess_fp8_weights_batched",
    "_alloc_colmajor_scale",
    "_Fp8PrefillBufs",
]
