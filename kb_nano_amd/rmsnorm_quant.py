"""Fused RMSNorm (+ residual add) + per-token-group FP8 quantization.

Drop-in for ``tasks/baseline/L1/rmsnorm_quant.py`` (kb_nano): the same two
modules with the same ``forward`` signatures and column-major scale output,
and the ops ``kb_nano_norm::rmsnorm_fp8_quant`` /
``kb_nano_norm::fused_add_rmsnorm_fp8_quant`` with the reference schemas
(registered by ``_ops``).  One gfx950 launch (``csrc/norm.hip``) per call,
one workgroup of 4 or 8 wavefronts per token.

Numerics (reference ``csrc/rmsnorm_quant.cu:21-201``): the normalized value
``(x * inv_rms) * w`` stays fp32 until the UE8M0 1x128 quantization; the
fused variant adds the residual first (fp32), stores it back as bf16, and
overwrites ``input`` with the normalized row.  bf16, fp16 or fp32
activations, as the reference dispatches (weight and residual of the
input's type), any hidden size that is a multiple of 8: rows of up to 16384
columns (8192 with the residual add) in registers, longer rows and the
fp16 / fp32 types by a kernel that reads each row twice, in the same
summation order.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _ops  # also registers torch.ops.kb_nano_norm.*
from ._ops import FP8, GROUP

_FP8_GROUP_SIZE = GROUP


def _outputs(input: torch.Tensor):
    hidden_size = input.size(-1)
    num_tokens = input.numel() // hidden_size
    num_groups = (hidden_size + _FP8_GROUP_SIZE - 1) // _FP8_GROUP_SIZE
    output_fp8 = torch.empty(num_tokens, hidden_size, dtype=FP8, device=input.device)
    output_scales = torch.empty_strided((num_tokens, num_groups), (1, max(num_tokens, 1)), dtype=torch.float32,
                                        device=input.device)
    return output_fp8, output_scales


class RMSNormFP8Quant(nn.Module):
    """``forward(input, weight, eps=1e-6) -> (output_fp8, output_scales)``:
    output_fp8 [num_tokens, hidden] float8_e4m3fn, output_scales [num_tokens,
    num_groups] float32 column-major (reference :65-98)."""

    def forward(self, input: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
        output_fp8, output_scales = _outputs(input)
        if torch.compiler.is_compiling():
            torch.ops.kb_nano_norm.rmsnorm_fp8_quant(output_fp8, output_scales, input, weight, eps)
        else:   # eager: the same launch without the dispatcher round trip
            _ops.rmsnorm_fp8_quant(output_fp8, output_scales, input, weight, eps)
        return output_fp8, output_scales


class FusedAddRMSNormFP8Quant(nn.Module):
    """``forward(input, residual, weight, eps=1e-6) -> (output_fp8,
    output_scales, residual)``; modifies ``input`` (normalized row) and
    ``residual`` (residual + input) in place (reference :101-134)."""

    def forward(self, input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        output_fp8, output_scales = _outputs(input)
        if torch.compiler.is_compiling():
            torch.ops.kb_nano_norm.fused_add_rmsnorm_fp8_quant(output_fp8, output_scales, input, residual, weight, eps)
        else:   # eager: the same launch without the dispatcher round trip
            _ops.rmsnorm_fp8_quant(output_fp8, output_scales, input, weight, eps, residual=residual)
        return output_fp8, output_scales, residual
