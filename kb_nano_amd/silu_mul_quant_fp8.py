"""Fused SiLU*Mul + per-token-group FP8 quant with column-major scales.

Drop-in for ``tasks/baseline/L1/silu_mul_quant_fp8.py`` (kb_nano): same class,
same ``forward`` signature, assertions and output layout, one gfx950 HIP
launch instead of the Triton kernel.

Numerics (reference :57-66): silu(gate) is rounded once to bf16 (correctly
rounded), multiplied by up (exact in fp32) and rounded to bf16, then each
1x128 group is quantized with a UE8M0 (or plain fp32) scale.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _ops  # also registers torch.ops.kb_nano_fp8.*
from ._ops import FP8, GROUP

_FP8_INFO = torch.finfo(FP8)
_GROUP_SIZE = GROUP


class SiluMulQuantFp8(nn.Module):
    """``forward(input, output=None, use_ue8m0=True, eps=1e-10) -> (q, s)``:
    input bf16 [M, 2*N'] (gate | up), q float8_e4m3fn [M, N'] (``output`` if
    given), s float32 [M, N'/128] column-major (storage [N'/128, M])."""

    def forward(self, input: torch.Tensor, output: torch.Tensor | None = None,
                use_ue8m0: bool = True, eps: float = 1e-10) -> tuple[torch.Tensor, torch.Tensor]:
        assert input.ndim == 2
        M, N = input.size()
        N_2 = N // 2
        assert M % _GROUP_SIZE == 0, f"M={M} must be divisible by {_GROUP_SIZE}"
        assert N_2 % _GROUP_SIZE == 0, f"N//2={N_2} must be divisible by {_GROUP_SIZE}"
        if output is None:
            output = torch.empty((M, N_2), dtype=FP8, device=input.device)
        output_scales = torch.empty_strided((M, N_2 // _GROUP_SIZE), (1, M), dtype=torch.float32,
                                            device=input.device)
        if torch.compiler.is_compiling():
            torch.ops.kb_nano_fp8.silu_mul_quant_fp8(input, output, output_scales, bool(use_ue8m0), float(eps))
        else:   # eager: the same launch without the dispatcher round trip
            _ops.silu_mul_quant_fp8(input, output, output_scales, bool(use_ue8m0), float(eps))
        return output, output_scales
