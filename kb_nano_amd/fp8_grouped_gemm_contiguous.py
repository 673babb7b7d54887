"""Grouped FP8 GEMM for MoE experts, contiguous layout.

Drop-in for ``tasks/baseline/L1/fp8_grouped_gemm_contiguous.py`` (kb_nano):
same class, ``alignment()``, gating helpers and op
``torch.ops.kb_nano_fp8_moe.m_grouped_gemm_nt_contiguous``, backed by the
gfx950 grouped GEMM kernel.

Layout contract: A is expert-contiguous [M_sum, K] fp8 with fp32 scales
[M_sum, K/128] (row- or column-major), B is [E, N, K] fp8 with fp32 scales
[E, ceil(N/128), K/128], C is [M_sum, N] bf16 written in place, and
``expert_ids[r]`` names row r's expert.  Rows are processed in 128-row blocks
(the alignment); each block uses the expert of its first row, rows with id -1
(padding) are not written.
"""
from __future__ import annotations

import functools
import os

import torch
import torch.nn as nn

from . import _ops  # also registers torch.ops.kb_nano_fp8_moe.*
from ._ops import is_e8m0_used

_ALIGNMENT = 128


@functools.cache
def _is_deep_gemm_supported() -> bool:
    """Reference :29-50 gates on env + import + SM90/SM100.  Here: the env
    switch ``VLLM_USE_DEEP_GEMM`` and a gfx950 device."""
    if not bool(int(os.environ.get("VLLM_USE_DEEP_GEMM", "1"))):
        return False
    if not torch.cuda.is_available():
        return False
    try:
        return torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName.startswith("gfx950")
    except Exception:
        return False


def _is_deep_gemm_e8m0_used() -> bool:
    """Reference :53-71: UE8M0 scale contract on (default) or off."""
    return is_e8m0_used()


def _resolve_alignment() -> int:
    """M/K alignment of the contiguous layout (reference :77-90): the grouped
    kernel's 128-row block."""
    return _ALIGNMENT


class Fp8GroupedGemmContiguous(nn.Module):
    """``(A_fp8, a_scale) @ (B_fp8, b_scale) -> C_bf16`` per expert-contiguous
    row block; ``forward(a_fp8, a_scale, b_fp8, b_scale, c_bf16, expert_ids)``
    writes C in place and returns None."""

    def __init__(self) -> None:
        super().__init__()
        self._alignment: int = _resolve_alignment()
        self._disable_ue8m0_cast: bool = not _is_deep_gemm_e8m0_used()

    def alignment(self) -> int:
        return self._alignment

    def forward(self, a_fp8: torch.Tensor, a_scale: torch.Tensor, b_fp8: torch.Tensor,
                b_scale: torch.Tensor, c_bf16: torch.Tensor, expert_ids: torch.Tensor) -> None:
        if torch.compiler.is_compiling():
            torch.ops.kb_nano_fp8_moe.m_grouped_gemm_nt_contiguous(
                a_fp8, a_scale, b_fp8, b_scale, c_bf16, expert_ids, self._disable_ue8m0_cast)
        else:   # eager: the same launch without the dispatcher round trip
            _ops.m_grouped_gemm_nt_contiguous(a_fp8, a_scale, b_fp8, b_scale, c_bf16, expert_ids,
                                              self._disable_ue8m0_cast)
