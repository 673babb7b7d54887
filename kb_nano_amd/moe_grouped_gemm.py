"""The free-function grouped GEMM entry that kb_nano's MoE block calls.

Mirrors ``tasks/baseline/L1/moe_grouped_gemm.py:32-83``: the gating helpers
``_is_deep_gemm_supported``, ``_deep_gemm_alignment``,
``_valid_deep_gemm_shape``, ``_valid_deep_gemm`` and the wrapper
``m_grouped_fp8_gemm_nt_contiguous((a, sa), (b, sb), out, expert_ids)``,
which always runs with ``disable_ue8m0_cast=True`` (checkpoint fp32 scales
used as given).
"""
from __future__ import annotations

import functools

import torch

from . import _ops
from .fp8_grouped_gemm_contiguous import _ALIGNMENT
from .fp8_grouped_gemm_contiguous import _is_deep_gemm_supported as _supported

_BLOCK_ALIGNMENT = _ALIGNMENT


def _is_deep_gemm_supported() -> bool:
    return _supported()


@functools.cache
def _deep_gemm_alignment() -> int:
    return _BLOCK_ALIGNMENT


def _valid_deep_gemm_shape(M: int, N: int, K: int) -> bool:
    align = _deep_gemm_alignment()
    return align <= M and N % align == 0 and K % align == 0


def _valid_deep_gemm(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> bool:
    """Same gate as the reference (:54-68): supported device, aligned shapes,
    N > 512, fp8 weights, contiguous operands."""
    if not _is_deep_gemm_supported():
        return False
    M = hidden_states.size(0)
    _, K, N = w2.size()
    if not _valid_deep_gemm_shape(M, N, K):
        return False
    if N <= 512:
        return False
    if w1.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
        return False
    return hidden_states.is_contiguous() and w1.is_contiguous() and w2.is_contiguous()


def m_grouped_fp8_gemm_nt_contiguous(a_and_scale, b_and_scale, output, expert_ids) -> None:
    """Grouped GEMM over an expert-contiguous A (reference :71-83)."""
    a, sa = a_and_scale
    b, sb = b_and_scale
    _ops.m_grouped_gemm_nt_contiguous(a, sa, b, sb, output, expert_ids, disable_ue8m0_cast=True)
