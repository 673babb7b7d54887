"""The MoE grouped GEMMs that kb_nano's MoE blocks call.

Mirrors ``tasks/baseline/L1/moe_grouped_gemm.py``:

  * :32-83, the contiguous layout: the gating helpers
    ``_is_deep_gemm_supported``, ``_deep_gemm_alignment``,
    ``_valid_deep_gemm_shape``, ``_valid_deep_gemm`` and the wrapper
    ``m_grouped_fp8_gemm_nt_contiguous((a, sa), (b, sb), out, expert_ids)``,
    which always runs with ``disable_ue8m0_cast=True`` (checkpoint fp32
    scales used as given);
  * :86-382, the sorted-token layout: ``MoeGroupedGemm.forward`` with the
    arguments of the reference's Triton ``_fused_moe_kernel`` launcher, and
    ``get_triton_config`` / ``_get_default_config`` (the names are kept; the
    configurations are this build's gfx950 kernel's).  Only the FP8 W8A8
    path with 128x128 block scales is built: BF16 experts and other block
    shapes raise ``NotImplementedError``.
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


# --------------------------------------------------------- sorted-token path

# Rows per expert block of the sorted-token layout.  The gfx950 kernel tiles
# 64 or 128 rows x 256 columns, so the block size is a multiple of 64:
# 64 while the routed pairs are few (decode: less padding per expert), 128
# beyond (fewer tiles).
_DEFAULT_CONFIG_HEURISTIC = {
    "small": {"BLOCK_SIZE_M": 64, "BLOCK_SIZE_N": 256, "BLOCK_SIZE_K": 128, "GROUP_SIZE_M": 4},
    "large": {"BLOCK_SIZE_M": 128, "BLOCK_SIZE_N": 256, "BLOCK_SIZE_K": 128, "GROUP_SIZE_M": 4},
}


def _get_default_config(M: int, E: int = 0, N: int = 0, block_shape: list[int] | None = None) -> dict:
    """Kernel configuration for M tokens (reference :273-279)."""
    return dict(_DEFAULT_CONFIG_HEURISTIC["small" if M <= 64 else "large"])


def get_triton_config(M: int, w1_shape: tuple[int, ...], w2_shape: tuple[int, ...], top_k: int, use_fp8: bool,
                      block_shape: list[int] | None = None) -> dict:
    """Configuration of the sorted-token GEMM for M tokens (reference
    :282-297; no tuning files: the block size is the only choice)."""
    E, _, N = w2_shape
    return _get_default_config(M, E, N, block_shape)


class MoeGroupedGemm(torch.nn.Module):
    """Sorted-token FP8 grouped GEMM (reference :300-382)."""

    @staticmethod
    def get_config(M: int, N: int = 0, E: int = 0, use_fp8: bool = False,
                   block_shape: list[int] | None = None) -> dict:
        return _get_default_config(M, E, N, block_shape)

    def forward(self, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, topk_weights: torch.Tensor | None,
                sorted_token_ids: torch.Tensor | None, expert_ids: torch.Tensor,
                num_tokens_post_padded: torch.Tensor, mul_routed_weight: bool, top_k: int,
                config: dict | None = None, a_scale: torch.Tensor | None = None,
                b_scale: torch.Tensor | None = None, use_fp8_w8a8: bool = False,
                block_shape: list[int] | None = None):
        """C[t] = (A[t // top_k] @ B[e]^T) (times topk_weights[t] when
        mul_routed_weight) for every routed pair t of the sorted-token layout;
        C has one row per pair (A.size(0) * top_k rows)."""
        if not use_fp8_w8a8 or block_shape is None or list(block_shape) != [128, 128]:
            raise NotImplementedError("MoeGroupedGemm: only FP8 W8A8 with 128x128 block scales is on this path "
                                      "(the reference runs other types through its Triton kernel)")
        if a_scale is None or b_scale is None:
            raise ValueError("MoeGroupedGemm: FP8 needs a_scale and b_scale")
        config = _get_default_config(A.size(0), N=B.size(1)) if config is None else config
        block_m = int(config["BLOCK_SIZE_M"])
        if block_m % 64 != 0:
            raise NotImplementedError(f"MoeGroupedGemm: BLOCK_SIZE_M={block_m}; the gfx950 kernel takes "
                                      f"multiples of 64 (align the tokens with get_triton_config's block size)")
        if sorted_token_ids is None:
            EM = expert_ids.numel() * block_m
        else:
            EM = sorted_token_ids.size(0)
            if A.size(0) < block_m:
                EM = min(EM, A.size(0) * top_k * block_m)
        num_valid = A.size(0) * top_k
        c = C.reshape(-1, C.size(-1))
        if c.size(0) != num_valid:
            raise ValueError(f"MoeGroupedGemm: C must hold {num_valid} rows, got {tuple(C.shape)}")
        w = None
        if mul_routed_weight:
            w = topk_weights.reshape(-1)
            w = w if w.dtype == torch.float32 and w.is_contiguous() else w.to(torch.float32).contiguous()
        _ops.fused_moe_gemm(A, a_scale, B, b_scale, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                            EM, block_m, top_k, topk_weights=w)
