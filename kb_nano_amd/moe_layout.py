"""Contiguous MoE layout: aligned row count, permute, unpermute-and-reduce.

Mirrors ``tasks/baseline/L2/fused_experts.py:32-136`` (kb_nano), the layout
contract the grouped GEMM consumes.  The permute and the reduction run in the
gfx950 kernels of ``csrc/moe.hip`` (``kbn_moe_permute_contiguous``,
``kbn_moe_unpermute_reduce``) where the reference chains ~40 torch ops; both
are asynchronous on the current stream with no host synchronisation, so they
can be captured into a HIP graph.

Layout: expert e owns rows [off[e], off[e] + roundup(count[e], align)) of
the permuted activations; its ``count[e]`` tokens fill the first rows in
(token, slot) order and carry ``expert_ids = e``; the remaining rows are zero
padding with ``expert_ids = -1``.  ``inv_perm[m, j]`` is the permuted row of
token m's j-th expert.
"""
from __future__ import annotations

import torch

from . import _ops

_GROUP = 128


def _compute_aligned_M(M: int, num_topk: int, local_num_experts: int, alignment: int) -> int:
    """M_sum = roundup(M*k + E*(align-1), align) (reference :32-39)."""
    total = M * num_topk + local_num_experts * (alignment - 1)
    return -(-total // alignment) * alignment


def _deepgemm_permute(hidden_states: torch.Tensor, a_scale: torch.Tensor, topk_ids: torch.Tensor,
                      local_num_experts: int, alignment: int, zero_padding: bool = True,
                      scale_colmajor: bool = False):
    """Scatter (token, slot) rows into the expert-contiguous layout
    (reference :42-116).  Returns (a_perm, a_scale_perm, expert_ids, inv_perm).

    ``zero_padding=False`` leaves the padding rows of ``a_perm`` and
    ``a_scale_perm`` unwritten: the grouped GEMM never writes a padding row of
    its output, so the experts layer does not need them zeroed.
    ``scale_colmajor=True`` returns ``a_scale_perm`` as a column-major view
    (strides ``(1, M_sum)``, same values): the grouped GEMM then reads each K
    block's row scales as one contiguous run instead of one cache line per
    row."""
    M, K = hidden_states.shape
    k = topk_ids.size(1)
    dev = hidden_states.device
    M_sum = _compute_aligned_M(M, k, local_num_experts, alignment)
    a_perm = torch.empty(M_sum, K, dtype=hidden_states.dtype, device=dev)
    if scale_colmajor:
        a_scale_perm = torch.empty(K // _GROUP, M_sum, dtype=torch.float32, device=dev).t()
    else:
        a_scale_perm = torch.empty(M_sum, K // _GROUP, dtype=torch.float32, device=dev)
    expert_ids = torch.empty(M_sum, dtype=torch.int32, device=dev)
    inv_perm = torch.empty(M, k, dtype=torch.int32, device=dev)
    _ops.moe_permute_contiguous(hidden_states, a_scale, topk_ids.contiguous(), local_num_experts, alignment, M_sum,
                                a_perm, a_scale_perm, expert_ids, inv_perm, zero_padding)
    return a_perm, a_scale_perm, expert_ids, inv_perm


def _deepgemm_permute_quant(hidden_states: torch.Tensor, topk_ids: torch.Tensor, local_num_experts: int,
                            alignment: int, zero_padding: bool = True, scale_colmajor: bool = False,
                            use_ue8m0: bool = True):
    """The 1x128 quant of bf16 ``hidden_states`` and ``_deepgemm_permute`` of
    its codes and scales in one launch: the same (a_perm, a_scale_perm,
    expert_ids, inv_perm) as the two steps, with no token-order fp8 copy."""
    M, K = hidden_states.shape
    k = topk_ids.size(1)
    dev = hidden_states.device
    M_sum = _compute_aligned_M(M, k, local_num_experts, alignment)
    a_perm = torch.empty(M_sum, K, dtype=torch.float8_e4m3fn, device=dev)
    if scale_colmajor:
        a_scale_perm = torch.empty(K // _GROUP, M_sum, dtype=torch.float32, device=dev).t()
    else:
        a_scale_perm = torch.empty(M_sum, K // _GROUP, dtype=torch.float32, device=dev)
    expert_ids = torch.empty(M_sum, dtype=torch.int32, device=dev)
    inv_perm = torch.empty(M, k, dtype=torch.int32, device=dev)
    _ops.moe_permute_quant_contiguous(hidden_states, topk_ids.contiguous(), local_num_experts, alignment, M_sum,
                                      a_perm, a_scale_perm, expert_ids, inv_perm, zero_padding, use_ue8m0)
    return a_perm, a_scale_perm, expert_ids, inv_perm


def _deepgemm_unpermute_and_reduce(mm2_out: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                                   inv_perm: torch.Tensor, output: torch.Tensor) -> None:
    """output[m] = sum_j topk_weights[m,j] * mm2_out[inv_perm[m,j]] in the
    output dtype (reference :119-136): products and sum in fp32, in slot
    order, rounded once to bf16."""
    if inv_perm.dtype != torch.int32:
        inv_perm = inv_perm.to(torch.int32)
    _ops.moe_unpermute_reduce(mm2_out, inv_perm.contiguous(), topk_weights.contiguous(), output)
