"""Contiguous MoE layout: aligned row count, permute, unpermute-and-reduce.

Mirrors ``tasks/baseline/L2/fused_experts.py:32-136`` (kb_nano), the layout
contract the grouped GEMM consumes.  All steps are device-side tensor ops
with fixed output shapes and no host synchronisation, so they can run inside
graph capture; they are the glue around the HIP kernels, not a kernel path.

Layout: expert e owns rows [off[e], off[e] + roundup(count[e], align)) of
the permuted activations; its ``count[e]`` tokens fill the first rows in
(token, slot) order and carry ``expert_ids = e``; the remaining rows are zero
padding with ``expert_ids = -1``.  ``inv_perm[m, j]`` is the permuted row of
token m's j-th expert.
"""
from __future__ import annotations

import torch

_GROUP = 128


def _compute_aligned_M(M: int, num_topk: int, local_num_experts: int, alignment: int) -> int:
    """M_sum = roundup(M*k + E*(align-1), align) (reference :32-39)."""
    total = M * num_topk + local_num_experts * (alignment - 1)
    return -(-total // alignment) * alignment


def _deepgemm_permute(hidden_states: torch.Tensor, a_scale: torch.Tensor, topk_ids: torch.Tensor,
                      local_num_experts: int, alignment: int):
    """Scatter (token, slot) rows into the expert-contiguous layout
    (reference :42-116).  Returns (a_perm, a_scale_perm, expert_ids, inv_perm)."""
    M, K = hidden_states.shape
    k = topk_ids.size(1)
    E = local_num_experts
    dev = hidden_states.device
    M_sum = _compute_aligned_M(M, k, E, alignment)

    flat = topk_ids.reshape(-1).to(torch.int64)
    n = flat.numel()
    counts = torch.zeros(E, dtype=torch.int64, device=dev).scatter_add_(0, flat, torch.ones_like(flat))
    seg = (counts + alignment - 1) // alignment * alignment
    offsets = torch.zeros(E + 1, dtype=torch.int64, device=dev)
    torch.cumsum(seg, 0, out=offsets[1:])

    # rank of each (token, slot) among its expert's rows, in (token, slot) order
    order = torch.argsort(flat, stable=True)
    first_sorted = torch.cumsum(counts, 0) - counts
    rank = torch.empty_like(flat)
    rank[order] = torch.arange(n, device=dev, dtype=torch.int64) - first_sorted[flat[order]]
    dest = offsets[flat] + rank

    pos = torch.arange(M_sum, device=dev, dtype=torch.int64)
    owner = (torch.searchsorted(offsets, pos, right=True) - 1).clamp_(0, E - 1)
    in_tokens = (pos - offsets[owner]) < counts[owner]
    expert_ids = torch.where(in_tokens, owner.to(torch.int32), torch.full_like(owner, -1, dtype=torch.int32))

    src = torch.arange(M, device=dev).repeat_interleave(k)
    a_perm = torch.zeros(M_sum, K, dtype=hidden_states.dtype, device=dev)
    a_scale_perm = torch.zeros(M_sum, K // _GROUP, dtype=torch.float32, device=dev)
    a_perm[dest] = hidden_states[src]
    a_scale_perm[dest] = a_scale[src]
    return a_perm, a_scale_perm, expert_ids, dest.view(M, k).to(torch.int32)


def _deepgemm_unpermute_and_reduce(mm2_out: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                                   inv_perm: torch.Tensor, output: torch.Tensor) -> None:
    """output[m] = sum_j topk_weights[m,j] * mm2_out[inv_perm[m,j]] in the
    output dtype (reference :119-136)."""
    M, H = output.shape
    k = topk_ids.size(1)
    rows = mm2_out.index_select(0, inv_perm.reshape(-1).to(torch.int64)).view(M, k, H)
    output.copy_((rows.to(output.dtype) * topk_weights.unsqueeze(-1)).sum(dim=1))
