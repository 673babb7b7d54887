"""MoE token-to-expert alignment with block padding (sorted-token layout).

Drop-in for ``tasks/baseline/L1/moe_align.py`` (kb_nano): ``MoeAlign`` keeps
its buffers, ``_ensure_buffers`` / ``_naive_forward`` / ``forward`` and return
values, with ``kbn_moe_align_block_size`` (one count, one scan and one
placement launch) in place of the sgl-kernel ``_C.moe_align_block_size``
(csrc/moe_align.cu).  Pairs of one expert come in (token, slot) order; the
reference's atomic placement may give any order inside an expert.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _ops


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def max_padded_slots(numel: int, num_experts: int, block_size: int) -> int:
    """The reference's sorted-token buffer size (moe_align.py:78-82)."""
    return numel * block_size if numel < num_experts else numel + num_experts * (block_size - 1)


class MoeAlign(nn.Module):
    """``forward(topk_ids, block_size, num_experts, naive=False) ->
    (sorted_token_ids | None, expert_ids, num_tokens_post_padded)``
    (reference tasks/baseline/L1/moe_align.py:17-101)."""

    def __init__(self):
        super().__init__()
        self._sorted_token_ids = None
        self._expert_ids = None
        self._num_tokens_post_padded = None
        self._cumsum_buffer = None
        self._naive_num_tokens_post_padded = None

    def _ensure_buffers(self, max_padded, max_blocks, num_experts, device):
        if self._sorted_token_ids is None or self._sorted_token_ids.size(0) < max_padded \
                or self._sorted_token_ids.device != device:
            self._sorted_token_ids = torch.empty(max_padded, dtype=torch.int32, device=device)
        if self._expert_ids is None or self._expert_ids.size(0) < max_blocks or self._expert_ids.device != device:
            self._expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=device)
        if self._num_tokens_post_padded is None or self._num_tokens_post_padded.device != device:
            self._num_tokens_post_padded = torch.zeros(1, dtype=torch.int32, device=device)
        if self._cumsum_buffer is None or self._cumsum_buffer.size(0) < num_experts + 1 \
                or self._cumsum_buffer.device != device:
            self._cumsum_buffer = torch.zeros(num_experts + 1, dtype=torch.int32, device=device)

    def _naive_forward(self, topk_ids: torch.Tensor, block_size: int):
        """One block per routed pair, no sort (reference :56-69)."""
        numel = topk_ids.numel()
        expert_ids = topk_ids.view(-1).to(torch.int32)
        if self._naive_num_tokens_post_padded is None or self._naive_num_tokens_post_padded.device != topk_ids.device:
            self._naive_num_tokens_post_padded = torch.empty(1, dtype=torch.int32, device=topk_ids.device)
        self._naive_num_tokens_post_padded.fill_(numel * block_size)
        return None, expert_ids, self._naive_num_tokens_post_padded

    def forward(self, topk_ids: torch.Tensor, block_size: int, num_experts: int, naive: bool = False):
        if naive:
            return self._naive_forward(topk_ids, block_size)
        numel = topk_ids.numel()
        max_padded = max_padded_slots(numel, num_experts, block_size)
        max_blocks = _cdiv(max_padded, block_size)
        self._ensure_buffers(max_padded, max_blocks, num_experts, topk_ids.device)
        sorted_token_ids = self._sorted_token_ids[:max_padded]
        expert_ids = self._expert_ids[:max_blocks]
        _ops.moe_align_block_size(topk_ids.reshape(-1).contiguous(), num_experts, block_size, sorted_token_ids,
                                  expert_ids, self._num_tokens_post_padded,
                                  self._cumsum_buffer[:num_experts + 1])
        return sorted_token_ids, expert_ids, self._num_tokens_post_padded
