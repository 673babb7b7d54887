"""Fused MoE experts over the sorted-token FP8 path.

Mirrors ``VllmFusedExperts`` of ``tasks/baseline/L2/vllm_fused_experts.py``
(kb_nano), DeepSeek-V3's FP8 expert path:

    1x128 quant -> moe_align_block_size (or the naive one-pair blocks)
    -> sorted-token GEMM1 (w13) -> SiLU*Mul + 1x128 quant
    -> sorted-token GEMM2 (w2, routed weights applied) -> moe_sum

Every step runs in this package's gfx950 kernels.  Intermediates are
allocated per call, as in the reference (no state shared between layers, so
graph captures hold no pointers into buffers a later call may replace).  The
reference's separate ``silu_and_mul`` and quant of the intermediate are one
fused launch here; the bf16 product between them is the same.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import _ops
from ._ops import FP8
from .fp8_linear import PerTokenGroupQuantFp8
from .moe_align import max_padded_slots
from .moe_grouped_gemm import MoeGroupedGemm, get_triton_config

_FP8_GROUP_SIZE = 128
SPARSITY_FACTOR = 4


def _moe_align_block_size_fresh(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """Freshly allocated sorted-token layout (reference :66-97)."""
    numel = topk_ids.numel()
    max_padded = max_padded_slots(numel, num_experts, block_size)
    max_blocks = -(-max_padded // block_size)
    device = topk_ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=device)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=device)
    num_tokens_post_pad = torch.empty(1, dtype=torch.int32, device=device)
    cumsum_buffer = torch.empty(num_experts + 1, dtype=torch.int32, device=device)
    _ops.moe_align_block_size(topk_ids.reshape(-1).contiguous(), num_experts, block_size, sorted_ids, expert_ids,
                              num_tokens_post_pad, cumsum_buffer)
    return sorted_ids, expert_ids, num_tokens_post_pad


class VllmFusedExperts(nn.Module):
    """``forward(hidden_states, w13, w2, topk_weights, topk_ids, num_experts,
    w13_scale, w2_scale, block_shape)`` (reference :100-237): bf16, fp16 or
    fp32 [M, K] hidden states, fp8 w13 [E, 2N, K] and w2 [E, K, N] with
    128x128 block scales, routing [M, top_k].  Returns [M, K] in the hidden
    states' dtype.  fp16 / fp32 hidden states are quantized from their own
    values (as the reference's quant widens them to fp32); the GEMM outputs,
    the SiLU*Mul product and the top-k sum stay bf16 and the sum is cast to
    the input dtype at the end, where the reference keeps those
    intermediates in the input dtype (:152-164)."""

    def __init__(self):
        super().__init__()
        self.moe_grouped_gemm = MoeGroupedGemm()
        self.per_token_group_quant_fp8 = PerTokenGroupQuantFp8()

    def forward(self, hidden_states: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, topk_weights: torch.Tensor,
                topk_ids: torch.Tensor, num_experts: int, w13_scale: torch.Tensor, w2_scale: torch.Tensor,
                block_shape: list[int]) -> torch.Tensor:
        assert hidden_states.is_contiguous(), "hidden_states must be contiguous"
        assert w13.stride(-1) == 1 and w2.stride(-1) == 1
        assert topk_weights.size() == topk_ids.size()
        assert hidden_states.dtype in (torch.bfloat16, torch.float16, torch.float32)
        M, K = hidden_states.size()
        E, N2, _ = w13.size()
        N = N2 // 2
        top_k = topk_ids.size(1)
        device = hidden_states.device
        dtype = torch.bfloat16   # the intermediates' dtype on this path

        config = get_triton_config(M, w13.shape, w2.shape, top_k, use_fp8=True, block_shape=block_shape)
        block_m = config["BLOCK_SIZE_M"]

        # one flat buffer viewed as GEMM1's and later GEMM2's output (:152-164)
        cache13 = torch.empty(M * top_k * max(N2, K), device=device, dtype=dtype)
        intermediate_cache1 = cache13[:M * top_k * N2].view(M * top_k, N2)
        intermediate_cache3 = cache13[:M * top_k * K].view(M * top_k, K)

        num_groups = math.ceil(K / _FP8_GROUP_SIZE)
        a1_fp8 = torch.empty(M, K, dtype=FP8, device=device)
        a1_scale = torch.empty(M, num_groups, dtype=torch.float32, device=device)
        self.per_token_group_quant_fp8(hidden_states, a1_fp8, a1_scale)

        naive = (M * top_k * SPARSITY_FACTOR) <= num_experts
        if naive:
            expert_ids = topk_ids.reshape(-1).to(torch.int32)
            num_tokens_post_padded = torch.full((1,), topk_ids.numel() * block_m, dtype=torch.int32, device=device)
            sorted_token_ids = None
        else:
            sorted_token_ids, expert_ids, num_tokens_post_padded = _moe_align_block_size_fresh(
                topk_ids, block_m, num_experts)

        self.moe_grouped_gemm(a1_fp8, w13, intermediate_cache1, topk_weights, sorted_token_ids, expert_ids,
                              num_tokens_post_padded, mul_routed_weight=False, top_k=top_k, config=config,
                              a_scale=a1_scale, b_scale=w13_scale, use_fp8_w8a8=True, block_shape=block_shape)

        # SiLU*Mul and the 1x128 quant of its bf16 result in one launch
        # (reference :203-219 runs silu_and_mul, then the quant)
        num_groups2 = math.ceil(N / _FP8_GROUP_SIZE)
        a2_fp8 = torch.empty(M * top_k, N, dtype=FP8, device=device)
        a2_scale = torch.empty(num_groups2, M * top_k, dtype=torch.float32, device=device).t()
        _ops.silu_mul_quant_fp8(intermediate_cache1, a2_fp8, a2_scale, use_ue8m0=True)

        self.moe_grouped_gemm(a2_fp8, w2, intermediate_cache3, topk_weights, sorted_token_ids, expert_ids,
                              num_tokens_post_padded, mul_routed_weight=True, top_k=1, config=config,
                              a_scale=a2_scale, b_scale=w2_scale, use_fp8_w8a8=True, block_shape=block_shape)

        out_hidden_states = torch.empty(M, K, device=device, dtype=dtype)
        _ops.moe_sum(intermediate_cache3.view(M, top_k, K), out_hidden_states)
        if hidden_states.dtype is not dtype:
            return out_hidden_states.to(hidden_states.dtype)
        return out_hidden_states
