"""A tiny model with the attribute layout kb_nano's FP8 modules have, for the
load-time and warmup tests: linear layers holding ``weight`` /
``weight_scale_inv`` and an ``Fp8Linear`` as ``linear_op``
(tasks/baseline/L1 users such as ReplicatedLinear), a DeepSeek-V3 style expert
stack (``w13_weight_scale_inv``, tasks/baseline/L2/deepseek_moe.py:101-119)
and a Qwen3-MoE style stack with a ``FusedExperts``
(tasks/baseline/L2/qwen3_moe.py:58-86, :171-182)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

import oracle


def _ckpt_weight(shape, rng):
    """fp8 codes with arbitrary (non power-of-two) fp32 block scales."""
    *lead, N, K = shape
    E = int(np.prod(lead)) if lead else 1
    q = np.empty((E, N, K), np.uint8)
    s = np.empty((E, -(-N // 128), -(-K // 128)), np.float32)
    for e in range(E):
        q[e], s[e] = oracle.quant_block128((rng.standard_normal((N, K)) * 0.03).astype(np.float32), use_ue8m0=False)
    s = (s * rng.uniform(0.5, 3.0, s.shape)).astype(np.float32)
    return q.reshape(shape), s.reshape(*lead, *s.shape[1:])


class ToyLinear(nn.Module):
    def __init__(self, N, K, rng, device):
        super().__init__()
        from kb_nano_amd import Fp8Linear
        q, s = _ckpt_weight((N, K), rng)
        self.weight = nn.Parameter(torch.from_numpy(q).view(torch.float8_e4m3fn).to(device), requires_grad=False)
        self.weight_scale_inv = nn.Parameter(torch.from_numpy(s).to(device), requires_grad=False)
        self.linear_op = Fp8Linear()

    def forward(self, x):
        return self.linear_op(x, self.weight, self.weight_scale_inv)


class ToyDeepSeekExperts(nn.Module):
    def __init__(self, E, H, I, rng, device):
        super().__init__()
        self.use_fp8 = True
        q13, s13 = _ckpt_weight((E, 2 * I, H), rng)
        q2, s2 = _ckpt_weight((E, H, I), rng)
        f8 = lambda q: nn.Parameter(torch.from_numpy(q).view(torch.float8_e4m3fn).to(device), requires_grad=False)
        f32 = lambda s: nn.Parameter(torch.from_numpy(s).to(device), requires_grad=False)
        self.w13, self.w2 = f8(q13), f8(q2)
        self.w13_weight_scale_inv, self.w2_weight_scale_inv = f32(s13), f32(s2)


class ToyQwen3Experts(nn.Module):
    def __init__(self, E, H, I, top_k, rng, device):
        super().__init__()
        from kb_nano_amd import FusedExperts
        self.use_fp8 = True
        self.num_experts, self.top_k, self.block_shape = E, top_k, [128, 128]
        q13, s13 = _ckpt_weight((E, 2 * I, H), rng)
        q2, s2 = _ckpt_weight((E, H, I), rng)
        f8 = lambda q: nn.Parameter(torch.from_numpy(q).view(torch.float8_e4m3fn).to(device), requires_grad=False)
        f32 = lambda s: nn.Parameter(torch.from_numpy(s).to(device), requires_grad=False)
        self.w13, self.w2 = f8(q13), f8(q2)
        self.w13_scale, self.w2_scale = f32(s13), f32(s2)
        self.fused_experts = FusedExperts()

    def forward(self, x, topk_weights, topk_ids):
        return self.fused_experts(x, self.w13, self.w2, topk_weights, topk_ids, self.num_experts,
                                  w13_scale=self.w13_scale, w2_scale=self.w2_scale,
                                  w13_scale_dg=getattr(self, "w13_scale_dg", None),
                                  w2_scale_dg=getattr(self, "w2_scale_dg", None),
                                  use_fp8_w8a8=True, block_shape=self.block_shape)


class ToyModel(nn.Module):
    def __init__(self, device, seed=0, H=512, E=4, I=640):
        super().__init__()
        rng = np.random.default_rng(seed)
        self.qkv = ToyLinear(768, H, rng, device)
        self.o = ToyLinear(H, 384, rng, device)
        self.qkv2 = ToyLinear(768, H, rng, device)          # same shape as qkv: shares prefill buffers
        self.ds_moe = ToyDeepSeekExperts(E, H, I, rng, device)
        self.qw_moe = ToyQwen3Experts(E, H, I, 2, rng, device)
