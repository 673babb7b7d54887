"""Synthetic inputs of the benchmark configurations, drawn on the CPU.

The recipe: values are drawn in fp32 from ``torch.Generator().manual_seed(s)``
on the CPU, scaled, cast to bf16 and copied to the GPU, so a CPU checker and
the kernels see identical bytes whatever device runs them.  Activations are
~N(0, 1); weights ~N(0, 0.02), quantized on the GPU in 128x128 blocks with
UE8M0 scales (``kbn_fp8_block_requant``).  Seeds are 0..4 for configurations
1..5; the MoE routing logits of configuration 4 come from seed 0.

Expert stacks are drawn one expert at a time, expert e from seed
``seed * 100003 + e``, on a thread pool (torch releases the GIL while it
draws), so the 11.3 G weights of configuration 4 take seconds, not minutes.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import torch

FP8 = torch.float8_e4m3fn
W_STD = 0.02

# (name, N, K) of the DeepSeek-V3 dense layers and the Llama-3.1-70B decode layers
DSV3 = [("q_b_proj", 24576, 1536), ("gate_up", 36864, 7168), ("down_proj", 7168, 18432), ("o_proj", 7168, 16384)]
LLAMA70B = [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate_up", 57344, 8192), ("down", 8192, 28672)]
# configuration 4: tokens, hidden, experts, top-k, 2 x intermediate, intermediate
MOE_CFG4 = dict(T=4096, H=7168, E=256, topk=8, I2=4096, I=2048)


def _threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def bf16_normal(shape, seed: int, std: float = 1.0, outlier_frac: float = 0.0,
                outlier_mul: float = 50.0) -> torch.Tensor:
    """CPU bf16 tensor: fp32 N(0, std) from a generator seeded `seed`; with
    `outlier_frac`, elements whose uniform draw (same generator, after the
    normals) is below it are multiplied by `outlier_mul`."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if std != 1.0:
        x = x * std
    if outlier_frac:
        x = torch.where(torch.rand(*shape, generator=g) < outlier_frac, x * outlier_mul, x)
    return x.bfloat16()


def quantize_weight(w_bf16: torch.Tensor, device) -> tuple[torch.Tensor, torch.Tensor]:
    """128x128 block quantization (UE8M0 scales) of a bf16 weight [N, K] on
    `device`: fp8 codes [N, K] and fp32 scales [ceil(N/128), ceil(K/128)]."""
    from .fp8_linear import _block_requant
    w = w_bf16.to(device, non_blocking=False).float()
    q, s = _block_requant(w, use_ue8m0=True, eps=1e-10)
    del w
    return q, s


def dense_weight(N: int, K: int, seed: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """A ~N(0, 0.02) weight [N, K] drawn on the CPU, quantized on `device`."""
    return quantize_weight(bf16_normal((N, K), seed, std=W_STD), device)


def expert_weights(E: int, N: int, K: int, seed: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """E experts of ~N(0, 0.02) weights [N, K] (expert e from seed
    seed * 100003 + e), quantized on `device` into fp8 [E, N, K] and fp32
    block scales [E, ceil(N/128), ceil(K/128)]."""
    w = torch.empty(E, N, K, dtype=FP8, device=device)
    s = torch.empty(E, -(-N // 128), -(-K // 128), device=device)

    def draw(e):
        return e, bf16_normal((N, K), seed * 100003 + e, std=W_STD)

    batch = _threads()
    with ThreadPoolExecutor(batch) as ex:
        for e0 in range(0, E, batch):
            for e, wb in ex.map(draw, range(e0, min(E, e0 + batch))):
                w[e], s[e] = quantize_weight(wb, device)
    return w, s


def moe_routing(T: int = MOE_CFG4["T"], E: int = MOE_CFG4["E"], topk: int = MOE_CFG4["topk"], seed: int = 0):
    """Top-k routing from seeded softmax logits ~N(0, 1) [T, E]: (topk_ids
    int64 [T, topk], topk_weights fp32 [T, topk], the renormalized top-k
    softmax probabilities), on the CPU."""
    g = torch.Generator().manual_seed(seed)
    probs = torch.softmax(torch.randn(T, E, generator=g), dim=-1)
    w, ids = torch.topk(probs, topk, dim=-1)
    return ids, (w / w.sum(dim=-1, keepdim=True)).float()
