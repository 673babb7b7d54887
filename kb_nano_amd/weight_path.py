"""Load-time weight path and buffer warmup around the FP8 linear operators.

Two pieces of kb_nano's engine that sit on either side of the L1 operators:

  * ``postprocess_model_fp8_weights(model)`` -- the model walk of
    ``_postprocess_fp8_weights`` (infra/weight_loader.py:1008-1082): every
    module whose ``linear_op`` is an ``Fp8Linear`` gets its weight and scale
    requantized (``postprocess_fp8_weights``); expert stacks with
    ``w13_weight_scale_inv`` / ``w2_weight_scale_inv`` (DeepSeek-V3's MoE,
    tasks/baseline/L2/deepseek_moe.py:101-119) are requantized in place, all
    experts of a tensor in one launch; stacks with ``w13_scale`` /
    ``w2_scale`` (Qwen3-MoE, tasks/baseline/L2/qwen3_moe.py:58-86) keep their
    checkpoint scales and get ``w13_scale_dg`` / ``w2_scale_dg`` parameters
    (``_postprocess_moe_fp8_weights``, :959-1005).  The reference builds
    those with DeepGEMM's ``transform_sf_into_required_layout(...,
    disable_ue8m0_cast=True)``; the grouped GEMM here reads the canonical
    fp32 ``[E, ceil(N/128), ceil(K/128)]`` scales directly, so the ``_dg``
    parameters share the checkpoint scales' storage.

  * ``warmup_fp8_linear(model, max_num_seqs, max_num_batched_tokens)`` --
    ``_warmup_deepgemm`` (infra/engine.py:584-666): decode buffers per
    ``Fp8Linear`` sized for ``max_num_seqs`` tokens, one shared
    ``_Fp8PrefillBufs`` per (N, K) sized for ``max_num_batched_tokens``, then
    one GEMM per unique shape at the reference's decode and prefill batch
    sizes.  There is no JIT here; the launches load the kernels' code object
    and let the caching allocator hold each shape's split-K workspace before a
    graph is captured.  ``VLLM_DEEP_GEMM_WARMUP=skip`` skips the launches and
    keeps the buffers, as in the reference.  ``FusedExperts`` layers (which
    run under graph capture here) also get their shared scratch buffers sized
    for ``max_num_batched_tokens``.
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn

from .fp8_linear import Fp8Linear, _Fp8PrefillBufs, postprocess_fp8_weights, postprocess_fp8_weights_batched
from .fused_experts import FusedExperts

__all__ = ["postprocess_model_fp8_weights", "warmup_fp8_linear", "DECODE_BATCH_SIZES", "PREFILL_BATCH_SIZES"]

PREFILL_BATCH_SIZES = (128, 256, 512, 1024, 2048, 4096, 8192, 16384)


def DECODE_BATCH_SIZES(max_decode: int) -> list[int]:
    """The reference's decode warmup sizes (infra/engine.py:616)."""
    return [b for b in [1, 2, 4, 8] + list(range(16, max_decode + 1, 16)) if b <= max_decode]


def _fp8_linear_modules(model: nn.Module):
    return [(m, m.linear_op) for m in model.modules() if isinstance(getattr(m, "linear_op", None), Fp8Linear)]


def _is_fp8_stack(m: nn.Module) -> bool:
    w13 = getattr(m, "w13", None)
    return isinstance(w13, torch.Tensor) and w13.dtype == torch.float8_e4m3fn and hasattr(m, "w2")


def postprocess_model_fp8_weights(model: nn.Module) -> tuple[int, int]:
    """Requantize every FP8 weight of ``model`` for the GEMMs (reference
    infra/weight_loader.py:1008-1082).  Returns (linear layers, expert weight
    slices) processed, counted as the reference counts them."""
    linear = _fp8_linear_modules(model)
    for module, _ in linear:
        w_new, s_new = postprocess_fp8_weights(module.weight.data, module.weight_scale_inv.data)
        module.weight = nn.Parameter(w_new, requires_grad=False)
        module.weight_scale_inv = nn.Parameter(s_new, requires_grad=False)

    moe_count = 0
    for module in model.modules():
        if not _is_fp8_stack(module) or not getattr(module, "use_fp8", True):
            continue
        if hasattr(module, "w13_weight_scale_inv"):          # DeepSeek-V3 style: requant in place
            for wname, sname in (("w13", "w13_weight_scale_inv"), ("w2", "w2_weight_scale_inv")):
                w = getattr(module, wname)
                postprocess_fp8_weights_batched(w.data, getattr(module, sname).data)
                moe_count += w.shape[0]
        elif getattr(module, "w13_scale", None) is not None:  # Qwen3-MoE style: scales kept, _dg views
            for sname in ("w13_scale", "w2_scale"):
                s = getattr(module, sname)
                module.register_parameter(sname + "_dg", nn.Parameter(s.data, requires_grad=False))
                moe_count += 1
    return len(linear), moe_count


def warmup_fp8_linear(model: nn.Module, max_num_seqs: int, max_num_batched_tokens: int,
                      device: torch.device | None = None) -> int:
    """Pre-allocate the FP8 linear buffers and run each weight shape once
    (reference infra/engine.py:584-666).  Returns the number of unique
    (N, K) weight shapes."""
    from . import _ops

    skip_launch = os.environ.get("VLLM_DEEP_GEMM_WARMUP", "").lower() == "skip"
    max_decode, max_prefill = int(max_num_seqs), int(max_num_batched_tokens)
    if device is None:
        p = next(model.parameters(), None)
        device = p.device if p is not None else torch.device("cuda")

    fp8_modules = _fp8_linear_modules(model)
    prefill_bufs: dict[tuple[int, int], _Fp8PrefillBufs] = {}
    seen: set[tuple[int, int]] = set()
    for module, linear_op in fp8_modules:
        w, ws = module.weight, module.weight_scale_inv
        N, K = w.shape
        linear_op._ensure_buffers(max_decode, K, N, device)
        key = (N, K)
        if key not in prefill_bufs:
            prefill_bufs[key] = _Fp8PrefillBufs(max_prefill, K, N, device)
        linear_op._pf = prefill_bufs[key]
        if skip_launch or key in seen:
            seen.add(key)
            continue
        seen.add(key)
        # the quantized activations' contents do not matter for a warmup
        # launch; zero them once so every launch reads defined values
        linear_op._a_buf.zero_()
        linear_op._s_buf.fill_(1.0)
        for m in DECODE_BATCH_SIZES(max_decode):
            _ops.fp8_gemm_nt(linear_op._a_buf[:m], linear_op._s_buf[:m], w, ws, linear_op._o_buf[:m])
        pf = prefill_bufs[key]
        pf.a.zero_()
        pf.s.fill_(1.0)
        for m in PREFILL_BATCH_SIZES:
            if max_decode < m <= max_prefill:
                _ops.fp8_gemm_nt(pf.a[:m], pf.s[:m], w, ws, pf.o[:m])

    for module in model.modules():
        fe = getattr(module, "fused_experts", None)
        if isinstance(fe, FusedExperts) and _is_fp8_stack(module):
            E, N2, K = module.w13.shape
            fe._reserve(max_prefill, K, N2, int(module.top_k), int(module.num_experts), device)

    if device.type == "cuda":
        torch.cuda.synchronize(device)
    return len(seen)
