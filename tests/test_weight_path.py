"""Host logic of the load-time weight walk and the buffer warmup
(infra/weight_loader.py:959-1082, infra/engine.py:584-666) on the CPU:
which modules are found, buffer sizes and sharing.  No kernel runs here."""
import pytest
import torch

from tests._toy_model import ToyModel


def test_warmup_skip_allocates_buffers(monkeypatch):
    from kb_nano_amd import warmup_fp8_linear
    from kb_nano_amd.fused_experts import _SHARED_BUF
    monkeypatch.setenv("VLLM_DEEP_GEMM_WARMUP", "skip")
    model = ToyModel(torch.device("cpu"))
    n = warmup_fp8_linear(model, max_num_seqs=48, max_num_batched_tokens=1024, device=torch.device("cpu"))
    assert n == 2                                            # (768, 512) and (512, 384)
    for lin, (N, K) in ((model.qkv, (768, 512)), (model.o, (512, 384)), (model.qkv2, (768, 512))):
        op = lin.linear_op
        assert op._a_buf.shape == (48, K) and op._a_buf.dtype == torch.float8_e4m3fn
        assert op._s_buf.shape == (48, K // 128) and op._s_buf.stride() == (1, 48)
        assert op._o_buf.shape == (48, N) and op._o_buf.dtype == torch.bfloat16
        assert op._pf.a.shape == (1024, K) and op._pf.o.shape == (1024, N)
    assert model.qkv.linear_op._pf is model.qkv2.linear_op._pf
    assert model.qkv.linear_op._pf is not model.o.linear_op._pf
    # the Qwen3-style FusedExperts scratch is sized for the prefill budget
    # (top_k 2, 4 experts, 128-row alignment: M_sum = 1024*2 + 4*127 rounded up)
    assert _SHARED_BUF.a_fp8_1.shape[0] >= 1024
    M_sum = -(-(1024 * 2 + 4 * 127) // 128) * 128
    assert _SHARED_BUF.dg_ws1.numel() >= M_sum * 1280 * 2   # bf16 GEMM1 output, 2I = 1280 columns
    assert _SHARED_BUF.dg_ws2.numel() >= M_sum * 640        # fp8 SiLU*Mul output, I = 640 columns


def test_decode_batch_sizes_follow_reference():
    from kb_nano_amd.weight_path import DECODE_BATCH_SIZES
    assert DECODE_BATCH_SIZES(48) == [1, 2, 4, 8, 16, 32, 48]
    assert DECODE_BATCH_SIZES(6) == [1, 2, 4]


def test_postprocess_walk_registers_qwen3_dg_scales():
    """Qwen3-style stacks keep their scales; the _dg parameters share them.
    (The DeepSeek-style stacks and linears need the GPU kernel.)"""
    from kb_nano_amd.weight_path import postprocess_model_fp8_weights
    import torch.nn as nn
    from tests._toy_model import ToyQwen3Experts
    import numpy as np
    m = nn.Module()
    m.moe = ToyQwen3Experts(2, 256, 128, 2, np.random.default_rng(1), torch.device("cpu"))
    assert postprocess_model_fp8_weights(m) == (0, 2)
    assert m.moe.w13_scale_dg.data_ptr() == m.moe.w13_scale.data_ptr()
    assert m.moe.w2_scale_dg.data_ptr() == m.moe.w2_scale.data_ptr()
