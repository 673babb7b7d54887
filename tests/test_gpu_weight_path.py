"""GPU tests of the load-time weight walk and the buffer warmup
(infra/weight_loader.py:959-1082, infra/engine.py:584-666) on a toy model
with kb_nano's module attribute layout: requantized weights bit-exact against
the oracle, forwards through the warmed buffers, and graph captures that
reuse them."""
import numpy as np
import pytest
import torch

import oracle
from tests._toy_model import ToyModel
from tests._util import assert_gemm_close, bf16_bits, fp8_codes

pytestmark = pytest.mark.gpu


def _snapshot(model):
    return {n: p.detach().cpu().clone() for n, p in model.named_parameters()}


def test_postprocess_model_matches_oracle(gpu_device):
    from kb_nano_amd import postprocess_model_fp8_weights
    from kb_nano_amd.fp8_linear import is_e8m0_used
    print("postprocess_model_fp8_weights toy model", flush=True)
    model = ToyModel(gpu_device, seed=1)
    before = _snapshot(model)
    n_lin, n_moe = postprocess_model_fp8_weights(model)
    torch.cuda.synchronize()
    assert (n_lin, n_moe) == (3, 2 * 4 + 2)
    ue = is_e8m0_used()
    for name in ("qkv", "o", "qkv2"):
        lin = getattr(model, name)
        q_ref, s_ref = oracle.block_requant(before[f"{name}.weight"].view(torch.uint8).numpy(),
                                            before[f"{name}.weight_scale_inv"].numpy(), use_ue8m0=ue)
        assert np.array_equal(fp8_codes(lin.weight), q_ref), name
        assert np.array_equal(lin.weight_scale_inv.cpu().numpy(), s_ref), name
    for w, s in (("w13", "w13_weight_scale_inv"), ("w2", "w2_weight_scale_inv")):
        q_ref, s_ref = oracle.block_requant(before[f"ds_moe.{w}"].view(torch.uint8).numpy(),
                                            before[f"ds_moe.{s}"].numpy(), use_ue8m0=ue)
        assert np.array_equal(fp8_codes(getattr(model.ds_moe, w)), q_ref), w
        assert np.array_equal(getattr(model.ds_moe, s).cpu().numpy(), s_ref), s
    # Qwen3-style stacks keep the checkpoint's codes and scales
    assert torch.equal(model.qw_moe.w13.cpu().view(torch.uint8), before["qw_moe.w13"].view(torch.uint8))
    assert model.qw_moe.w13_scale_dg.data_ptr() == model.qw_moe.w13_scale.data_ptr()


def test_warmup_then_forward_and_graph_capture(gpu_device):
    """After the warmup, decode-sized forwards land in the per-module buffers
    and prefill-sized ones in the shared per-shape buffers; a captured decode
    step replays bit-identically to eager with eager work in between."""
    from kb_nano_amd import postprocess_model_fp8_weights, warmup_fp8_linear
    from kb_nano_amd.fp8_linear import is_e8m0_used
    dev = gpu_device
    print("warmup_fp8_linear toy model", flush=True)
    model = ToyModel(dev, seed=2)
    postprocess_model_fp8_weights(model)
    assert warmup_fp8_linear(model, max_num_seqs=32, max_num_batched_tokens=512) == 2
    g = torch.Generator(device=dev).manual_seed(5)

    x = torch.randn(16, 512, generator=g, device=dev).bfloat16()
    y = model.qkv(x)
    assert y.data_ptr() == model.qkv.linear_op._o_buf.data_ptr()
    xp = torch.randn(300, 512, generator=g, device=dev).bfloat16()
    yp = model.qkv2(xp)
    assert yp.data_ptr() == model.qkv2.linear_op._pf.o.data_ptr() == model.qkv.linear_op._pf.o.data_ptr()
    qa, sa = oracle.quant_group128(bf16_bits(xp))
    ref = oracle.gemm_nt_sample(qa, sa, fp8_codes(model.qkv2.weight), model.qkv2.weight_scale_inv.cpu().numpy(),
                                ue8m0=is_e8m0_used())
    assert_gemm_close(yp, ref, "prefill through the shared buffers")

    step = lambda inp: model.o(model.qkv(inp)[:, :384])
    eager = step(x).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = step(x)
    x2 = torch.randn(16, 512, generator=g, device=dev).bfloat16()
    for rep in range(3):
        other = step(x2).clone()                        # eager work on the same buffers
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), f"replay {rep}"
        assert not torch.equal(other, eager)


def test_warmup_reserves_fused_experts_scratch(gpu_device):
    """The warmup sizes FusedExperts' shared scratch for the prefill budget,
    so a later call and a capture reuse it instead of growing it."""
    from kb_nano_amd import postprocess_model_fp8_weights, warmup_fp8_linear
    from kb_nano_amd.fused_experts import _SHARED_BUF
    dev = gpu_device
    print("warmup FusedExperts reservation", flush=True)
    model = ToyModel(dev, seed=3)
    postprocess_model_fp8_weights(model)
    warmup_fp8_linear(model, max_num_seqs=32, max_num_batched_tokens=512)
    ptrs = [t.data_ptr() for t in (_SHARED_BUF.a_fp8_1, _SHARED_BUF.dg_ws1, _SHARED_BUF.dg_ws2)]
    M = 500
    g = torch.Generator(device=dev).manual_seed(7)
    h = torch.randn(M, 512, generator=g, device=dev).bfloat16()
    ids = torch.stack([torch.randperm(4, generator=g, device=dev)[:2] for _ in range(M)]).to(torch.int32)
    wt = torch.softmax(torch.randn(M, 2, generator=g, device=dev), -1)
    out = model.qw_moe(h, wt, ids)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert [t.data_ptr() for t in (_SHARED_BUF.a_fp8_1, _SHARED_BUF.dg_ws1, _SHARED_BUF.dg_ws2)] == ptrs
