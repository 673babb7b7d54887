"""GPU parity of the GEMM over bf16 activations (kbn_fp8_gemm_bf16a; op
kb_nano_fp8::flashinfer_blockscale_gemm, tasks/baseline/L1/fp8_linear.py:126-153,
taken by Fp8Linear.forward for small M at :398-417).

The kernel quantizes each 1x128 activation group itself.  Its output must
equal per_token_group_quant_fp8 (UE8M0) followed by fp8_gemm_nt bit for bit,
on every shape, split plan and special value, and agree with the oracle
(oracle quant + float64 GEMM) within the north-star bf16 tolerance."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, fp8_codes, seeded_bf16

pytestmark = pytest.mark.gpu


def _weights(N, K, seed, dev):
    from kb_nano_amd import synthetic
    return synthetic.dense_weight(N, K, seed=seed, device=dev)


def _quant_then_gemm(x, W, sW, eps=1e-10):
    from kb_nano_amd import _ops
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=x.device)
    s = _alloc_colmajor_scale(M, K // 128, x.device)
    _ops.per_token_group_quant_fp8(x, q, s, eps=eps, use_ue8m0=True)
    D = torch.full((M, W.shape[0]), float("nan"), dtype=torch.bfloat16, device=x.device)
    _ops.fp8_gemm_nt(q, s, W, sW, D, use_ue8m0=True)
    return D


def _fused(x, W, sW, eps=1e-10):
    from kb_nano_amd import _ops
    D = torch.full((x.shape[0], W.shape[0]), float("nan"), dtype=torch.bfloat16, device=x.device)
    _ops.fp8_gemm_bf16a(x, W, sW, D, eps=eps)
    return D


def _assert_same_bits(got, ref, what):
    g, r = got.view(torch.int16).cpu(), ref.view(torch.int16).cpu()
    n = int((g != r).sum())
    assert n == 0, f"{what}: {n} of {g.numel()} outputs differ from quant + GEMM"


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (5, 384, 1024), (8, 1000, 2048), (17, 200, 1536),
                                   (31, 640, 4096), (32, 2048, 2048), (33, 512, 8192), (48, 8192, 8192),
                                   (64, 2048, 2048), (64, 1024, 28672), (40, 4096, 7168)])
def test_bf16a_equals_quant_then_gemm(gpu_device, M, N, K):
    """Short K (data-parallel), long K (split tails summed in the split
    launch or by the separate reduction), ragged N, M across the tile."""
    x = seeded_bf16((M, K), seed=M * 7 + K, outlier_frac=1e-3).to(gpu_device)
    W, sW = _weights(N, K, seed=N + K, dev=gpu_device)
    ref = _quant_then_gemm(x, W, sW)
    got = _fused(x, W, sW)
    torch.cuda.synchronize()
    _assert_same_bits(got, ref, f"bf16a {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(3, 384, 1024), (64, 256, 2048)])
def test_bf16a_matches_oracle(gpu_device, M, N, K):
    x = seeded_bf16((M, K), seed=5 + M)
    W, sW = _weights(N, K, seed=11, dev=gpu_device)
    qa, sa = oracle.quant_group128(bf16_bits(x))
    ref = oracle.gemm_nt_sample(qa, sa, fp8_codes(W), sW.cpu().numpy())
    got = _fused(x.to(gpu_device), W, sW)
    torch.cuda.synchronize()
    assert_gemm_close(got, ref, f"bf16a {M}x{N}x{K} vs oracle")


@pytest.mark.parametrize("eps", [1e-10, 1e-36])
def test_bf16a_special_values(gpu_device, eps):
    """Groups with zeros, infinities, NaN, the largest and subnormal bf16
    values take the quant kernel's general path where it does (an infinite
    or NaN absmax; with eps = 1e-36 a zero group's scale is subnormal): the
    codes, scales and so the outputs (NaN positions included) are the same
    bits as quant + GEMM."""
    M, N, K = 24, 256, 1024
    x = seeded_bf16((M, K), seed=77)
    x[1].zero_()
    x[2, 5] = float("inf")
    x[3, 130] = float("-inf")
    x[4, 300] = float("nan")
    x[5, :128] = 3.3895e38            # bf16 max
    x[6] = 1e-40                       # bf16 subnormals
    x[7, 256:384] = 0.0                # one zero group inside a row
    x[8, 0] = float("nan")
    x[8, 1] = float("inf")             # NaN and inf in one group
    x[9, 640:768] = -7e-39
    W, sW = _weights(N, K, seed=3, dev=gpu_device)
    xd = x.to(gpu_device)
    ref = _quant_then_gemm(xd, W, sW, eps=eps)
    got = _fused(xd, W, sW, eps=eps)
    torch.cuda.synchronize()
    _assert_same_bits(got, ref, f"special values eps={eps}")


LLAMA70B = [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate_up", 57344, 8192), ("down", 8192, 28672)]


@pytest.mark.parametrize("name,N,K", LLAMA70B)
def test_bf16a_cfg5_full_size(gpu_device, name, N, K):
    """Config 5 (Llama-3.1-70B decode shapes, BASELINE recipe weights) at
    every M: bit-identical to quant + GEMM, both outputs (prefilled with NaN)
    entirely written, so a tile both paths skipped cannot pass as equal (the
    oracle comparison at every tile is test_fp8_linear_cfg5_every_tile)."""
    from kb_nano_amd import synthetic
    from tests._util import assert_all_written
    W, sW = _weights(N, K, seed=4, dev=gpu_device)
    for M in (1, 8, 32, 64):
        x = synthetic.bf16_normal((M, K), seed=40 + M).to(gpu_device)
        ref = _quant_then_gemm(x, W, sW)
        got = _fused(x, W, sW)
        torch.cuda.synchronize()
        assert_all_written(ref, f"cfg5 {name} M={M} quant + GEMM")
        assert_all_written(got, f"cfg5 {name} M={M} bf16a")
        _assert_same_bits(got, ref, f"cfg5 {name} M={M}")


def test_bf16a_op_linear_and_graph(gpu_device):
    """The reference op name runs the kernel; Fp8Linear takes it for small
    M (installed output buffer reused); graph replays (split launches with
    their arrival counters) repeat the eager bits."""
    from kb_nano_amd import Fp8Linear
    M, N, K = 16, 8192, 8192
    x = seeded_bf16((M, K), seed=123).to(gpu_device)
    W, sW = _weights(N, K, seed=9, dev=gpu_device)
    ref = _quant_then_gemm(x, W, sW)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu_device)
    torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm(x, W, sW, out)
    lin = Fp8Linear()
    y = lin(x, W, sW)
    lin._ensure_buffers(64, K, N, gpu_device)
    y2 = lin(x, W, sW)
    torch.cuda.synchronize()
    _assert_same_bits(out, ref, "op")
    _assert_same_bits(y, ref, "Fp8Linear")
    _assert_same_bits(y2, ref, "Fp8Linear, installed buffers")
    assert y2.data_ptr() == lin._o_buf.data_ptr()

    g = torch.cuda.CUDAGraph()
    gout = torch.empty(M, N, dtype=torch.bfloat16, device=gpu_device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm(x, W, sW, gout)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm(x, W, sW, gout)
    for i in range(4):
        gout.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        _assert_same_bits(gout, ref, f"graph replay {i}")
        # eager work between replays
        _fused(x, W, sW)
        torch.cuda.synchronize()


def test_bf16a_rejects_large_m(gpu_device):
    from kb_nano_amd import _ops
    x = torch.zeros(65, 256, dtype=torch.bfloat16, device=gpu_device)
    W = torch.zeros(128, 256, dtype=torch.float8_e4m3fn, device=gpu_device)
    sW = torch.ones(1, 2, device=gpu_device)
    with pytest.raises(ValueError, match="M=65"):
        _ops.fp8_gemm_bf16a(x, W, sW, torch.empty(65, 128, dtype=torch.bfloat16, device=gpu_device))


def test_bf16a_random_shapes(gpu_device):
    """24 seeded random shapes (M 1..64, ragged N, K up to 16384: data-
    parallel, split with the sum in the split launch or in the separate
    reduction), each bit-identical to quant + GEMM."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        M = int(rng.integers(1, 65))
        N = int(rng.integers(1, 4097))
        K = 128 * int(rng.integers(1, 129))
        x = seeded_bf16((M, K), seed=case, outlier_frac=1e-3).to(gpu_device)
        W, sW = _weights(N, K, seed=case + 100, dev=gpu_device)
        ref = _quant_then_gemm(x, W, sW)
        got = _fused(x, W, sW)
        torch.cuda.synchronize()
        _assert_same_bits(got, ref, f"case {case}: bf16a {M}x{N}x{K}")


def test_bf16a_op_honours_scale_contract(gpu_device, monkeypatch):
    """The registered op (reference fp8_linear.py:126-153) under the FP32
    contract (VLLM_USE_DEEP_GEMM_E8M0=0) with non-power-of-two weight scales
    uses them as given: equal bit for bit to quant (fp32 scales) + fp8_gemm_nt
    under that contract, within tolerance of the oracle with the unrounded
    scales, and not equal to the UE8M0 result.  Under UE8M0 with M = 100
    (past the fused kernel's 64 rows) it runs quant + GEMM."""
    from kb_nano_amd import _ops
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    M, N, K = 16, 1024, 2048
    x = seeded_bf16((M, K), seed=31)
    W, sW = _weights(N, K, seed=32, dev=gpu_device)
    sW = sW * 1.37
    xd = x.to(gpu_device)
    monkeypatch.setattr(_ops, "is_e8m0_used", lambda: False)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm(xd, W, sW, out)
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=gpu_device)
    s = _alloc_colmajor_scale(M, K // 128, gpu_device)
    _ops.per_token_group_quant_fp8(xd, q, s, use_ue8m0=False)
    ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    _ops.fp8_gemm_nt(q, s, W, sW, ref, use_ue8m0=False)
    torch.cuda.synchronize()
    _assert_same_bits(out, ref, "FP32 contract op")
    qa, sa = oracle.quant_group128(bf16_bits(x), use_ue8m0=False)
    assert_gemm_close(out, oracle.gemm_nt_sample(qa, sa, fp8_codes(W), sW.cpu().numpy(), ue8m0=False),
                      "FP32 contract op vs oracle")
    rounded = _fused(xd, W, sW)
    torch.cuda.synchronize()
    assert int((rounded.view(torch.int16) != out.view(torch.int16)).sum()) > N, "contract had no effect"

    monkeypatch.setattr(_ops, "is_e8m0_used", lambda: True)
    M2 = 100
    x2 = seeded_bf16((M2, K), seed=33).to(gpu_device)
    sW2 = sW / 1.37
    out2 = torch.full((M2, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm(x2, W, sW2, out2)
    ref2 = _quant_then_gemm(x2, W, sW2)
    torch.cuda.synchronize()
    _assert_same_bits(out2, ref2, "UE8M0 op at M=100")
