"""GPU parity of the fused MoE experts layer (tasks/baseline/L2/fused_experts.py:
246-283) against the oracle's composition of the same steps: 1x128 quant ->
contiguous permute -> grouped GEMM1 -> SiLU*Mul + quant -> grouped GEMM2 ->
weighted unpermute.  The GEMMs are checked to the bf16 tolerance, so the
end-to-end output is too (max relative error <= 1e-2, cosine >= 0.9999)."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, from_bits, seeded_bf16, to_fp8

pytestmark = pytest.mark.gpu


def _experts(E, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    codes, scales = [], []
    for _ in range(E):
        w = (torch.randn(N, K, generator=g) * 0.02).numpy()
        q, s = oracle.quant_block128(w, use_ue8m0=False)   # checkpoint-style fp32 block scales
        codes.append(q)
        scales.append(s)
    return np.stack(codes), np.stack(scales)


def _oracle_moe(hidden_bits, topk, topk_w, w13, s13, w2, s2, E):
    M, K = hidden_bits.shape
    k = topk.shape[1]
    qa, sa = oracle.quant_group128(hidden_bits, use_ue8m0=True)
    ids, dest, M_sum = oracle.permute_contiguous(topk, E, 128)
    src = np.repeat(np.arange(M), k)
    A = np.zeros((M_sum, K), dtype=np.uint8)
    sA = np.zeros((M_sum, K // 128), dtype=np.float32)
    A[dest] = qa[src]
    sA[dest] = sa[src]
    mm1 = oracle.grouped_gemm_nt_sample(A, sA, w13, s13, ids, ue8m0=False)
    mm1[ids < 0] = 0.0                                    # padding rows: never read downstream
    mm1_bits = oracle.f32_to_bf16_bits(mm1.astype(np.float32))
    q2, sq2 = oracle.silu_mul_quant(mm1_bits, use_ue8m0=True)
    mm2 = oracle.grouped_gemm_nt_sample(q2, sq2, w2, s2, ids, ue8m0=False)
    mm2[ids < 0] = 0.0
    mm2_bf16 = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(mm2.astype(np.float32)))
    return oracle.unpermute_and_reduce(mm2_bf16, dest.reshape(M, k), topk_w).astype(np.float64)


@pytest.mark.parametrize("M,K,I,E,k", [(160, 512, 640, 8, 2), (130, 256, 768, 16, 4)])
def test_fused_experts_matches_oracle(gpu_device, M, K, I, E, k):
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    hidden = seeded_bf16((M, K), seed=M + K)
    rng = np.random.default_rng(M)
    topk = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int64)
    topk_w = rng.random((M, k)).astype(np.float32)
    topk_w /= topk_w.sum(axis=1, keepdims=True)
    w13, s13 = _experts(E, 2 * I, K, seed=1)
    w2, s2 = _experts(E, K, I, seed=2)
    ref = _oracle_moe(bf16_bits(hidden), topk, topk_w, w13, s13, w2, s2, E)

    out = FusedExperts()(from_bits(bf16_bits(hidden), dev), to_fp8(w13, dev), to_fp8(w2, dev),
                         torch.from_numpy(topk_w).to(dev), torch.from_numpy(topk).to(dev), E,
                         w13_scale=torch.from_numpy(s13).to(dev), w2_scale=torch.from_numpy(s2).to(dev),
                         use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    assert out.shape == (M, K) and out.dtype == torch.bfloat16
    assert_gemm_close(out, ref, f"FusedExperts M={M} K={K} I={I} E={E} k={k}")


def test_fused_experts_rejects_paths_it_does_not_take(gpu_device):
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    h = torch.zeros(128, 256, dtype=torch.bfloat16, device=dev)
    w13 = torch.zeros(4, 1536, 256, dtype=torch.float8_e4m3fn, device=dev)
    w2 = torch.zeros(4, 256, 768, dtype=torch.float8_e4m3fn, device=dev)
    ids = torch.zeros(128, 2, dtype=torch.int64, device=dev)
    w = torch.ones(128, 2, device=dev)
    with pytest.raises(NotImplementedError):   # BF16 experts run on the reference's Triton kernel
        FusedExperts()(h, w13, w2, w, ids, 4, use_fp8_w8a8=False)
    small = torch.zeros(4, 256, 256, dtype=torch.float8_e4m3fn, device=dev)
    with pytest.raises(NotImplementedError):   # intermediate N <= 512: outside the grouped-GEMM gate
        FusedExperts()(h, torch.zeros(4, 512, 256, dtype=torch.float8_e4m3fn, device=dev), small, w, ids, 4,
                       w13_scale=torch.ones(4, 4, 2, device=dev), w2_scale=torch.ones(4, 2, 2, device=dev),
                       use_fp8_w8a8=True)
