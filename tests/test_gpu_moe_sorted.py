"""GPU parity of the sorted-token MoE path (DeepSeek-V3's FP8 experts in
kb_nano): moe_align_block_size (tasks/baseline/L1/csrc/moe_align.cu) and
moe_sum (csrc/moe_sum.cu) bit for bit against the oracle (and moe_sum against
torch.sum, the reference's at::sum_out, for top_k > 4); the sorted-token
FP8 GEMM (tasks/baseline/L1/moe_grouped_gemm.py:86-189) and the whole
VllmFusedExperts layer (tasks/baseline/L2/vllm_fused_experts.py:100-237)
to the bf16 tolerance against the oracle's float64 composition."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, from_bits, seeded_bf16, to_fp8

pytestmark = pytest.mark.gpu


def _routing(M, k, E, seed, invalid=False):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int64)
    if invalid and M > 4:
        ids[1, 0] = -1
        ids[3, k - 1] = E
    return ids


@pytest.mark.parametrize("M,k,E,block,dtype", [(4096, 8, 256, 128, torch.int64), (64, 8, 256, 64, torch.int32),
                                               (7, 2, 64, 64, torch.int64), (300, 6, 33, 128, torch.int32),
                                               (1, 1, 4, 64, torch.int32), (2000, 4, 1024, 64, torch.int64)])
def test_moe_align_matches_oracle(gpu_device, M, k, E, block, dtype):
    from kb_nano_amd.moe_align import MoeAlign
    print(f"moe_align M={M} k={k} E={E} block={block}", flush=True)
    ids = _routing(M, k, E, seed=M + E, invalid=True)
    al = MoeAlign()
    sorted_ids, expert_ids, post = al(torch.from_numpy(ids).to(dtype).to(gpu_device), block, E)
    torch.cuda.synchronize()
    s_ref, e_ref, total, cumsum = oracle.moe_align_block_size(ids, E, block)
    assert int(post.item()) == total
    assert np.array_equal(sorted_ids.cpu().numpy(), s_ref)
    assert np.array_equal(expert_ids[:total // block].cpu().numpy(), e_ref)
    assert np.array_equal(al._cumsum_buffer[:E + 1].cpu().numpy(), cumsum)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 8, 9, 16])
@pytest.mark.parametrize("H", [7168, 100])
def test_moe_sum_matches_oracle_and_torch(gpu_device, k, H):
    from kb_nano_amd.moe_sum import MoeSum
    print(f"moe_sum k={k} H={H}", flush=True)
    M = 96
    g = torch.Generator().manual_seed(k * 100 + H)
    x = (torch.randn(M, k, H, generator=g) * torch.exp(torch.randn(M, k, 1, generator=g) * 3)).bfloat16()
    out = MoeSum()(x.view(M * k, H).to(gpu_device), k)
    torch.cuda.synchronize()
    ref = oracle.moe_sum(bf16_bits(x))
    assert np.array_equal(bf16_bits(out), ref)
    if k > 4 or k == 1:        # the reference calls at::sum_out here
        assert torch.equal(out, torch.sum(x.to(gpu_device), dim=1))


def test_moe_sum_exact_order_cases(gpu_device):
    """The oracle's order-distinguishing rows (see test_oracle) through the kernel."""
    from kb_nano_amd import _ops
    rows = [[1.0, 2.0 ** -8, 2.0 ** -8, 0.0, 0.0, 0.0, 0.0, 0.0],
            [2.0 ** 24, 1.0, 1.0, 0.0, -(2.0 ** 24), 0.0, 0.0, 0.0]]
    for k, row in ((3, rows[0][:3]), (8, rows[1])):
        x = torch.tensor(row, dtype=torch.float32).bfloat16().view(1, k, 1).expand(1, k, 8).contiguous()
        out = torch.empty(1, 8, dtype=torch.bfloat16, device=gpu_device)
        _ops.moe_sum(x.to(gpu_device), out)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), oracle.moe_sum(bf16_bits(x)))


def _experts(E, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    codes, scales = [], []
    for _ in range(E):
        w = (torch.randn(N, K, generator=g) * 0.02).numpy()
        q, s = oracle.quant_block128(w, use_ue8m0=False)   # checkpoint-style fp32 block scales
        codes.append(q)
        scales.append(s)
    return np.stack(codes), np.stack(scales)


@pytest.mark.parametrize("M,k,E,N,K,block,weighted", [(96, 8, 16, 512, 512, 128, False),
                                                      (40, 4, 8, 384, 256, 64, True),
                                                      (3, 8, 64, 256, 384, 64, True)])
def test_fused_moe_gemm_matches_oracle(gpu_device, M, k, E, N, K, block, weighted):
    """Gathered A rows, per-block experts, scattered output rows; pairs with
    invalid ids are never placed and their output rows stay untouched."""
    from kb_nano_amd import MoeGroupedGemm
    dev = gpu_device
    print(f"fused_moe_gemm M={M} k={k} E={E} N={N} K={K} block={block}", flush=True)
    ids = _routing(M, k, E, seed=M * 3 + N, invalid=True)
    a = seeded_bf16((M, K), seed=M + K)
    qa, sa = oracle.quant_group128(bf16_bits(a))
    B, sB = _experts(E, N, K, seed=E + N)
    w = np.random.default_rng(5).uniform(0.1, 1.0, (M, k)).astype(np.float32)
    s_ids, e_ids, total, _ = oracle.moe_align_block_size(ids, E, block)
    e_buf = np.full(-(-s_ids.size // block), -1, dtype=np.int32)   # the reference's buffer size; tail unused
    e_buf[:e_ids.size] = e_ids
    C = torch.full((M * k, N), 7.0, dtype=torch.bfloat16, device=dev)
    MoeGroupedGemm()(to_fp8(qa, dev), to_fp8(B, dev), C, torch.from_numpy(w).to(dev),
                     torch.from_numpy(s_ids).to(dev), torch.from_numpy(e_buf).to(dev),
                     torch.tensor([total], dtype=torch.int32, device=dev), weighted, k,
                     config={"BLOCK_SIZE_M": block}, a_scale=torch.from_numpy(sa).to(dev),
                     b_scale=torch.from_numpy(sB).to(dev), use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    ref = oracle.fused_moe_gemm_sample(qa, sa, B, sB, s_ids, e_ids, total, block, M * k, k,
                                       w if weighted else None)
    pairs = sorted(ref)
    assert_gemm_close(C[pairs], np.stack([ref[t] for t in pairs]), "sorted-token GEMM")
    unplaced = [t for t in range(M * k) if t not in ref]
    assert len(unplaced) == (2 if M > 4 else 0)
    if unplaced:
        assert bool((C[unplaced] == 7.0).all())


def test_fused_moe_gemm_dealt_tile_order(gpu_device):
    """A padded row grid large enough that whole column groups of row tiles
    are dealt to the XCDs round-robin (more than 8 groups of 16 row tiles)
    and whose tail holds row tiles no expert owns: every placed pair matches
    the oracle on sampled columns of both column tiles, incl. tile edges, and
    the two unplaceable pairs stay untouched."""
    from kb_nano_amd import MoeGroupedGemm
    dev = gpu_device
    M, k, E, N, K, block = 2048, 8, 64, 512, 256, 128
    print("fused_moe_gemm dealt tile order", flush=True)
    ids = _routing(M, k, E, seed=77, invalid=True)
    a = seeded_bf16((M, K), seed=78)
    qa, sa = oracle.quant_group128(bf16_bits(a))
    B, sB = _experts(E, N, K, seed=79)
    s_ids, e_ids, total, _ = oracle.moe_align_block_size(ids, E, block)
    padded = s_ids.size                     # rows of the padded grid (the reference's upper bound)
    assert padded // block >= 8 * 16 * 1 and total < padded - 2 * block   # dealt rounds, empty tail
    e_buf = np.full(-(-padded // block), -1, dtype=np.int32)
    e_buf[:e_ids.size] = e_ids
    C = torch.full((M * k, N), 7.0, dtype=torch.bfloat16, device=dev)
    MoeGroupedGemm()(to_fp8(qa, dev), to_fp8(B, dev), C, None,
                     torch.from_numpy(s_ids).to(dev), torch.from_numpy(e_buf).to(dev),
                     torch.tensor([total], dtype=torch.int32, device=dev), False, k,
                     config={"BLOCK_SIZE_M": block}, a_scale=torch.from_numpy(sa).to(dev),
                     b_scale=torch.from_numpy(sB).to(dev), use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    cols = np.array([0, 1, 127, 128, 200, 255, 256, 300, 383, 384, 500, 511])
    ref = oracle.fused_moe_gemm_sample(qa, sa, B, sB, s_ids, e_ids, total, block, M * k, k, cols=cols)
    pairs = sorted(ref)
    assert len(pairs) == M * k - 2
    got = C[pairs][:, torch.from_numpy(cols).to(dev)]
    assert_gemm_close(got, np.stack([ref[t] for t in pairs]), "sorted-token GEMM, dealt tiles")
    unplaced = [t for t in range(M * k) if t not in ref]
    assert bool((C[unplaced] == 7.0).all())


def test_fused_moe_gemm_naive_blocks(gpu_device):
    """No sorted list: block b holds pair b alone (the reference's naive
    assignment for very few tokens)."""
    from kb_nano_amd import MoeGroupedGemm
    dev = gpu_device
    M, k, E, N, K, block = 2, 8, 64, 512, 256, 64
    print("fused_moe_gemm naive", flush=True)
    ids = _routing(M, k, E, seed=9)
    a = seeded_bf16((M, K), seed=3)
    qa, sa = oracle.quant_group128(bf16_bits(a))
    B, sB = _experts(E, N, K, seed=4)
    C = torch.empty(M * k, N, dtype=torch.bfloat16, device=dev)
    flat = ids.reshape(-1).astype(np.int32)
    MoeGroupedGemm()(to_fp8(qa, dev), to_fp8(B, dev), C, None, None, torch.from_numpy(flat).to(dev),
                     torch.tensor([M * k * block], dtype=torch.int32, device=dev), False, k,
                     config={"BLOCK_SIZE_M": block}, a_scale=torch.from_numpy(sa).to(dev),
                     b_scale=torch.from_numpy(sB).to(dev), use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    ref = oracle.fused_moe_gemm_sample(qa, sa, B, sB, None, flat, M * k * block, block, M * k, k, naive=True)
    assert_gemm_close(C, np.stack([ref[t] for t in range(M * k)]), "naive blocks")


def _oracle_vllm_moe(hidden_bits, topk, topk_w, w13, s13, w2, s2, E, block):
    """The reference's step order (vllm_fused_experts.py:140-237) in the
    oracle: quant, align, GEMM1 -> bf16, SiLU*Mul + quant, GEMM2 * w -> bf16,
    moe_sum.  ``hidden_bits``: bf16 bit patterns, or fp16 / fp32 values
    (quantized as such; the intermediates stay bf16 as on this path)."""
    M, K = hidden_bits.shape
    k = topk.shape[1]
    if hidden_bits.dtype == np.uint16:
        qa, sa = oracle.quant_group128(hidden_bits, use_ue8m0=True)
    else:
        qa, sa = oracle.quant_group128_f32(hidden_bits, use_ue8m0=True)
    s_ids, e_ids, total, _ = oracle.moe_align_block_size(topk, E, block)
    r1 = oracle.fused_moe_gemm_sample(qa, sa, w13, s13, s_ids, e_ids, total, block, M * k, k)
    mm1 = np.stack([r1[t] for t in range(M * k)]).astype(np.float32)
    q2, sq2 = oracle.silu_mul_quant(oracle.f32_to_bf16_bits(mm1), use_ue8m0=True)
    r2 = oracle.fused_moe_gemm_sample(q2, sq2, w2, s2, s_ids, e_ids, total, block, M * k, 1, topk_w)
    mm2 = oracle.f32_to_bf16_bits(np.stack([r2[t] for t in range(M * k)]).astype(np.float32))
    return oracle.bf16_bits_to_f32(oracle.moe_sum(mm2.reshape(M, k, -1))).astype(np.float64)


@pytest.mark.parametrize("M,K,I,E,k", [(96, 512, 640, 16, 8), (2, 256, 256, 64, 8)])
def test_vllm_fused_experts_matches_oracle(gpu_device, M, K, I, E, k):
    from kb_nano_amd import VllmFusedExperts
    from kb_nano_amd.moe_grouped_gemm import get_triton_config
    dev = gpu_device
    print(f"VllmFusedExperts M={M} K={K} I={I} E={E} k={k}", flush=True)
    hidden = seeded_bf16((M, K), seed=M + K)
    topk = _routing(M, k, E, seed=M + 1)
    rng = np.random.default_rng(M)
    topk_w = rng.random((M, k)).astype(np.float32)
    topk_w /= topk_w.sum(axis=1, keepdims=True)
    w13, s13 = _experts(E, 2 * I, K, seed=1)
    w2, s2 = _experts(E, K, I, seed=2)
    block = get_triton_config(M, w13.shape, w2.shape, k, True, [128, 128])["BLOCK_SIZE_M"]
    ref = _oracle_vllm_moe(bf16_bits(hidden), topk, topk_w, w13, s13, w2, s2, E, block)
    out = VllmFusedExperts()(from_bits(bf16_bits(hidden), dev), to_fp8(w13, dev), to_fp8(w2, dev),
                             torch.from_numpy(topk_w).to(dev), torch.from_numpy(topk).to(dev), E,
                             torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev), [128, 128])
    torch.cuda.synchronize()
    assert_gemm_close(out, ref, "VllmFusedExperts")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_vllm_fused_experts_fp16_fp32_hidden(gpu_device, dtype):
    """fp16 / fp32 hidden states, which the reference accepts (:131): the
    output has the input dtype and matches the oracle's composition on the
    same values (their own quant, bf16 intermediates)."""
    from kb_nano_amd import VllmFusedExperts
    from kb_nano_amd.moe_grouped_gemm import get_triton_config
    dev = gpu_device
    M, K, I, E, k = 80, 512, 384, 16, 4
    print(f"VllmFusedExperts {dtype}", flush=True)
    hidden = torch.randn(M, K, generator=torch.Generator().manual_seed(12)).to(dtype)
    topk = _routing(M, k, E, seed=13)
    rng = np.random.default_rng(14)
    topk_w = rng.random((M, k)).astype(np.float32)
    topk_w /= topk_w.sum(axis=1, keepdims=True)
    w13, s13 = _experts(E, 2 * I, K, seed=15)
    w2, s2 = _experts(E, K, I, seed=16)
    block = get_triton_config(M, w13.shape, w2.shape, k, True, [128, 128])["BLOCK_SIZE_M"]
    ref = _oracle_vllm_moe(hidden.numpy(), topk, topk_w, w13, s13, w2, s2, E, block)
    args = (to_fp8(w13, dev), to_fp8(w2, dev), torch.from_numpy(topk_w).to(dev), torch.from_numpy(topk).to(dev), E,
            torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev), [128, 128])
    out = VllmFusedExperts()(hidden.to(dev), *args)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (M, K)
    assert_gemm_close(out, ref, f"VllmFusedExperts {dtype}")


def test_sorted_and_contiguous_layers_agree(gpu_device):
    """The two MoE layers of the reference compute the same function:
    VllmFusedExperts (sorted-token) and FusedExperts (contiguous) agree to
    the bf16 tolerance on the same routed batch."""
    from kb_nano_amd import FusedExperts, VllmFusedExperts
    dev = gpu_device
    M, K, I, E, k = 160, 512, 640, 8, 2
    print("sorted vs contiguous layer", flush=True)
    hidden = from_bits(bf16_bits(seeded_bf16((M, K), seed=4)), dev)
    topk = torch.from_numpy(_routing(M, k, E, seed=6)).to(dev)
    topk_w = torch.softmax(torch.randn(M, k, device=dev), -1)
    w13, s13 = _experts(E, 2 * I, K, seed=1)
    w2, s2 = _experts(E, K, I, seed=2)
    W13, W2, S13, S2 = to_fp8(w13, dev), to_fp8(w2, dev), torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev)
    a = VllmFusedExperts()(hidden, W13, W2, topk_w, topk, E, S13, S2, [128, 128])
    b = FusedExperts()(hidden, W13, W2, topk_w, topk, E, w13_scale=S13, w2_scale=S2, use_fp8_w8a8=True,
                       block_shape=[128, 128])
    torch.cuda.synchronize()
    assert_gemm_close(a, b.float().cpu().numpy().astype(np.float64), "sorted vs contiguous")


def test_vllm_fused_experts_graph_capture(gpu_device):
    """Captured into a HIP graph, every replay (with eager calls on other data
    in between) reproduces the eager output bit for bit."""
    from kb_nano_amd import VllmFusedExperts
    dev = gpu_device
    M, K, I, E, k = 64, 512, 640, 16, 8
    print("VllmFusedExperts graph capture", flush=True)
    w13, s13 = _experts(E, 2 * I, K, seed=1)
    w2, s2 = _experts(E, K, I, seed=2)
    W13, W2, S13, S2 = to_fp8(w13, dev), to_fp8(w2, dev), torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev)
    layer = VllmFusedExperts()

    def inputs(seed):
        h = from_bits(bf16_bits(seeded_bf16((M, K), seed=seed)), dev)
        ids = torch.from_numpy(_routing(M, k, E, seed)).to(dev)
        wt = torch.softmax(torch.randn(M, k, device=dev), -1)
        return h, ids, wt

    run = lambda h, ids, wt: layer(h, W13, W2, wt, ids, E, S13, S2, [128, 128])
    h, ids, wt = inputs(21)
    eager = run(h, ids, wt).clone()
    h2, ids2, wt2 = inputs(22)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(h, ids, wt)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = run(h, ids, wt)
    for rep in range(3):
        other = run(h2, ids2, wt2)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), f"replay {rep}"
        assert not torch.equal(other, eager)
