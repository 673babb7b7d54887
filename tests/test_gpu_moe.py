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


@pytest.mark.parametrize("M,K,I,E,k", [(160, 512, 640, 8, 2), (200, 1024, 768, 16, 6)])
def test_fused_experts_glu_epilogue_equals_separate_launches(gpu_device, M, K, I, E, k):
    """GEMM1 with SiLU*Mul + quant in its epilogue gives the same layer output, bit for bit, as
    GEMM1 to bf16 followed by the separate SiLU*Mul + quant launch; so does the quant of the
    hidden states folded into the permute, against the quant launch followed by the permute."""
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    hidden = from_bits(bf16_bits(seeded_bf16((M, K), seed=M + 7)), dev)
    topk = torch.from_numpy(_routing(M, k, E, seed=M))
    topk_w = torch.from_numpy(np.random.default_rng(M + 1).random((M, k)).astype(np.float32))
    w13, s13 = _experts(E, 2 * I, K, seed=3)
    w2, s2 = _experts(E, K, I, seed=4)
    args = (hidden, to_fp8(w13, dev), to_fp8(w2, dev), topk_w.to(dev), topk.to(dev), E)
    kw = dict(w13_scale=torch.from_numpy(s13).to(dev), w2_scale=torch.from_numpy(s2).to(dev),
              use_fp8_w8a8=True, block_shape=[128, 128])
    outs = []
    for fuse, fuse_q in ((False, False), (True, False), (False, True), (True, True)):
        layer = FusedExperts()
        layer.fuse_gate_up_silu, layer.fuse_quant_permute = fuse, fuse_q
        print(f"FusedExperts M={M} I={I} E={E} k={k} fuse={fuse} fuse_quant_permute={fuse_q}", flush=True)
        outs.append(layer(*args, **kw))
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(outs[0].view(torch.int16), o.view(torch.int16))


@pytest.mark.parametrize("M,K,I,E,k", [(160, 512, 640, 8, 2), (200, 1024, 768, 16, 6)])
def test_fused_experts_ue8m0_kernels_on_power_of_two_scales(gpu_device, M, K, I, E, k):
    """With every weight block scale a power of two the layer runs the UE8M0
    GEMM kernels under the reference's FP32 contract: the output is the same,
    bit for bit, as with the FP32-contract kernels (with and without GEMM1's
    SiLU*Mul+quant epilogue), and the oracle's within tolerance.  Scales that
    are not all powers of two keep the FP32-contract kernels."""
    from kb_nano_amd import _ops
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    hb = bf16_bits(seeded_bf16((M, K), seed=M + 11))
    hidden = from_bits(hb, dev)
    topk_np = _routing(M, k, E, seed=M + 3)
    topk_w_np = np.random.default_rng(M + 5).random((M, k)).astype(np.float32)
    g = torch.Generator().manual_seed(E + K)
    def experts(N, Kd):
        codes, scales = zip(*(oracle.quant_block128((torch.randn(N, Kd, generator=g) * 0.02).numpy(),
                                                    use_ue8m0=True) for _ in range(E)))
        return np.stack(codes), np.stack(scales)
    w13, s13 = experts(2 * I, K)
    w2, s2 = experts(K, I)
    s13_d, s2_d = torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev)
    assert _ops.scales_are_pow2(s13_d) and _ops.scales_are_pow2(s2_d)
    assert not _ops.scales_are_pow2(s13_d * 1.1)
    args = (hidden, to_fp8(w13, dev), to_fp8(w2, dev), torch.from_numpy(topk_w_np).to(dev),
            torch.from_numpy(topk_np).to(dev), E)
    kw = dict(w13_scale=s13_d, w2_scale=s2_d, use_fp8_w8a8=True, block_shape=[128, 128])
    outs = []
    for exact, fuse in ((True, True), (True, False), (False, True), (False, False)):
        layer = FusedExperts()
        layer.ue8m0_when_exact, layer.fuse_gate_up_silu = exact, fuse
        print(f"FusedExperts M={M} E={E} ue8m0_when_exact={exact} fuse={fuse}", flush=True)
        outs.append(layer(*args, **kw))
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(outs[0].view(torch.int16), o.view(torch.int16))
    ref = _oracle_moe(hb, topk_np, topk_w_np, w13, s13, w2, s2, E)
    assert_gemm_close(outs[0], ref, f"FusedExperts pow2 scales M={M} E={E}")


def test_fused_experts_under_inference_mode(gpu_device):
    """Weights created and the layer called under torch.inference_mode (the
    tensors have no version counter): the same bits as outside it."""
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    M, K, I, E, k = 160, 512, 640, 8, 2
    hidden = from_bits(bf16_bits(seeded_bf16((M, K), seed=21)), dev)
    topk = torch.from_numpy(_routing(M, k, E, seed=22)).to(dev)
    topk_w = torch.from_numpy(np.random.default_rng(23).random((M, k)).astype(np.float32)).to(dev)
    g = torch.Generator().manual_seed(24)
    def experts(N, Kd):
        codes, scales = zip(*(oracle.quant_block128((torch.randn(N, Kd, generator=g) * 0.02).numpy(),
                                                    use_ue8m0=True) for _ in range(E)))
        return to_fp8(np.stack(codes), dev), torch.from_numpy(np.stack(scales)).to(dev)
    w13, s13 = experts(2 * I, K)
    w2, s2 = experts(K, I)
    kw = dict(use_fp8_w8a8=True, block_shape=[128, 128])
    ref = FusedExperts()(hidden, w13, w2, topk_w, topk, E, w13_scale=s13, w2_scale=s2, **kw)
    with torch.inference_mode():
        iw13, is13, iw2, is2 = w13.clone(), s13.clone(), w2.clone(), s2.clone()
        layer = FusedExperts()
        outs = [layer(hidden, iw13, iw2, topk_w, topk, E, w13_scale=is13, w2_scale=is2, **kw) for _ in range(2)]
    torch.cuda.synchronize()
    assert is13.is_inference()
    for o in outs:
        assert torch.equal(ref.view(torch.int16), o.view(torch.int16))


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


# ------------------------------------------------------------------ layout
# The permute and the unpermute-and-reduce kernels (fused_experts.py:42-136)
# against the oracle: the layout is index-exact, the copied rows byte-exact,
# and the reduction bit-exact (same products, fp32 sum in slot order).

def _routing(M, k, E, seed):
    rng = np.random.default_rng(seed)
    if M == 0:
        return np.zeros((0, k), dtype=np.int64)
    return np.argsort(rng.random((M, E)), axis=1)[:, :k].astype(np.int64)   # k distinct experts per token


def _rand_bytes(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, shape, dtype=torch.uint8, generator=g)


@pytest.mark.parametrize("M,k,E,align,K,ids_dtype,colmajor,ue8m0,zero_padding", [
    (200, 8, 32, 128, 7168, torch.int64, True, True, False),     # the experts layer's call
    (300, 6, 256, 128, 640, torch.int32, False, True, True),     # 5 groups: a partly idle pass
    (64, 1, 4, 128, 128, torch.int64, True, False, True),        # one group, fp32 scales
    (1, 8, 8, 128, 1024, torch.int32, False, False, False),
    (0, 4, 8, 128, 256, torch.int64, False, True, True),
    (5000, 8, 1024, 1, 384, torch.int32, True, True, False),     # most experts, no padding
])
def test_permute_quant_equals_quant_then_permute(gpu_device, M, k, E, align, K, ids_dtype, colmajor, ue8m0,
                                                  zero_padding):
    """The permute with the 1x128 quant folded in writes the same bytes as
    per_token_group_quant_fp8 followed by the permute: codes and scales of
    every routed pair's row (special values included: NaN, infinities, zero
    rows, values that round to 448), expert ids, inv_perm (dropped ids -1),
    and zeroed or untouched padding rows."""
    from kb_nano_amd import _ops
    from kb_nano_amd.moe_layout import _compute_aligned_M, _deepgemm_permute, _deepgemm_permute_quant
    dev = gpu_device
    print(f"permute+quant M={M} k={k} E={E} K={K} ue8m0={ue8m0} zero_padding={zero_padding}", flush=True)
    x = seeded_bf16((M, K), seed=M + K + k)
    if M >= 4:
        x[0, :128] = float("nan")
        x[1, 5] = float("inf")
        x[2, :] = 0.0
        x[3, 7] = 448.0 * 1.03
    topk = torch.from_numpy(_routing(M, k, E, seed=M + 1)).to(ids_dtype)
    if M >= 2:
        topk[1, 0] = -1
        topk[M - 1, k - 1] = E + 3
    xd, td = x.to(dev), topk.to(dev)
    M_sum = _compute_aligned_M(M, k, E, align)
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    sq = torch.empty(M, K // 128, device=dev)
    _ops.per_token_group_quant_fp8(xd, q, sq, use_ue8m0=ue8m0)
    ref = _deepgemm_permute(q, sq, td, E, align, zero_padding=zero_padding, scale_colmajor=colmajor)
    got = _deepgemm_permute_quant(xd, td, E, align, zero_padding=zero_padding, scale_colmajor=colmajor,
                                  use_ue8m0=ue8m0)
    torch.cuda.synchronize()
    assert got[1].stride() == ref[1].stride()
    ids = ref[2].cpu().numpy()
    assert np.array_equal(ids, got[2].cpu().numpy()) and torch.equal(ref[3], got[3])
    rows = torch.from_numpy(np.flatnonzero(ids >= 0)).to(dev)
    assert torch.equal(ref[0].view(torch.uint8)[rows], got[0].view(torch.uint8)[rows])
    assert torch.equal(ref[1][rows].view(torch.int32), got[1][rows].view(torch.int32))
    if zero_padding and M_sum > rows.numel():
        pad = torch.from_numpy(np.flatnonzero(ids < 0)).to(dev)
        assert not got[0].view(torch.uint8)[pad].any() and not got[1][pad].any()


@pytest.mark.parametrize("M,k,E,align,K,ids_dtype,colmajor", [
    (200, 8, 32, 128, 256, torch.int64, False),
    (1, 1, 1, 128, 128, torch.int32, False),
    (0, 4, 8, 128, 128, torch.int64, False),
    (300, 6, 256, 128, 7168, torch.int32, True),
    (5000, 8, 1024, 1, 128, torch.int32, False),      # most experts, no padding
    (70000, 4, 64, 16, 128, torch.int64, False),      # > 256 x 1024 pairs: 2048-pair chunks
])
def test_permute_matches_oracle(gpu_device, M, k, E, align, K, ids_dtype, colmajor):
    from kb_nano_amd.moe_layout import _deepgemm_permute
    dev = gpu_device
    print(f"permute M={M} k={k} E={E} align={align} K={K}", flush=True)
    topk = _routing(M, k, E, seed=M + E)
    ids_o, dest_o, M_sum = oracle.permute_contiguous(topk, E, align)
    x = _rand_bytes((M, K), seed=1)
    xs = torch.rand(K // 128, M).t() if colmajor else torch.rand(M, K // 128)
    a_perm, s_perm, ids, inv = _deepgemm_permute(x.to(dev).view(torch.float8_e4m3fn), xs.to(dev),
                                                 torch.from_numpy(topk).to(ids_dtype).to(dev), E, align)
    torch.cuda.synchronize()
    assert a_perm.shape == (M_sum, K) and s_perm.shape == (M_sum, K // 128)
    assert ids.dtype == torch.int32 and inv.dtype == torch.int32 and inv.shape == (M, k)
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    assert np.array_equal(inv.cpu().numpy().reshape(-1), dest_o)
    xp = a_perm.view(torch.uint8).cpu().numpy()
    sp = s_perm.cpu().numpy()
    src = np.repeat(np.arange(M), k)
    assert np.array_equal(xp[dest_o], x.numpy()[src])
    assert np.array_equal(sp[dest_o], xs.contiguous().numpy()[src])
    pad = ids_o < 0
    assert not xp[pad].any() and not sp[pad].any()       # torch.zeros padding, as in the reference


@pytest.mark.parametrize("zero_padding", [True, False])
def test_permute_column_major_scales(gpu_device, zero_padding):
    """scale_colmajor: the same values in a (1, M_sum)-strided view."""
    from kb_nano_amd.moe_layout import _deepgemm_permute
    dev = gpu_device
    M, k, E, K = 300, 8, 64, 1024
    topk = _routing(M, k, E, seed=31)
    ids_o, dest_o, M_sum = oracle.permute_contiguous(topk, E, 128)
    x = _rand_bytes((M, K), seed=5).to(dev).view(torch.float8_e4m3fn)
    xs = torch.rand(M, K // 128, device=dev)
    t = torch.from_numpy(topk).to(dev)
    ref = _deepgemm_permute(x, xs, t, E, 128)
    got = _deepgemm_permute(x, xs, t, E, 128, zero_padding=zero_padding, scale_colmajor=True)
    torch.cuda.synchronize()
    assert got[1].stride() == (1, M_sum)
    d = torch.from_numpy(dest_o).to(dev)
    assert torch.equal(got[1][d], ref[1][d]) and torch.equal(got[1][d], xs.repeat_interleave(k, 0))
    assert torch.equal(got[2], ref[2]) and torch.equal(got[3], ref[3])
    if zero_padding:
        assert torch.equal(got[1], ref[1]) and torch.equal(got[0].view(torch.uint8), ref[0].view(torch.uint8))


def test_permute_without_zero_padding_leaves_padding_rows(gpu_device):
    from kb_nano_amd import _ops
    dev = gpu_device
    M, k, E, K = 130, 4, 16, 256
    topk = _routing(M, k, E, seed=5)
    ids_o, dest_o, M_sum = oracle.permute_contiguous(topk, E, 128)
    x = _rand_bytes((M, K), seed=2).to(dev)
    xs = torch.rand(M, 2, device=dev)
    xp = torch.full((M_sum, K), 0xAB, dtype=torch.uint8, device=dev)
    sp = torch.full((M_sum, 2), -3.0, device=dev)
    ids = torch.full((M_sum,), 77, dtype=torch.int32, device=dev)
    inv = torch.empty(M, k, dtype=torch.int32, device=dev)
    _ops.moe_permute_contiguous(x, xs, torch.from_numpy(topk).to(dev), E, 128, M_sum, xp, sp, ids, inv,
                                zero_padding=False)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    pad = torch.from_numpy(ids_o < 0).to(dev)
    assert torch.all(xp[pad] == 0xAB) and torch.all(sp[pad] == -3.0)
    d = torch.from_numpy(dest_o).to(dev)
    assert torch.equal(xp[d], x.repeat_interleave(k, 0)) and torch.equal(sp[d], xs.repeat_interleave(k, 0))


def test_permute_drops_out_of_range_ids(gpu_device):
    from kb_nano_amd.moe_layout import _deepgemm_permute
    dev = gpu_device
    M, k, E, K = 64, 4, 8, 128
    topk = _routing(M, k, E, seed=9)
    topk[3, 1] = -1
    topk[10, 0] = E
    topk[11, 3] = 1 << 40                                 # would wrap to a valid id in 32 bits
    ids_o, dest_o, M_sum = oracle.permute_contiguous(topk, E, 128)
    assert (dest_o < 0).sum() == 3
    x = _rand_bytes((M, K), seed=3)
    a_perm, s_perm, ids, inv = _deepgemm_permute(x.to(dev), torch.rand(M, 1, device=dev),
                                                 torch.from_numpy(topk).to(dev), E, 128)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    assert np.array_equal(inv.cpu().numpy().reshape(-1), dest_o)
    ok = dest_o >= 0
    assert np.array_equal(a_perm.cpu().numpy()[dest_o[ok]], x.numpy()[np.repeat(np.arange(M), k)[ok]])


def _unpermute_inputs(M, k, H, rows, wdtype, seed, holes):
    g = torch.Generator().manual_seed(seed)
    y = (torch.randn(rows, H, generator=g) * 3).bfloat16()
    inv = torch.stack([torch.randperm(rows, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    if holes:   # slots outside [0, rows) contribute nothing
        inv[0, 0] = -1
        inv[M // 2, k - 1] = rows + 5
    w = torch.softmax(torch.randn(M, k, generator=g), -1).to(wdtype)
    return y, inv, w


@pytest.mark.parametrize("M,k,H,rows,wdtype", [
    (300, 8, 7168, 3000, torch.float32),
    (77, 6, 200, 500, torch.bfloat16),
    (1, 1, 8, 1, torch.float32),
    (64, 9, 1032, 900, torch.float32),       # top_k not a multiple of 4, H not of 1024
])
def test_unpermute_matches_oracle(gpu_device, M, k, H, rows, wdtype):
    from kb_nano_amd.moe_layout import _deepgemm_unpermute_and_reduce
    dev = gpu_device
    print(f"unpermute M={M} k={k} H={H} w={wdtype}", flush=True)
    y, inv, w = _unpermute_inputs(M, k, H, rows, wdtype, seed=M, holes=rows > k)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    _deepgemm_unpermute_and_reduce(y.to(dev), torch.zeros(M, k, dtype=torch.int64, device=dev), w.to(dev),
                                   inv.to(dev), out)
    torch.cuda.synchronize()
    ref = oracle.unpermute_and_reduce(oracle.bf16_bits_to_f32(bf16_bits(y)), inv.numpy(), w.float().numpy(),
                                      bf16_products=wdtype == torch.bfloat16)
    assert np.array_equal(bf16_bits(out), oracle.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
def test_unpermute_matches_reference_torch_formula(gpu_device, wdtype):
    """The reference's own torch ops (fused_experts.py:130-136) run on the GPU.
    The products are the same; torch may add them in another order, which
    moves the fp32 sum by at most top_k * 2^-24 * sum|p_j|, so the bf16
    results differ by at most one bf16 ulp plus that."""
    from kb_nano_amd.moe_layout import _deepgemm_unpermute_and_reduce
    dev = gpu_device
    M, k, H, rows = 256, 8, 2048, 4096
    y, inv, w = _unpermute_inputs(M, k, H, rows, wdtype, seed=11, holes=False)
    y, inv, w = y.to(dev), inv.to(dev), w.to(dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    _deepgemm_unpermute_and_reduce(y, None, w, inv, out)
    ref = torch.empty_like(out)
    prods = y[inv.to(torch.int64).view(-1)].view(M, k, H).to(ref.dtype) * w.unsqueeze(-1)
    ref.copy_(prods.sum(dim=1))
    mass = prods.float().abs().sum(dim=1)
    torch.cuda.synchronize()
    got, want = out.float(), ref.float()
    ulp = torch.maximum(got.abs(), want.abs()) * 2.0 ** -7
    bound = ulp + k * 2.0 ** -24 * mass
    assert torch.all((got - want).abs() <= bound)
    assert np.mean(bf16_bits(out) == bf16_bits(ref)) > 0.99


def test_layout_cfg4_full_size(gpu_device):
    """Config 4's routing (4096 tokens, top-8 of 256 experts from seeded
    softmax logits, hidden 7168): permute index- and byte-exact, unpermute
    bit-exact, at full size."""
    from kb_nano_amd.moe_layout import _deepgemm_permute, _deepgemm_unpermute_and_reduce
    dev = gpu_device
    T, H, E, k = 4096, 7168, 256, 8
    g = torch.Generator().manual_seed(0)
    topk = torch.topk(torch.softmax(torch.randn(T, E, generator=g), -1), k, dim=-1).indices
    ids_o, dest_o, M_sum = oracle.permute_contiguous(topk.numpy(), E, 128)
    assert M_sum == 65280
    x = _rand_bytes((T, H), seed=4)
    xs = torch.rand(T, H // 128, generator=g)
    a_perm, s_perm, ids, inv = _deepgemm_permute(x.to(dev).view(torch.float8_e4m3fn), xs.to(dev), topk.to(dev),
                                                 E, 128)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    assert np.array_equal(inv.cpu().numpy().reshape(-1), dest_o)
    d = torch.from_numpy(dest_o).to(dev)
    assert torch.equal(a_perm.view(torch.uint8)[d], x.to(dev).repeat_interleave(k, 0))
    assert torch.equal(s_perm[d], xs.to(dev).repeat_interleave(k, 0))
    assert not torch.any(a_perm.view(torch.uint8)[torch.from_numpy(ids_o < 0).to(dev)])
    del a_perm, s_perm
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    y = (torch.randn(M_sum, H, generator=g)).bfloat16()
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    _deepgemm_unpermute_and_reduce(y.to(dev), topk.to(dev), w.to(dev), inv, out)
    torch.cuda.synchronize()
    ref = oracle.unpermute_and_reduce(oracle.bf16_bits_to_f32(bf16_bits(y)), dest_o.reshape(T, k), w.numpy())
    assert np.array_equal(bf16_bits(out), oracle.f32_to_bf16_bits(ref))


def test_fused_experts_graph_capture(gpu_device):
    """The layer captured into a HIP graph: every replay, with eager calls on
    other data in between, reproduces the eager output bit for bit."""
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    M, K, I, E, k = 160, 512, 640, 8, 2
    rng = np.random.default_rng(3)
    w13, s13 = _experts(E, 2 * I, K, seed=1)
    w2, s2 = _experts(E, K, I, seed=2)
    w13, w2 = to_fp8(w13, dev), to_fp8(w2, dev)
    s13, s2 = torch.from_numpy(s13).to(dev), torch.from_numpy(s2).to(dev)

    def inputs(seed):
        h = from_bits(bf16_bits(seeded_bf16((M, K), seed=seed)), dev)
        ids = torch.from_numpy(_routing(M, k, E, seed)).to(dev)
        wt = torch.softmax(torch.randn(M, k, device=dev), -1)
        return h, ids, wt

    layer = FusedExperts()
    run = lambda h, ids, wt: layer(h, w13, w2, wt, ids, E, w13_scale=s13, w2_scale=s2, use_fp8_w8a8=True,
                                   block_shape=[128, 128])
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
        other = run(h2, ids2, wt2)                        # eager work reusing the shared buffers
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), f"replay {rep}"
        assert not torch.equal(other, eager)
