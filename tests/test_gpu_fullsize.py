"""GPU parity at the full sizes of BASELINE configurations 4 and 5, the shapes
the reference calls:

* config 4: the contiguous grouped GEMMs (tasks/baseline/L2/fused_experts.py:
  264-279 -> tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:112-118) with
  E = 256 experts, 4096 tokens routed top-8 by seed-0 logits (M_sum = 65,280,
  48,256 rows in expert segments), gate_up w13 [256, 4096, 7168] and down
  w2 [256, 7168, 2048], under both scale contracts, and the whole FusedExperts
  layer (fused_experts.py:246-283);
* config 5: Fp8Linear at the Llama-3.1-70B decode shapes (qkv 10240x8192,
  o 8192x8192, gate_up 57344x8192, down 8192x28672) at M in {1, 8, 32, 64}
  (tasks/baseline/L1/fp8_linear.py:398-417, :105-110).

Inputs follow the BASELINE recipe (CPU generators, seeds 3 and 4; routing
from seed 0; kb_nano_amd.synthetic).  The float64 oracle is evaluated at
sampled rows and columns: the first and last row of several expert segments,
random rows, both ends of the column range and of sampled 128-column blocks.
Tolerance: max relative error <= 1e-2, cosine >= 0.9999, atol = rtol = 1e-2.
Padding rows of the grouped GEMM's output (expert id -1) must stay unwritten
(they start as NaN) and every valid row must be written."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, fp8_codes

pytestmark = pytest.mark.gpu


def _cols(N: int, rng, n_rand: int = 64) -> np.ndarray:
    blocks = rng.choice(-(-N // 128), size=min(8, -(-N // 128)), replace=False)
    edges = np.concatenate([blocks * 128, np.minimum(blocks * 128 + 127, N - 1)])
    return np.unique(np.concatenate([[0, N - 1], edges, rng.integers(0, N, n_rand)]))


# ---------------------------------------------------------------- config 4

@pytest.fixture(scope="module")
def cfg4(gpu_device):
    from kb_nano_amd import _ops, synthetic
    from kb_nano_amd.moe_layout import _deepgemm_permute
    c = synthetic.MOE_CFG4
    dev = gpu_device
    print("cfg4: routing, hidden, permute", flush=True)
    topk_ids, topk_w = synthetic.moe_routing()
    hidden = synthetic.bf16_normal((c["T"], c["H"]), seed=3)
    a_tok = torch.empty(c["T"], c["H"], dtype=torch.float8_e4m3fn, device=dev)
    s_tok = torch.empty(c["T"], c["H"] // 128, device=dev)
    _ops.per_token_group_quant_fp8(hidden.to(dev), a_tok, s_tok)
    a_perm, s_perm, expert_ids, inv_perm = _deepgemm_permute(a_tok, s_tok, topk_ids.to(dev), c["E"], 128)
    print("cfg4: drawing w13 [256, 4096, 7168] and w2 [256, 7168, 2048]", flush=True)
    w13, s13 = synthetic.expert_weights(c["E"], c["I2"], c["H"], seed=3, device=dev)
    w2, s2 = synthetic.expert_weights(c["E"], c["H"], c["I"], seed=30, device=dev)
    torch.cuda.synchronize()
    ids = expert_ids.cpu().numpy()
    assert a_perm.shape[0] == 65280 and int(sum(ids[r] >= 0 for r in range(0, 65280, 128))) * 128 == 48256
    return dict(topk_ids=topk_ids, topk_w=topk_w, hidden=hidden, a_perm=a_perm, s_perm=s_perm,
                expert_ids=expert_ids, ids=ids, w13=w13, s13=s13, w2=w2, s2=s2)


def _segment_rows(ids: np.ndarray, rng, n_experts: int = 10) -> np.ndarray:
    """First and last valid row of sampled experts' segments (the first and
    last expert included) plus one random valid row of each."""
    present = np.unique(ids[ids >= 0])
    pick = np.unique(np.concatenate([[present[0], present[-1]], rng.choice(present, n_experts, replace=False)]))
    rows = []
    for e in pick:
        r = np.flatnonzero(ids == e)
        rows += [r[0], r[-1], rng.choice(r)]
    return np.unique(np.array(rows, dtype=np.int64))


def _check_grouped(C, A, sA, B, sB, ids, ue8m0, rng, what):
    dev = C.device
    pad = torch.from_numpy(ids < 0).to(dev)
    assert bool(torch.isnan(C[pad]).all()), f"{what}: a padding row was written"
    assert bool(torch.isfinite(C[~pad]).all()), f"{what}: a valid row was not written (or is not finite)"
    rows = _segment_rows(ids, rng)
    experts = np.unique(ids[rows])
    remap = {int(e): i for i, e in enumerate(experts)}
    et = torch.from_numpy(experts).to(dev)
    rt = torch.from_numpy(rows).to(dev)
    N = B.shape[1]
    cols = _cols(N, rng)
    qa = fp8_codes(A[rt])
    sa = sA[rt].cpu().numpy()
    sub_ids = np.array([remap[int(e)] for e in ids[rows]], dtype=np.int32)
    ref = oracle.grouped_gemm_nt_sample(qa, sa, fp8_codes(B[et]), sB[et].cpu().numpy(), sub_ids, cols=cols,
                                        ue8m0=ue8m0)
    got = C[rt][:, torch.from_numpy(cols).to(dev)]
    assert_gemm_close(got, ref, f"{what} ({len(rows)} rows of {len(experts)} experts)")


@pytest.mark.parametrize("which", ["gate_up", "down"])
@pytest.mark.parametrize("disable_ue8m0_cast", [False, True])
def test_grouped_gemm_cfg4_full_size(gpu_device, cfg4, which, disable_ue8m0_cast):
    """Both grouped GEMMs of config 4 at full size.  The FP32 contract runs
    with block scales scaled by per-block factors in [1, 1.75), so the
    accumulator rescale between K blocks is exercised, and with column-major
    activation scales (the layer's layout); the UE8M0 contract with the
    reference permute's row-major scales."""
    from kb_nano_amd import _ops, synthetic
    dev = gpu_device
    c = synthetic.MOE_CFG4
    rng = np.random.default_rng(4 + 2 * int(disable_ue8m0_cast) + (which == "down"))
    M_sum = cfg4["a_perm"].shape[0]
    if which == "gate_up":
        A, sA, B, sB = cfg4["a_perm"], cfg4["s_perm"], cfg4["w13"], cfg4["s13"]
    else:
        # GEMM2's input: a 1x128-quantized bf16 [M_sum, 2048] activation
        x = synthetic.bf16_normal((M_sum, c["I"]), seed=33).to(dev)
        A = torch.empty(M_sum, c["I"], dtype=torch.float8_e4m3fn, device=dev)
        sA = torch.empty(M_sum, c["I"] // 128, device=dev)
        _ops.per_token_group_quant_fp8(x, A, sA)
        del x
        B, sB = cfg4["w2"], cfg4["s2"]
    if disable_ue8m0_cast:
        g = torch.Generator(device=dev).manual_seed(7)
        sB = sB * (1 + 0.75 * torch.rand(sB.shape, generator=g, device=dev))
        sA = sA.t().contiguous().t()
    N = B.shape[1]
    print(f"cfg4 grouped {which} N={N} K={B.shape[2]} disable_ue8m0_cast={disable_ue8m0_cast}", flush=True)
    C = torch.full((M_sum, N), float("nan"), dtype=torch.bfloat16, device=dev)
    _ops.m_grouped_gemm_nt_contiguous(A, sA, B, sB, C, cfg4["expert_ids"], disable_ue8m0_cast)
    torch.cuda.synchronize()
    _check_grouped(C, A, sA, B, sB, cfg4["ids"], not disable_ue8m0_cast, rng,
                   f"cfg4 {which} ue8m0={not disable_ue8m0_cast}")


def _oracle_expert_tokens(hidden_bits, tokens, topk_ids, topk_w, w13, s13, w2, s2):
    """The layer's steps for the given tokens, in the oracle: 1x128 quant,
    GEMM1 against each routed expert, bf16 rounding, SiLU*Mul + quant, GEMM2,
    bf16 rounding, and the weighted top-k sum in slot order."""
    out = []
    dev = w13.device
    for m in tokens:
        qa, sa = oracle.quant_group128(hidden_bits[m:m + 1])
        es = [int(e) for e in topk_ids[m]]
        et = torch.tensor(es, device=dev)
        W13, S13 = fp8_codes(w13[et]), s13[et].cpu().numpy()
        W2, S2 = fp8_codes(w2[et]), s2[et].cpu().numpy()
        mm1 = np.concatenate([oracle.gemm_nt_sample(qa, sa, W13[j], S13[j]) for j in range(len(es))])
        q2, sq2 = oracle.silu_mul_quant(oracle.f32_to_bf16_bits(mm1.astype(np.float32)))
        mm2 = np.concatenate([oracle.gemm_nt_sample(q2[j:j + 1], sq2[j:j + 1], W2[j], S2[j]) for j in range(len(es))])
        mm2_bf16 = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(mm2.astype(np.float32)))
        inv = np.arange(len(es), dtype=np.int64)[None, :]
        out.append(oracle.unpermute_and_reduce(mm2_bf16, inv, topk_w[m:m + 1]))
    return np.concatenate(out).astype(np.float64)


def test_fused_experts_cfg4_full_size(gpu_device, cfg4):
    """FusedExperts (quant, permute, grouped GEMM1, SiLU*Mul+quant, grouped
    GEMM2, unpermute) at config 4, checked on sampled tokens against the
    oracle's composition of the same steps."""
    from kb_nano_amd.fused_experts import FusedExperts
    dev = gpu_device
    E = cfg4["w13"].shape[0]
    print("cfg4 FusedExperts layer", flush=True)
    out = FusedExperts()(cfg4["hidden"].to(dev), cfg4["w13"], cfg4["w2"], cfg4["topk_w"].to(dev),
                         cfg4["topk_ids"].to(dev), E, w13_scale=cfg4["s13"], w2_scale=cfg4["s2"],
                         use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    assert out.shape == cfg4["hidden"].shape and bool(torch.isfinite(out).all())
    tokens = np.array([0, 1234, 2977, 4095])
    ref = _oracle_expert_tokens(bf16_bits(cfg4["hidden"]), tokens, cfg4["topk_ids"].numpy(),
                                cfg4["topk_w"].numpy(), cfg4["w13"], cfg4["s13"], cfg4["w2"], cfg4["s2"])
    assert_gemm_close(out[torch.from_numpy(tokens).to(dev)], ref, "FusedExperts cfg4")
    print("cfg4 FusedExperts layer, GEMM1 to bf16 + separate SiLU*Mul+quant", flush=True)
    layer = FusedExperts()
    layer.fuse_gate_up_silu = False
    out2 = layer(cfg4["hidden"].to(dev), cfg4["w13"], cfg4["w2"], cfg4["topk_w"].to(dev), cfg4["topk_ids"].to(dev),
                 E, w13_scale=cfg4["s13"], w2_scale=cfg4["s2"], use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "fused GLU epilogue differs at config 4"
    # config 4's block scales are powers of two: the layer ran the UE8M0 kernels; the
    # FP32-contract kernels give the same bits
    from kb_nano_amd import _ops
    assert _ops.scales_are_pow2(cfg4["s13"]) and _ops.scales_are_pow2(cfg4["s2"])
    print("cfg4 FusedExperts layer, FP32-contract kernels", flush=True)
    layer = FusedExperts()
    layer.ue8m0_when_exact = False
    out3 = layer(cfg4["hidden"].to(dev), cfg4["w13"], cfg4["w2"], cfg4["topk_w"].to(dev), cfg4["topk_ids"].to(dev),
                 E, w13_scale=cfg4["s13"], w2_scale=cfg4["s2"], use_fp8_w8a8=True, block_shape=[128, 128])
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out3.view(torch.int16)), "UE8M0 kernels differ at config 4"


# ---------------------------------------------------------------- config 5

@pytest.mark.parametrize("name,N,K", [(n, N, K) for n, N, K in
                                      [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate_up", 57344, 8192),
                                       ("down", 8192, 28672)]])
def test_fp8_linear_cfg5_every_tile(gpu_device, name, N, K):
    """Config 5 at every (shape, M) through the three entry points a decode
    step can take: fp8_gemm_nt on the quantized input (with its split-K
    workspace), Fp8Linear.forward into installed buffers (quant + GEMM, or,
    where the plan prefers it, the GEMM over bf16 activations), and the
    bf16-activation GEMM itself.  Each output is prefilled with NaN and must
    come back entirely written and finite, and each is compared with oracle
    quant + oracle GEMM at a point inside every 64x64 block (every tile of
    every plan, split tails included) plus the edge rows and columns."""
    from kb_nano_amd import Fp8Linear, _ops, synthetic
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    from tests._util import assert_all_written, tile_cover
    dev = gpu_device
    print(f"cfg5 {name} N={N} K={K}: drawing the weight", flush=True)
    W, sW = synthetic.dense_weight(N, K, seed=4, device=dev)
    qw, sw = fp8_codes(W), sW.cpu().numpy()
    rng = np.random.default_rng(N + K)
    for M in (1, 8, 32, 64):
        print(f"cfg5 {name} M={M}", flush=True)
        x = synthetic.bf16_normal((M, K), seed=40 + M)
        xd = x.to(dev)
        rows, cols = tile_cover(M, N, rng)
        qa, sa = oracle.quant_group128(bf16_bits(x))
        ref = oracle.gemm_nt_sample(qa, sa, qw, sw, rows=rows, cols=cols, ue8m0=True)
        rt, ct = torch.from_numpy(rows).to(dev), torch.from_numpy(cols).to(dev)

        q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
        s = _alloc_colmajor_scale(M, K // 128, dev)
        _ops.per_token_group_quant_fp8(xd, q, s)
        D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        _ops.fp8_gemm_nt(q, s, W, sW, D, use_ue8m0=True)

        lin = Fp8Linear()
        lin._ensure_buffers(M, K, N, dev)
        lin._o_buf.fill_(float("nan"))
        y = lin(xd, W, sW)

        Dx = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        _ops.fp8_gemm_bf16a(xd, W, sW, Dx)
        torch.cuda.synchronize()
        assert y.shape == (M, N) and y.data_ptr() == lin._o_buf.data_ptr()
        for out, path in ((D, "fp8_gemm_nt"), (y, "Fp8Linear"), (Dx, "fp8_gemm_bf16a")):
            assert_all_written(out, f"cfg5 {name} M={M} {path}")
            assert_gemm_close(out[rt][:, ct], ref, f"cfg5 {name} M={M} {path} ({len(rows)} x {len(cols)} points)")
