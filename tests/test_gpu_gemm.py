"""GPU parity of the block-scaled FP8 GEMMs against the float64 oracle
(tasks/baseline/L1/fp8_linear.py:89-118, :335-450;
tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:100-170).

Tolerance (north star): max relative error <= 1e-2, cosine >= 0.9999, and
elementwise atol = rtol = 1e-2 against the dequantize-then-matmul oracle."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, fp8_codes, quantized_gemm_inputs, seeded_bf16, to_fp8

pytestmark = pytest.mark.gpu


def _gemm_gpu(qa, sa, qw, sw, dev, ue8m0=True, col_major=True):
    from kb_nano_amd import _ops
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    M, K = qa.shape
    N = qw.shape[0]
    A = to_fp8(qa, dev)
    if col_major:
        sA = _alloc_colmajor_scale(M, K // 128, dev)
        sA.copy_(torch.from_numpy(sa))
    else:
        sA = torch.from_numpy(sa).to(dev)
    W = to_fp8(qw, dev)
    sW = torch.from_numpy(sw).to(dev)
    D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    _ops.fp8_gemm_nt(A, sA, W, sW, D, use_ue8m0=ue8m0)
    torch.cuda.synchronize()
    return D


@pytest.mark.parametrize("M,N,K", [(64, 2048, 2048), (1, 256, 128), (3, 384, 1024), (65, 640, 1536),
                                   (130, 256, 2048), (300, 512, 1024), (512, 768, 4096)])
@pytest.mark.parametrize("ue8m0", [True, False])
def test_gemm_matches_oracle(gpu_device, M, N, K, ue8m0):
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + N + K)
    if not ue8m0:
        # non power-of-two weight scales exercise the fp32 promotion path
        sw = (sw * np.float32(1.37)).astype(np.float32)
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=ue8m0)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=ue8m0)
    assert_gemm_close(D, ref, f"gemm {M}x{N}x{K} ue8m0={ue8m0}")


def test_gemm_row_major_scales_and_ragged_n(gpu_device):
    M, N, K = 77, 200, 512
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=9)
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, col_major=False)
    assert_gemm_close(D, ref, "ragged N")


def test_gemm_ue8m0_contract_rounds_scales(gpu_device):
    """Under the UE8M0 contract a non power-of-two scale acts as the next
    power of two up (the oracle's ue8m0 mode)."""
    M, N, K = 64, 256, 512
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=4)
    sw = (sw * np.float32(1.37)).astype(np.float32)
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=True)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=True)
    assert_gemm_close(D, ref, "ue8m0 cast")


def test_gemm_single_k_block_special_case(gpu_device):
    """Only K block 1 is non-zero: the output must carry that block's scales
    (a wrong scale index or K-block offset fails this)."""
    M, N, K = 64, 256, 384
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=12)
    qa[:, :128] = 0
    qa[:, 256:] = 0
    sa[:, 1] *= 8
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device)
    assert_gemm_close(D, ref, "single K block")


@pytest.mark.parametrize("name,N,K", [("q_b_proj", 24576, 1536), ("gate_up", 36864, 7168),
                                      ("down_proj", 7168, 18432), ("o_proj", 7168, 16384)])
@pytest.mark.parametrize("M", [128, 4096])
def test_gemm_dsv3_every_tile(gpu_device, name, N, K, M):
    """BASELINE config 3 at full size, inputs drawn on the CPU by the BASELINE
    recipe (seed 2 for the weights, 20 for the activations).  The output is
    prefilled with NaN and must come back entirely written and finite; the
    oracle is evaluated on a row set x column set that puts a point inside
    every 64x64 block of the output (so inside every tile of every plan,
    split-tail tiles included) plus the first and last rows and columns of
    the edge tiles."""
    from kb_nano_amd import _ops, synthetic
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    from tests._util import assert_all_written, tile_cover
    print(f"cfg3 {name} M={M}", flush=True)
    a = synthetic.bf16_normal((M, K), seed=20).to(gpu_device)
    A = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=gpu_device)
    sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
    _ops.per_token_group_quant_fp8(a, A, sA)
    W, sW = synthetic.dense_weight(N, K, seed=2, device=gpu_device)
    D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    _ops.fp8_gemm_nt(A, sA, W, sW, D, use_ue8m0=True)
    torch.cuda.synchronize()
    assert_all_written(D, f"{name} M={M}")
    rows, cols = tile_cover(M, N, np.random.default_rng(M + N))
    qa = fp8_codes(A[torch.from_numpy(rows).to(gpu_device)])
    sa = sA[torch.from_numpy(rows).to(gpu_device)].cpu().numpy()
    qw = fp8_codes(W)
    ref = oracle.gemm_nt_sample(qa, sa, qw, sW.cpu().numpy(), cols=cols)
    got = D[torch.from_numpy(rows).to(gpu_device)][:, torch.from_numpy(cols).to(gpu_device)]
    assert_gemm_close(got, ref, f"{name} M={M} ({len(rows)} x {len(cols)} points)")


@pytest.mark.parametrize("M,N,K", [(1, 7168, 18432), (8, 8192, 8192), (64, 1024, 28672), (100, 7168, 16384),
                                   (77, 203, 65536), (256, 768, 32768), (200, 2048, 16384)])
@pytest.mark.parametrize("ue8m0", [True, False])
def test_gemm_split_tail_matches_data_parallel(gpu_device, M, N, K, ue8m0):
    """Split-K tail (the partly empty last wave of tiles split over K into
    fp32 workspace slabs + ordered reduction) against the oracle and against
    the data-parallel kernel (kbn_fp8_gemm_nt, no workspace): both within
    tolerance, and equal up to fp32 summation order."""
    import ctypes

    from kb_nano_amd._lib import lib
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    L = lib()
    ws = L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, int(ue8m0))
    assert ws > 0, "shape expected to split its tail"
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=N + K)
    if not ue8m0:
        sw = (sw * np.float32(1.37)).astype(np.float32)
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(K).integers(0, N, 94)]))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=ue8m0, cols=cols)
    A = to_fp8(qa, gpu_device)
    sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
    sA.copy_(torch.from_numpy(sa))
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    outs = []
    for split in (False, True):
        D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        buf = torch.empty(ws, dtype=torch.uint8, device=gpu_device) if split else None
        rc = L.kbn_fp8_gemm_nt_ws(A.data_ptr(), K, sA.data_ptr(), 1, M, W.data_ptr(), K, sW.data_ptr(), K // 128,
                                  D.data_ptr(), N, M, N, K, int(ue8m0),
                                  ctypes.c_void_p(buf.data_ptr()) if split else None, ws if split else 0,
                                  torch.cuda.current_stream().cuda_stream)
        assert rc == 0, L.kbn_last_error()
        torch.cuda.synchronize()
        assert_gemm_close(D[:, torch.from_numpy(cols).to(gpu_device)], ref, f"split={split} {M}x{N}x{K}")
        outs.append(D.float())
    diff = (outs[0] - outs[1]).abs()
    assert torch.all(diff <= 1e-2 * outs[0].abs() + 1e-3), float(diff.max())


def test_gemm_cfg1_golden_fixture(gpu_device):
    """BASELINE config 1 (M=64, N=K=2048, seed 0) against the committed
    oracle slice (tests/golden/gemm_cfg1.npz), within the bf16 tolerance."""
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemm_cfg1.npz"), allow_pickle=False)
    M, N, K = int(d["M"]), int(d["N"]), int(d["K"])
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=int(d["seed"]))
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device)
    assert_gemm_close(D[:16, :64], d["out_slice"], "cfg1 golden slice")


# ------------------------------------------------------------- Fp8Linear

def test_fp8_linear_end_to_end(gpu_device):
    """Fp8Linear.forward = quant (UE8M0, column-major) + block-scaled GEMM,
    checked against oracle quant + oracle GEMM; with buffers installed the
    output is a view of the reused buffer (reference :419-450)."""
    from kb_nano_amd import Fp8Linear
    M, N, K = 48, 384, 1024
    x = seeded_bf16((2, M // 2, K), seed=31)
    _, _, qw, sw = quantized_gemm_inputs(M, N, K, seed=31)
    qa, sa = oracle.quant_group128(bf16_bits(x.reshape(M, K)))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
    lin = Fp8Linear()
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    y = lin(x.to(gpu_device), W, sW)
    torch.cuda.synchronize()
    assert y.shape == (2, M // 2, N) and y.dtype == torch.bfloat16
    assert_gemm_close(y.reshape(M, N), ref, "Fp8Linear")
    lin._ensure_buffers(128, K, N, gpu_device)
    y2 = lin(x.to(gpu_device), W, sW)
    torch.cuda.synchronize()
    assert y2.data_ptr() == lin._o_buf.data_ptr()
    assert torch.equal(y2, y)
    bias = torch.randn(N, device=gpu_device).bfloat16()
    y3 = lin(x.to(gpu_device), W, sW, bias)
    torch.cuda.synchronize()
    assert torch.equal(y3, (y + bias))


def test_fp8_linear_decode_sizes(gpu_device):
    from kb_nano_amd import Fp8Linear
    N, K = 512, 2048
    _, _, qw, sw = quantized_gemm_inputs(8, N, K, seed=5)
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    for M in (1, 8, 32, 64):
        x = seeded_bf16((M, K), seed=M)
        qa, sa = oracle.quant_group128(bf16_bits(x))
        ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
        y = Fp8Linear()(x.to(gpu_device), W, sW)
        torch.cuda.synchronize()
        assert_gemm_close(y, ref, f"decode M={M}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fp8_linear_fp16_fp32_input(gpu_device, dtype):
    """fp16 / fp32 activations, which the reference's Fp8Linear quantizes as
    well (its quant widens them to fp32; only its bf16 FlashInfer branch
    needs bf16): the quant of the values themselves, then the GEMM, bf16
    out; every M path (decode sizes that take the bf16-input GEMM for bf16,
    installed buffers, prefill) against the oracle's float-input quant and
    GEMM, and bit-identical to the two ops called in turn."""
    from kb_nano_amd import Fp8Linear, _ops
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    N, K = 512, 2048
    _, _, qw, sw = quantized_gemm_inputs(8, N, K, seed=7)
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    for M, installed in ((1, False), (32, False), (64, True), (200, False)):
        print(f"Fp8Linear {dtype} M={M} installed={installed}", flush=True)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(dtype)
        qa, sa = oracle.quant_group128_f32(x.numpy())
        ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
        lin = Fp8Linear()
        if installed:
            lin._ensure_buffers(128, K, N, gpu_device)
        y = lin(x.to(gpu_device), W, sW)
        q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=gpu_device)
        s = _alloc_colmajor_scale(M, K // 128, gpu_device)
        _ops.per_token_group_quant_fp8(x.to(gpu_device), q, s)
        y2 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu_device)
        _ops.fp8_gemm_nt(q, s, W, sW, y2)
        torch.cuda.synchronize()
        assert y.dtype == torch.bfloat16 and y.shape == (M, N)
        assert np.array_equal(fp8_codes(q), qa)
        assert_gemm_close(y, ref, f"Fp8Linear {dtype} M={M}")
        assert torch.equal(y, y2)


def test_postprocess_weights_roundtrip(gpu_device):
    """Requant of UE8M0 block weights is value-preserving."""
    from kb_nano_amd import postprocess_fp8_weights
    _, _, qw, sw = quantized_gemm_inputs(8, 384, 512, seed=8)
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    W2, sW2 = postprocess_fp8_weights(W, sW)
    deq = lambda w, s: w.float() * s.repeat_interleave(128, 0)[:w.shape[0]].repeat_interleave(128, 1)[:, :w.shape[1]]
    assert torch.equal(deq(W2, sW2), deq(W, sW))


# ---------------------------------------------------------------- grouped

def _grouped_case(E, N, K, M_tok, topk, seed, dev, col_major_a=False):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((M_tok, E))
    topk_ids = np.argsort(-logits, axis=1)[:, :topk]
    ids, dest, M_sum = oracle.permute_contiguous(topk_ids, E, 128)
    a = seeded_bf16((M_tok, K), seed=seed)
    qa_tok, sa_tok = oracle.quant_group128(bf16_bits(a))
    src = np.repeat(np.arange(M_tok), topk)
    qa = np.zeros((M_sum, K), dtype=np.uint8)
    sa = np.zeros((M_sum, K // 128), dtype=np.float32)
    qa[dest] = qa_tok[src]
    sa[dest] = sa_tok[src]
    g = torch.Generator().manual_seed(seed + 1)
    qb = np.empty((E, N, K), dtype=np.uint8)
    sb = np.empty((E, -(-N // 128), K // 128), dtype=np.float32)
    for e in range(E):
        qb[e], sb[e] = oracle.quant_block128((torch.randn(N, K, generator=g) * 0.02).numpy())
    return ids, qa, sa, qb, sb, M_sum


@pytest.mark.parametrize("ue8m0", [True, False])
def test_grouped_gemm_matches_oracle(gpu_device, ue8m0):
    from kb_nano_amd import Fp8GroupedGemmContiguous
    from kb_nano_amd import _ops
    E, N, K = 6, 384, 1024
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N, K, M_tok=96, topk=2, seed=3, dev=gpu_device)
    if not ue8m0:
        sb = (sb * np.float32(0.83)).astype(np.float32)
    dev = gpu_device
    C = torch.full((M_sum, N), 7.0, dtype=torch.bfloat16, device=dev)
    A, sA = to_fp8(qa, dev), torch.from_numpy(sa).to(dev)
    B, sB = to_fp8(qb, dev), torch.from_numpy(sb).to(dev)
    idt = torch.from_numpy(ids).to(dev)
    _ops.m_grouped_gemm_nt_contiguous(A, sA, B, sB, C, idt, disable_ue8m0_cast=not ue8m0)
    torch.cuda.synchronize()
    ref = oracle.grouped_gemm_nt_sample(qa, sa, qb, sb, ids, ue8m0=ue8m0)
    valid = ids >= 0
    assert_gemm_close(C[torch.from_numpy(valid).to(dev)], ref[valid], f"grouped ue8m0={ue8m0}")
    assert torch.all(C[torch.from_numpy(~valid).to(dev)] == 7.0), "padding rows must stay unwritten"
    # the module wrapper and the free function reach the same kernel
    C2 = torch.full_like(C, 7.0)
    Fp8GroupedGemmContiguous()(A, sA, B, sB, C2, idt)
    torch.cuda.synchronize()
    assert Fp8GroupedGemmContiguous().alignment() == 128
    if ue8m0:
        assert torch.equal(C2, C)


def test_grouped_gemm_free_function_colmajor_scales(gpu_device):
    """moe_grouped_gemm.py:71-83 path (disable_ue8m0_cast=True) with the
    column-major A scales SiluMulQuantFp8 produces."""
    from kb_nano_amd import m_grouped_fp8_gemm_nt_contiguous
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    E, N, K = 4, 256, 512
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N, K, M_tok=64, topk=2, seed=8, dev=gpu_device)
    dev = gpu_device
    sA = _alloc_colmajor_scale(M_sum, K // 128, dev)
    sA.copy_(torch.from_numpy(sa))
    C = torch.zeros((M_sum, N), dtype=torch.bfloat16, device=dev)
    m_grouped_fp8_gemm_nt_contiguous((to_fp8(qa, dev), sA), (to_fp8(qb, dev), torch.from_numpy(sb).to(dev)),
                                     C, torch.from_numpy(ids).to(dev))
    torch.cuda.synchronize()
    ref = oracle.grouped_gemm_nt_sample(qa, sa, qb, sb, ids)
    valid = ids >= 0
    assert_gemm_close(C[torch.from_numpy(valid).to(dev)], ref[valid], "grouped free fn")


@pytest.mark.parametrize("K", [1024, 2560])
@pytest.mark.parametrize("ue8m0", [True, False])
def test_grouped_gemm_padding_garbage_is_isolated(gpu_device, K, ue8m0):
    """Padding rows (id -1) may hold anything: FusedExperts leaves them
    unwritten.  NaN codes and infinite or NaN scales there change no bit of
    the output, whether the kernel reads those rows as zeros (K <= 2048) or
    fetches them (longer K); padding output rows stay unwritten."""
    from kb_nano_amd import _ops
    E, N = 5, 256
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N, K, M_tok=80, topk=2, seed=21, dev=gpu_device)
    dev = gpu_device
    pad = ids < 0
    assert pad.any()
    qa2, sa2 = qa.copy(), sa.copy()
    qa2[pad] = 0x7F                       # e4m3 NaN
    sa2[pad] = np.float32(np.inf)
    sa2[np.ix_(pad, np.arange(0, K // 128, 2))] = np.float32(np.nan)
    B, sB, idt = to_fp8(qb, dev), torch.from_numpy(sb).to(dev), torch.from_numpy(ids).to(dev)
    outs = []
    for q_, s_ in ((qa, sa), (qa2, sa2)):
        C = torch.full((M_sum, N), 7.0, dtype=torch.bfloat16, device=dev)
        _ops.m_grouped_gemm_nt_contiguous(to_fp8(q_, dev), torch.from_numpy(s_).to(dev), B, sB, C, idt,
                                          disable_ue8m0_cast=not ue8m0)
        outs.append(C)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.all(outs[1][torch.from_numpy(pad).to(dev)] == 7.0)


@pytest.mark.parametrize("E,N2,K,M_tok,topk", [(6, 512, 1024, 96, 2), (5, 768, 2560, 80, 2), (8, 4096, 7168, 64, 8)])
@pytest.mark.parametrize("ue8m0", [True, False])
def test_grouped_gemm_silu_quant_equals_two_launches(gpu_device, E, N2, K, M_tok, topk, ue8m0):
    """GEMM1 with SiLU*Mul + 1x128 quant in its epilogue writes exactly the
    codes and scales of the grouped GEMM into a bf16 buffer followed by the
    row-skipping SiLU*Mul+quant kernel (both scale contracts of the GEMM,
    UE8M0 and FP32 quant scales, column-major and row-major scale layouts),
    leaves rows with id -1 untouched, and its output also matches the oracle's
    SiLU*Mul+quant of the oracle's GEMM to the bf16 GEMM tolerance."""
    from kb_nano_amd import _ops
    print(f"gemm+silu {E}x{N2}x{K} tokens={M_tok} top{topk} ue8m0={ue8m0}", flush=True)
    dev = gpu_device
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N2, K, M_tok=M_tok, topk=topk, seed=N2 + K, dev=dev)
    if not ue8m0:
        sb = (sb * np.float32(1.37)).astype(np.float32)
    A, sA = to_fp8(qa, dev), torch.from_numpy(sa).to(dev)
    B, sB, idt = to_fp8(qb, dev), torch.from_numpy(sb).to(dev), torch.from_numpy(ids).to(dev)
    N = N2 // 2
    valid = torch.from_numpy(ids >= 0).to(dev)
    for q_ue8m0 in (False, True):      # the last run (UE8M0) is checked against the oracle below
        for col_major in (False, True):
            C = torch.empty((M_sum, N2), dtype=torch.bfloat16, device=dev)
            _ops.m_grouped_gemm_nt_contiguous(A, sA, B, sB, C, idt, disable_ue8m0_cast=not ue8m0)
            q1 = torch.full((M_sum, N), 0x5A, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
            shape, strides = (M_sum, N // 128), ((1, M_sum) if col_major else (N // 128, 1))
            s1 = torch.empty_strided(shape, strides, device=dev).fill_(-3.0)
            _ops.silu_mul_quant_fp8(C, q1, s1, q_ue8m0, 1e-10, row_ids=idt)
            q2 = torch.full_like(q1.view(torch.uint8), 0x5A).view(torch.float8_e4m3fn)
            s2 = torch.empty_strided(shape, strides, device=dev).fill_(-3.0)
            _ops.grouped_gemm_silu_quant(A, sA, B, sB, idt, not ue8m0, q2, s2, q_ue8m0, 1e-10)
            torch.cuda.synchronize()
            assert torch.equal(q2.view(torch.uint8), q1.view(torch.uint8)), (q_ue8m0, col_major)
            assert torch.equal(s2, s1), (q_ue8m0, col_major)
            assert torch.all(q2.view(torch.uint8)[~valid] == 0x5A) and torch.all(s2[~valid] == -3.0)
    # against the oracle: SiLU*Mul+quant of the oracle GEMM, dequantized
    ref_h = oracle.grouped_gemm_nt_sample(qa, sa, qb, sb, ids, ue8m0=ue8m0)
    v = ids >= 0
    hb = oracle.f32_to_bf16_bits(ref_h[v].astype(np.float32))
    qo, so = oracle.silu_mul_quant(hb, use_ue8m0=True)
    deq = lambda c, sc: oracle.e4m3_decode(c).astype(np.float64) * np.repeat(sc, 128, axis=1)
    got = deq(fp8_codes(q2[valid]), s2[valid].cpu().numpy())
    ref = deq(qo, so)
    # codes may differ by one e4m3 step where the bf16 GEMM rows differ in the last bit
    err = np.abs(got - ref).mean() / np.abs(ref).mean()
    cos = (got * ref).sum() / np.sqrt((got * got).sum() * (ref * ref).sum())
    assert err < 0.02 and cos > 0.999, (err, cos)


@pytest.mark.parametrize("K", [1024, 2560])
@pytest.mark.parametrize("ue8m0", [True, False])
def test_grouped_gemm_segment_end_fragments(gpu_device, K, ue8m0):
    """Blocks holding 1, 32, 33, 64, 65, 96, 97, 128 and 20 rows of their
    expert, and one with a hole (rows 64-95 id -1 between live rows): each
    wavefront of a 128-row tile skips the 32-row fragments past its last live
    row, so every case of 0, 1 or 2 live fragments per wavefront and both
    sides of each 32-row boundary occur.  Padding rows hold random codes and
    scales.  The plain kernel matches the oracle on every live row, the
    kernel with the SiLU*Mul+quant epilogue equals the two launches bit for
    bit, and no padding row is written."""
    from kb_nano_amd import _ops
    dev = gpu_device
    print(f"grouped segment ends K={K} ue8m0={ue8m0}", flush=True)
    E, N2 = 3, 512
    counts = [1, 32, 33, 64, 65, 96, 97, 128, 20, 128]
    ids = np.full(128 * len(counts), -1, dtype=np.int32)
    for b, c in enumerate(counts):
        ids[128 * b: 128 * b + c] = b % E
    ids[128 * 9 + 64: 128 * 9 + 96] = -1                     # the hole
    M_sum = ids.size
    a = seeded_bf16((M_sum, K), seed=K + 3)
    qa, sa = oracle.quant_group128(bf16_bits(a))
    g = torch.Generator().manual_seed(K)
    qb = np.empty((E, N2, K), dtype=np.uint8)
    sb = np.empty((E, N2 // 128, K // 128), dtype=np.float32)
    for e in range(E):
        qb[e], sb[e] = oracle.quant_block128((torch.randn(N2, K, generator=g) * 0.02).numpy())
    if not ue8m0:
        sb = (sb * np.float32(1.37)).astype(np.float32)
    A, sA = to_fp8(qa, dev), torch.from_numpy(sa).to(dev)
    B, sB, idt = to_fp8(qb, dev), torch.from_numpy(sb).to(dev), torch.from_numpy(ids).to(dev)
    valid = ids >= 0
    vt = torch.from_numpy(valid).to(dev)
    C = torch.full((M_sum, N2), 7.0, dtype=torch.bfloat16, device=dev)
    _ops.m_grouped_gemm_nt_contiguous(A, sA, B, sB, C, idt, disable_ue8m0_cast=not ue8m0)
    N = N2 // 2
    q1 = torch.full((M_sum, N), 0x5A, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    s1 = torch.empty_strided((M_sum, N // 128), (1, M_sum), device=dev).fill_(-3.0)
    _ops.silu_mul_quant_fp8(C, q1, s1, True, 1e-10, row_ids=idt)
    q2 = torch.full_like(q1.view(torch.uint8), 0x5A).view(torch.float8_e4m3fn)
    s2 = torch.empty_strided((M_sum, N // 128), (1, M_sum), device=dev).fill_(-3.0)
    _ops.grouped_gemm_silu_quant(A, sA, B, sB, idt, not ue8m0, q2, s2, True, 1e-10)
    torch.cuda.synchronize()
    ref = oracle.grouped_gemm_nt_sample(qa, sa, qb, sb, ids, ue8m0=ue8m0)
    assert_gemm_close(C[vt], ref[valid], f"segment ends K={K} ue8m0={ue8m0}")
    assert torch.all(C[~vt] == 7.0), "padding rows must stay unwritten"
    assert torch.equal(q2.view(torch.uint8), q1.view(torch.uint8)) and torch.equal(s2, s1)
    assert torch.all(q2.view(torch.uint8)[~vt] == 0x5A) and torch.all(s2[~vt] == -3.0)


# ------------------------------------------------- FP32 scale contract
# disable_ue8m0_cast: the scales' exponents go to the MFMA, their
# significands are carried per row and the running sum is rescaled when they
# change between K blocks.  These cases vary the significand in every block.

def _scale_factors(shape, rng, lo=-3, hi=3):
    """Factors 2^e * m with a random e in [lo, hi] and m in [1, 2): applied to
    real quant scales they keep realistic magnitudes but make consecutive K
    blocks differ in both exponent and significand."""
    return (rng.uniform(1.0, 2.0, size=shape) * np.exp2(rng.integers(lo, hi + 1, size=shape))).astype(np.float32)


@pytest.mark.parametrize("M,N,K", [(1, 256, 2048), (100, 384, 4096), (300, 512, 3072), (1000, 640, 1024),
                                   (77, 203, 65536), (8, 8192, 8192)])
def test_gemm_fp32_scales_vary_per_block(gpu_device, M, N, K):
    rng = np.random.default_rng(M + K)
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + N)
    sa = (sa * _scale_factors(sa.shape, rng)).astype(np.float32)
    sw = (sw * _scale_factors(sw.shape, rng)).astype(np.float32)
    cols = np.arange(0, N, max(1, N // 512)) if N > 1024 else None
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=False, cols=cols)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=False)
    got = D if cols is None else D[:, torch.from_numpy(cols).to(gpu_device)]
    assert_gemm_close(got, ref, f"fp32 scales {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(300, 512, 768), (96, 1024, 512), (1, 256, 896), (40, 384, 640)])
def test_gemm_fp32_contract_equals_ue8m0_on_power_of_two_scales(gpu_device, M, N, K):
    """Power-of-two scales: both contracts add the same MFMA products in the
    same order (no rescale, no split at fewer than 8 K blocks), so the outputs
    are identical bit for bit."""
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=5)
    D1 = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=True)
    D0 = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=False)
    assert torch.equal(D0, D1)


def test_gemm_fp32_zero_scale_blocks(gpu_device):
    """A zero scale takes the E8M0 operand's floor, 2^-127, so its block adds
    at most 2^-127 of what it would add at scale 1 (the quant kernels never
    produce zero scales: their amax is clamped to eps)."""
    M, N, K = 200, 384, 1536
    rng = np.random.default_rng(8)
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=8)
    sa = (sa * _scale_factors(sa.shape, rng)).astype(np.float32)
    sw = (sw * _scale_factors(sw.shape, rng)).astype(np.float32)
    sa[::7, 3] = 0.0
    sa[5, :] = 0.0
    sw[1, 5] = 0.0
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=False)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=False)
    assert_gemm_close(D, ref, "fp32 zero-scale blocks")
    assert torch.all(D[5].float().abs() < 1e-30)       # every block of row 5 has scale 0


@pytest.mark.parametrize("col_major_a", [False, True])
def test_grouped_gemm_fp32_scales_vary_per_block(gpu_device, col_major_a):
    from kb_nano_amd import _ops
    dev = gpu_device
    E, N, K = 5, 640, 2048
    rng = np.random.default_rng(12)
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N, K, M_tok=150, topk=3, seed=12, dev=dev)
    sa = (sa * _scale_factors(sa.shape, rng)).astype(np.float32)
    sb = (sb * _scale_factors(sb.shape, rng)).astype(np.float32)
    C = torch.full((M_sum, N), 7.0, dtype=torch.bfloat16, device=dev)
    sA = torch.from_numpy(sa).to(dev)
    if col_major_a:
        sA = sA.t().contiguous().t()
    _ops.m_grouped_gemm_nt_contiguous(to_fp8(qa, dev), sA, to_fp8(qb, dev), torch.from_numpy(sb).to(dev), C,
                                      torch.from_numpy(ids).to(dev), disable_ue8m0_cast=True)
    torch.cuda.synchronize()
    ref = oracle.grouped_gemm_nt_sample(qa, sa, qb, sb, ids, ue8m0=False)
    valid = ids >= 0
    assert_gemm_close(C[torch.from_numpy(valid).to(dev)], ref[valid], "grouped fp32 scales")
    assert torch.all(C[torch.from_numpy(~valid).to(dev)] == 7.0)


def test_grouped_gemm_fp32_contract_equals_ue8m0_on_power_of_two_scales(gpu_device):
    from kb_nano_amd import _ops
    dev = gpu_device
    E, N, K = 4, 512, 1024
    ids, qa, sa, qb, sb, M_sum = _grouped_case(E, N, K, M_tok=130, topk=2, seed=4, dev=dev)
    for s_ in (sa[ids >= 0], sb):   # the oracle's quant gives power-of-two (UE8M0) scales
        assert np.all(np.frexp(s_)[0] == 0.5)
    args = (to_fp8(qa, dev), torch.from_numpy(sa).to(dev), to_fp8(qb, dev), torch.from_numpy(sb).to(dev))
    idt = torch.from_numpy(ids).to(dev)
    C1 = torch.zeros(M_sum, N, dtype=torch.bfloat16, device=dev)
    C0 = torch.zeros(M_sum, N, dtype=torch.bfloat16, device=dev)
    _ops.m_grouped_gemm_nt_contiguous(*args, C1, idt, disable_ue8m0_cast=False)
    _ops.m_grouped_gemm_nt_contiguous(*args, C0, idt, disable_ue8m0_cast=True)
    torch.cuda.synchronize()
    assert torch.equal(C0, C1)


@pytest.mark.parametrize("M,N,K", [(1, 8192, 8192), (8, 7168, 16384), (16, 1024, 28672), (32, 8192, 8192),
                                   (24, 10240, 8192), (64, 1024, 28672),
                                   # 33-48 rows with at most 4 splits: summed in the split launch
                                   (48, 8192, 8192), (40, 10240, 8192), (48, 2048, 2048),
                                   # tile counts that are not a multiple of the 8 XCDs: the splits of
                                   # some tiles run on two XCDs and count into the same counter
                                   (1, 1664, 16384), (3, 200, 32768), (16, 1920, 12288)])
def test_gemm_split_fused_reduction_repeats_on_streams_and_graphs(gpu_device, M, N, K):
    """Up to 32 rows (48 when a tile has at most 4 splits), the split-K tail
    is summed by the last workgroup of each tile to finish, counted with
    per-tile arrival counters that each launch leaves at zero (more rows: a
    separate reduction launch, M=64 here).  The sum runs in split order whichever workgroup is last, so
    every call gives the same bits: repeated calls on one stream, calls on
    two streams in flight together, and replays of a captured graph (with
    eager calls between replays) all equal the first call.  Outputs start as
    NaN, so a tile whose reduction did not run is caught."""
    from kb_nano_amd import _ops
    from kb_nano_amd._lib import lib
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    assert lib().kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1) > 0, "shape expected to split its tail"
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + N + K)
    A = to_fp8(qa, gpu_device)
    sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
    sA.copy_(torch.from_numpy(sa))
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)

    def fresh():
        return torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)

    D0 = fresh()
    _ops.fp8_gemm_nt(A, sA, W, sW, D0, use_ue8m0=True)
    torch.cuda.synchronize()
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(K).integers(0, N, 94)]))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=True, cols=cols)
    assert_gemm_close(D0[:, torch.from_numpy(cols).to(gpu_device)], ref, f"fused split {M}x{N}x{K}")
    bits0 = bf16_bits(D0)

    for i in range(3):
        D = fresh()
        _ops.fp8_gemm_nt(A, sA, W, sW, D, use_ue8m0=True)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(D), bits0), f"repeat {i}"

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [fresh() for _ in range(6)]
    torch.cuda.synchronize()
    for i, D in enumerate(outs):   # no synchronisation between: the two streams' launches may overlap
        with torch.cuda.stream(s1 if i % 2 == 0 else s2):
            _ops.fp8_gemm_nt(A, sA, W, sW, D, use_ue8m0=True)
    torch.cuda.synchronize()
    for i, D in enumerate(outs):
        assert np.array_equal(bf16_bits(D), bits0), f"two-stream call {i}"

    Dg = fresh()
    _ops.fp8_gemm_nt(A, sA, W, sW, Dg, use_ue8m0=True)   # warm the caching allocator on this stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _ops.fp8_gemm_nt(A, sA, W, sW, Dg, use_ue8m0=True)
    torch.cuda.synchronize()
    for rep in range(3):
        Dg.fill_(float("nan"))
        De = fresh()
        _ops.fp8_gemm_nt(A, sA, W, sW, De, use_ue8m0=True)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(Dg), bits0), f"graph replay {rep}"
        assert np.array_equal(bf16_bits(De), bits0), f"eager call between replays {rep}"


def test_gemm_fused_splitk_forked_capture(gpu_device):
    """Split GEMMs with the fused (counter-based) reduction on two streams
    forked into one graph capture: the branches share the capture id, so each
    capturing stream must get its own counter region.  Three GEMMs (two of
    them the same shape, so their tile counters coincide) run on the main
    and the side branch of the graph; every replay, with eager calls and NaN
    refills between replays, must give the bits of the eager calls."""
    from kb_nano_amd import _ops
    from kb_nano_amd._lib import lib
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    shapes = [(1, 8192, 8192), (8, 7168, 16384), (8, 7168, 16384)]
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        assert M <= 16 and lib().kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1) > 0, "fused split expected"
        qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=100 + i)
        A = to_fp8(qa, gpu_device)
        sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
        sA.copy_(torch.from_numpy(sa))
        W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
        cases.append((A, sA, W, sW, torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)))

    def run(case, out=None):
        A, sA, W, sW, D = case
        _ops.fp8_gemm_nt(A, sA, W, sW, D if out is None else out, use_ue8m0=True)

    for c in cases:
        run(c)
    torch.cuda.synchronize()
    eager = [bf16_bits(c[4]) for c in cases]
    for c, (M, N, K) in zip(cases, shapes):
        cols = np.arange(0, N, 97)
        qa, sa = fp8_codes(c[0]), c[1].cpu().numpy()
        ref = oracle.gemm_nt_sample(qa, sa, fp8_codes(c[2]), c[3].cpu().numpy(), ue8m0=True, cols=cols)
        assert_gemm_close(c[4][:, torch.from_numpy(cols).to(gpu_device)], ref, f"eager {M}x{N}x{K}")

    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        main = torch.cuda.current_stream()
        side.wait_stream(main)
        run(cases[0])
        run(cases[1])
        with torch.cuda.stream(side):
            run(cases[2])
        main.wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(4):
        for c in cases:
            c[4].fill_(float("nan"))
        extra = torch.full_like(cases[1][4], float("nan"))
        run(cases[1], extra)          # an eager call between replays
        g.replay()
        torch.cuda.synchronize()
        for i, c in enumerate(cases):
            assert np.array_equal(bf16_bits(c[4]), eager[i]), f"replay {rep}, GEMM {i}"
        assert np.array_equal(bf16_bits(extra), eager[1]), f"eager call between replays {rep}"


@pytest.mark.parametrize("M,N,K", [(100, 2304, 4096), (1, 7168, 18432), (8, 8192, 8192), (64, 2048, 2048),
                                   (77, 200, 1152), (300, 1024, 2048), (512, 768, 8704)])
def test_gemm_packed_row_scales_equal_block_scales(gpu_device, M, N, K):
    """DeepGEMM's packed per-row UE8M0 weight scales (int32 [N, ceil(K/512)],
    MN-major; the reference's own fp8_linear scenarios pass this layout,
    bench/kernels/benchmark_scenarios/small/shape_registry.yaml:18719-18737):
    with the block scales' exponents repeated on every row of a block, the
    output is the fp32-block-scale GEMM's bit for bit (data-parallel, split
    tails summed in the split launch and by the reduction, 128x128 and
    256x256 tiles, K not a multiple of 512), every output written."""
    from kb_nano_amd import _ops
    from tests._util import assert_all_written
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + 2 * N + K)
    sw = (sw * np.float32(1.37)).astype(np.float32)   # rounded up to powers of two by both paths
    ref = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=True)
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    A = to_fp8(qa, gpu_device)
    sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
    sA.copy_(torch.from_numpy(sa))
    W = to_fp8(qw, gpu_device)
    packed = _ops.pack_ue8m0_weight_scales(torch.from_numpy(sw).to(gpu_device), N, K)
    assert packed.dtype == torch.int32 and packed.shape == (N, -(-K // 512)) and packed.stride(0) == 1
    D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    _ops.fp8_gemm_nt(A, sA, W, packed, D)
    torch.cuda.synchronize()
    assert_all_written(D, f"packed {M}x{N}x{K}")
    assert np.array_equal(bf16_bits(D), bf16_bits(ref)), f"packed scales != block scales at {M}x{N}x{K}"


def test_gemm_packed_row_scales_per_row_exponents(gpu_device):
    """Exponents that differ on every weight row and K block (row-major int32
    storage this time): each output column n checked against the float64
    oracle with W row n's own scales (a one-row block of the oracle)."""
    from kb_nano_amd import _ops
    M, N, K = 48, 320, 1408          # 11 K blocks: 3 words, the last with 3 bytes used
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=77)
    rng = np.random.default_rng(5)
    KB = K // 128
    # each row's exponent within +-2 of its block's own (realistic magnitudes)
    e_blk = ((np.repeat(sw, 128, axis=0)[:N].view(np.uint32) >> 23) & 0xFF).astype(np.int64)
    e = (e_blk + rng.integers(-2, 3, size=(N, KB))).astype(np.uint32)
    words = -(-KB // 4)
    ep = np.zeros((N, 4 * words), dtype=np.uint32)
    ep[:, :KB] = e
    packed = (ep[:, 0::4] | (ep[:, 1::4] << 8) | (ep[:, 2::4] << 16) | (ep[:, 3::4] << 24)).astype(np.uint32)
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    A = to_fp8(qa, gpu_device)
    sA = _alloc_colmajor_scale(M, KB, gpu_device)
    sA.copy_(torch.from_numpy(sa))
    W = to_fp8(qw, gpu_device)
    P = torch.from_numpy(packed.view(np.int32)).to(gpu_device)
    D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    _ops.fp8_gemm_nt(A, sA, W, P, D)
    torch.cuda.synchronize()
    row_scale = np.ldexp(np.float32(1.0), e.astype(np.int32) - 127).astype(np.float32)   # [N, KB]
    ref = np.concatenate([oracle.gemm_nt_sample(qa, sa, qw[n:n + 1], row_scale[n:n + 1], ue8m0=True)
                          for n in range(N)], axis=1)
    assert_gemm_close(D, ref, "per-row packed exponents")


def test_fp8_linear_with_packed_scales(gpu_device):
    """Fp8Linear given the reference's packed int32 weight_scale_inv: the
    same output as with the equivalent fp32 block scales, eager and into
    installed buffers, at M = 16 and 100."""
    from kb_nano_amd import Fp8Linear, _ops
    N, K = 2304, 4096
    _, _, qw, sw = quantized_gemm_inputs(16, N, K, seed=41)
    W = to_fp8(qw, gpu_device)
    sW = torch.from_numpy(sw).to(gpu_device)
    packed = _ops.pack_ue8m0_weight_scales(sW, N, K)
    for M in (16, 100):
        x = seeded_bf16((M, K), seed=M).to(gpu_device)
        ref = Fp8Linear()(x, W, sW)
        got = Fp8Linear()(x, W, packed)
        lin = Fp8Linear()
        lin._ensure_buffers(128, K, N, gpu_device)
        got2 = lin(x, W, packed)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(got), bf16_bits(ref)), f"M={M}"
        assert np.array_equal(bf16_bits(got2), bf16_bits(ref)), f"M={M} installed buffers"


@pytest.mark.parametrize("M,N,K", [(3000, 7168, 8192), (4096, 7168, 8192), (512, 768, 8192)])
def test_gemm_mixed_256_192_plan(gpu_device, M, N, K):
    """256x256 tiles whose last wave would be partly empty move their last
    columns to 256x192 tiles in a second launch when K >= 8192 (two full
    waves instead of 1.75, DeepSeek-V3 down / o at M = 4096; or only 256x192
    tiles when they fill one wave better).  The 96-column wave tiles straddle 128-row weight
    scale blocks, so each 32-column fragment takes its own block scale.
    Ragged M, NaN-prefilled output entirely written, a point of every
    64x64 block against the float64 oracle, non-power-of-two weight scales
    rounded up under the UE8M0 contract."""
    from tests._util import assert_all_written, tile_cover
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + N + K + 1)
    sw = (sw * np.float32(1.37)).astype(np.float32)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device, ue8m0=True)
    assert_all_written(D, f"mixed plan {M}x{N}x{K}")
    rows, cols = tile_cover(M, N, np.random.default_rng(M + K))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, rows=rows, cols=cols, ue8m0=True)
    got = D[torch.from_numpy(rows).to(gpu_device)][:, torch.from_numpy(cols).to(gpu_device)]
    assert_gemm_close(got, ref, f"mixed plan {M}x{N}x{K}")


def _plan(M, N, K, bf16a=False):
    import ctypes
    from kb_nano_amd._lib import lib
    out = np.zeros(9, dtype=np.int64)
    assert lib().kbn_debug_gemm_plan(M, N, K, 1, int(bf16a), out.ctypes.data) == 0
    return out


@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (64, 2048, 2048), (17, 1024, 7168), (64, 4096, 7168),
                                   (33, 200, 1152), (48, 3072, 2048), (8, 4032, 7168)])
def test_gemm_narrow_64x64_plans(gpu_device, M, N, K):
    """Weight-streaming shapes with narrow weights (N <= 4096, M <= 64) run
    64x64 tiles with K split and summed in the split launch.  Every 64x64
    block of the NaN-prefilled output is written and matches the float64
    oracle; the packed per-row scales, the allocation-free entry point and
    graph replays give the same bits as the workspace entry point, and the
    bf16-activation GEMM gives the bits of quant + GEMM."""
    import ctypes
    from kb_nano_amd import _ops
    from kb_nano_amd._lib import lib
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    from tests._util import assert_all_written, tile_cover
    print(f"narrow {M}x{N}x{K}", flush=True)
    plan = _plan(M, N, K)
    assert plan[0] == 64 and plan[1] == 64 and plan[5] > 1 and plan[7] == 1, plan
    assert np.array_equal(plan, _plan(M, N, K, bf16a=True))
    x = seeded_bf16((M, K), seed=M + K).to(gpu_device)
    A = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=gpu_device)
    sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
    _ops.per_token_group_quant_fp8(x, A, sA)
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=N + K)
    W = to_fp8(qw, gpu_device)
    sW = torch.from_numpy(sw).to(gpu_device)
    D = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    _ops.fp8_gemm_nt(A, sA, W, sW, D, use_ue8m0=True)
    torch.cuda.synchronize()
    assert_all_written(D, f"narrow {M}x{N}x{K}")
    rows, cols = tile_cover(M, N, np.random.default_rng(M + N))
    ref = oracle.gemm_nt_sample(fp8_codes(A), sA.cpu().numpy(), qw, sw, rows=rows, cols=cols, ue8m0=True)
    got = D[torch.from_numpy(rows).to(gpu_device)][:, torch.from_numpy(cols).to(gpu_device)]
    assert_gemm_close(got, ref, f"narrow {M}x{N}x{K}")
    base = bf16_bits(D)
    # bf16 activations, quantized inside the GEMM: the same bits
    D2 = torch.full_like(D, float("nan"))
    _ops.fp8_gemm_bf16a(x, W, sW, D2)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(D2), base), "bf16a != quant + GEMM"
    # packed per-row UE8M0 exponents of the same (power-of-two) block scales
    packed = _ops.pack_ue8m0_weight_scales(sW, N, K)
    D3 = torch.full_like(D, float("nan"))
    _ops.fp8_gemm_nt(A, sA, W, packed, D3)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(D3), base), "packed scales != block scales"
    # the allocation-free entry point
    D4 = torch.full_like(D, float("nan"))
    st = torch.cuda.current_stream().cuda_stream
    rc = lib().kbn_fp8_gemm_nt_noalloc(A.data_ptr(), K, sA.data_ptr(), sA.stride(0), sA.stride(1), W.data_ptr(), K,
                                       sW.data_ptr(), sW.stride(0), D4.data_ptr(), N, M, N, K, 1, st)
    assert rc == 0, lib().kbn_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(D4), base), "noalloc != workspace entry point"
    # graph replays (the split launch's arrival counters under capture)
    D5 = torch.full_like(D, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _ops.fp8_gemm_nt(A, sA, W, sW, D5, use_ue8m0=True)
    torch.cuda.current_stream().wait_stream(side)
    D6 = torch.full_like(D, float("nan"))
    with torch.cuda.stream(side):
        _ops.fp8_gemm_bf16a(x, W, sW, D6)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _ops.fp8_gemm_nt(A, sA, W, sW, D5, use_ue8m0=True)
        _ops.fp8_gemm_bf16a(x, W, sW, D6)
    for _ in range(3):
        D5.fill_(float("nan"))
        D6.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(D5), base), "graph replay"
        assert np.array_equal(bf16_bits(D6), base), "graph replay, bf16 activations"
        _ops.fp8_gemm_nt(A, sA, W, sW, D4, use_ue8m0=True)   # eager work between replays
        _ops.fp8_gemm_bf16a(x, W, sW, D2)
        torch.cuda.synchronize()
    del g


@pytest.mark.parametrize("M,N,K,tile", [(16, 200, 896, (64, 128, 1)), (48, 9000, 1024, (64, 128, 1)),
                                        (100, 200, 896, (128, 128, 1)), (128, 3000, 1536, (128, 128, 1)),
                                        (16, 1032, 4096, (64, 64, 4)), (16, 8200, 2048, (64, 128, 3)),
                                        (20, 1004, 1024, (64, 64, 2))])
def test_gemm_whole_line_store_paths(gpu_device, M, N, K, tile):
    """Tiles of 16 or more live rows leave the GEMM through LDS as whole
    lines (short-K data-parallel tiles: the bf16 block; split tiles: the fp32
    slab); tiles of fewer rows, and rows whose stride is not a multiple of
    8 columns, store directly.  Each shape plans as `tile` (bm, bn, splits)
    for both M and M - 1; the NaN-prefilled output is fully written and
    matches the oracle in every 64x64 block, and the first M - 1 rows are
    bit-identical to the run on those rows alone (M = 16 against 15: the
    staged path against the direct one on the same rows)."""
    print(f"store paths {M}x{N}x{K}", flush=True)
    from tests._util import assert_all_written, tile_cover
    for m in (M, M - 1):
        p = _plan(m, N, K)
        assert (p[0], p[1], p[5]) == tile, (m, p)
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M * 3 + N + K)
    D = _gemm_gpu(qa, sa, qw, sw, gpu_device)
    assert_all_written(D, f"{M}x{N}x{K}")
    rows, cols = tile_cover(M, N, np.random.default_rng(M + N + K))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, rows=rows, cols=cols, ue8m0=True)
    got = D[torch.from_numpy(rows).to(gpu_device)][:, torch.from_numpy(cols).to(gpu_device)]
    assert_gemm_close(got, ref, f"store paths {M}x{N}x{K}")
    D1 = _gemm_gpu(qa[:M - 1], sa[:M - 1], qw, sw, gpu_device)
    assert np.array_equal(bf16_bits(D1), bf16_bits(D[:M - 1])), "rows depend on the row count"
