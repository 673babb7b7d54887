"""Pins the CPU oracle against independent checks (no GPU needed).

Each test compares the oracle with something it does not share code with:
torch's own fp8 cast and log2/ceil/pow formula (the reference's CPU path,
tasks/reference/L1/fp8_linear.py:41-64 and bench/kernels/scenario_registry.py:
54-55, 147-221), 40-digit decimal arithmetic, float64 brute force and closed
forms.  A plausible slip in the oracle (wrong rounding tie, dropped scale,
transposed operand, wrong gate/up column) fails at least one of them.
"""
import decimal
import math
import os

import numpy as np
import pytest
import torch

import oracle

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def _finite_mask(bits):
    return (bits & 0x7F80) != 0x7F80


# --------------------------------------------------------------------- e4m3

def test_e4m3_encode_exhaustive_vs_torch():
    bits = ALL_BF16[_finite_mask(ALL_BF16)]
    x = _bf16_tensor(bits).float()
    want = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = oracle.e4m3_encode(x.numpy())
    # torch keeps the sign on NaN codes; compare NaN-ness for those
    nan_w = (want & 0x7F) == 0x7F
    nan_g = (got & 0x7F) == 0x7F
    assert np.array_equal(nan_w, nan_g)
    assert np.array_equal(want[~nan_w], got[~nan_w])


def test_e4m3_known_answers():
    # RNE ties, subnormals and saturation boundaries (hand-derived)
    cases = {1.0625: 0x38, 1.1875: 0x3A, 2.0 ** -10: 0x00, 1.5 * 2.0 ** -9: 0x02,
             2.0 ** -9: 0x01, 448.0: 0x7E, 464.0: 0x7E, -448.0: 0xFE, 0.0: 0x00,
             2.0 ** -6: 0x08, 7.5 * 2.0 ** -9: 0x08, 6.5 * 2.0 ** -9: 0x06}
    for v, code in cases.items():
        assert oracle.e4m3_encode(np.float32(v)) == code, v
    assert oracle.e4m3_encode(np.float32(465.0)) & 0x7F == 0x7F


def test_e4m3_decode_roundtrip():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    vals = oracle.e4m3_decode(codes)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals, want)
    assert np.array_equal(oracle.e4m3_encode(vals), np.where(vals == 0, 0, codes) | (codes & 0x80))


def test_fast_encoder_matches_scalar():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100,
                        oracle.e4m3_decode(np.arange(127, dtype=np.uint8)),
                        (oracle.e4m3_decode(np.arange(126, dtype=np.uint8)) +
                         oracle.e4m3_decode(np.arange(1, 127, dtype=np.uint8))) / 2])
    v = np.clip(v, -448, 448).astype(np.float32)
    assert np.array_equal(oracle._encode_fast(v), oracle.e4m3_encode(v))


# -------------------------------------------------------------------- UE8M0

def test_ue8m0_exhaustive_vs_reference_formula():
    bits = ALL_BF16[(ALL_BF16 < 0x7F80)]          # +0 .. max finite, subnormals included
    amax = _bf16_tensor(bits).float()
    ratio = amax.clamp_min(1e-10) / 448.0
    want = torch.pow(2.0, torch.ceil(torch.log2(ratio))).numpy()
    got = oracle.ue8m0_from_ratio(ratio.numpy())
    assert np.array_equal(got, want)
    # all-zero group: 2^ceil(log2(1e-10/448)) = 2^-42
    assert oracle.ue8m0_from_ratio(np.float32(np.float32(1e-10) / np.float32(448.0))) == 2.0 ** -42


def test_ue8m0_powers_of_two_are_fixed_points():
    p = np.float32(2.0) ** np.arange(-126, 127, dtype=np.float32)
    assert np.array_equal(oracle.ue8m0_from_ratio(p), p)
    assert np.array_equal(oracle.ue8m0_from_ratio(p * np.float32(1.0000001)), p * 2)


# --------------------------------------------------------------------- silu

def _silu_decimal(g: float) -> float:
    with decimal.localcontext() as ctx:
        ctx.prec = 40
        d = decimal.Decimal(g)
        return float(d / (1 + (-d).exp()))


def _bf16_round_exact(v_str_decimal) -> int:
    """Correctly round a Decimal to bf16 bits (independent of the C code)."""
    d = v_str_decimal
    if d == 0:
        return 0x8000 if d.is_signed() else 0
    sign = 0x8000 if d < 0 else 0
    a = abs(d)
    e = a.adjusted()  # rough decimal exponent
    # binary exponent: find k with 2^k <= a < 2^(k+1)
    k = int(math.floor(float(a.ln() / decimal.Decimal(2).ln()))) if a > 0 else 0
    while decimal.Decimal(2) ** k > a:
        k -= 1
    while decimal.Decimal(2) ** (k + 1) <= a:
        k += 1
    q = max(k - 7, -133)
    scaled = a / (decimal.Decimal(2) ** q)
    r = int(scaled.to_integral_value(rounding=decimal.ROUND_HALF_EVEN))
    v = float(r) * 2.0 ** q
    if v >= 2.0 ** 128:
        return sign | 0x7F80
    return sign | int(np.float32(v).view(np.uint32) >> 16)


def test_silu_table_vs_decimal_exhaustive():
    table = oracle.silu_bf16_table()
    bits = ALL_BF16[_finite_mask(ALL_BF16)]
    g = oracle.bf16_bits_to_f32(bits).astype(np.float64)
    mism = []
    with decimal.localcontext() as ctx:
        ctx.prec = 50
        for b, gv in zip(bits.tolist(), g.tolist()):
            if gv > 200.0:
                want = b  # silu(g) = g * (1 - ~e^-200): rounds back to g
            elif gv < -200.0:
                want = 0x8000  # |silu| < 1e-84: below half the min bf16 subnormal
            else:
                d = decimal.Decimal(gv)
                want = _bf16_round_exact(d / (1 + (-d).exp()))
            if int(table[b]) != want:
                mism.append((b, gv, int(table[b]), want))
    assert not mism, mism[:10]


def test_silu_literal_torch_mismatch_rate_is_small():
    """Where the correctly rounded table departs from the literal fp32 form
    g / (1 + exp(-g)) of tasks/baseline/L1/silu_mul_quant_fp8.py:57-59 (run
    here as torch's F.silu on fp32, then rounded to bf16): 145 of the 65,280
    finite gates (0.22%).  Every mismatch is either one bf16 ulp (the fp32
    roundings of exp, the add and the divide landing on the other side of a
    bf16 rounding midpoint) or a gate below -88.72, where the fp32 exp(-g)
    overflows and the literal form gives -0 while the true value is a tiny
    negative number that bf16 still represents."""
    bits = ALL_BF16[_finite_mask(ALL_BF16)]
    g = _bf16_tensor(bits).float()
    lit = torch.nn.functional.silu(g).bfloat16().view(torch.int16).numpy().astype(np.uint16)
    table = oracle.silu_bf16_table()[bits]
    mism = lit != table
    assert np.mean(mism) < 0.005
    ulp1 = np.abs(lit.astype(np.int32) - table.astype(np.int32)) == 1
    overflow = (g.numpy() < -88.72) & (lit == 0x8000)
    assert np.all(ulp1[mism] | overflow[mism])
    assert np.all(table[overflow] & 0x8000)        # still negative (or -0) in the table


# ------------------------------------------------------------------- quant

def _torch_reference_quant(x_bf16: torch.Tensor, use_ue8m0=True, eps=1e-10):
    """tasks/reference/L1/fp8_linear.py:41-64 (the reference CPU path)."""
    info = torch.finfo(torch.float8_e4m3fn)
    flat = x_bf16.float()
    M, K = flat.shape
    grouped = flat.view(M, K // 128, 128)
    scale = grouped.abs().amax(dim=-1).clamp_min(eps) / info.max
    if use_ue8m0:
        scale = torch.pow(2.0, torch.ceil(torch.log2(scale)))
    expanded = scale.repeat_interleave(128, dim=-1)
    q = torch.clamp(flat / expanded, info.min, info.max).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), scale.numpy()


def _edge_tensor(rows=16):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(rows, 1024, generator=g)
    x[0] = 0.0                                    # all-zero groups -> 2^-42
    x[1, :128] = 448.0 * torch.linspace(-1, 1, 128)
    x[2, :] = torch.randn(1024, generator=g) * 1e-30   # tiny values, subnormal codes
    x[3, ::7] *= 50.0                             # outliers
    x[4, :] = 3.0e38 * torch.sign(torch.randn(1024, generator=g))  # near bf16 max
    x[5, 128:256] = 1.0
    x[5, 130] = 448.0 * 2 ** 3                    # amax exactly 448 * 2^k
    return x.bfloat16()


@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_quant_group128_vs_reference_formula(use_ue8m0):
    x = torch.cat([_edge_tensor(), torch.randn(48, 1024, generator=torch.Generator().manual_seed(1)).bfloat16()])
    bits = x.view(torch.int16).numpy().astype(np.uint16)
    q, s = oracle.quant_group128(bits, use_ue8m0=use_ue8m0)
    qw, sw = _torch_reference_quant(x, use_ue8m0)
    assert np.array_equal(s, sw)
    assert np.array_equal(q, qw)


def _edge_tensor_typed(dtype, rows=16):
    """Edge rows at the range of fp16 or fp32: zeros, a 448 ramp, each type's
    subnormals, outliers, values near the type's max, an amax of 448 * 2^k."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(rows, 1024, generator=g)
    big = 6.0e4 if dtype == torch.float16 else 3.0e38
    tiny = 3.0e-7 if dtype == torch.float16 else 1.0e-39    # fp16 / fp32 subnormals
    x[0] = 0.0
    x[1, :128] = 448.0 * torch.linspace(-1, 1, 128)
    x[2, :] = torch.randn(1024, generator=g) * tiny
    x[3, ::7] *= 50.0
    x[4, :] = big * torch.sign(torch.randn(1024, generator=g))
    x[5, 128:256] = 1.0
    x[5, 130] = 448.0 * 2 ** 3
    x[6, :] = torch.randn(1024, generator=g) * 1e-3
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_quant_group128_f32_vs_reference_formula(dtype, use_ue8m0):
    """fp16 / fp32 inputs: the oracle's float-input quant against the
    reference's formula executed by torch on the same values (its kernel
    widens them to fp32, tasks/baseline/L1/fp8_linear.py:197)."""
    x = torch.cat([_edge_tensor_typed(dtype),
                   torch.randn(48, 1024, generator=torch.Generator().manual_seed(2)).to(dtype)])
    q, s = oracle.quant_group128_f32(x.numpy(), use_ue8m0=use_ue8m0)
    qw, sw = _torch_reference_quant(x, use_ue8m0)
    assert np.array_equal(s, sw)
    assert np.array_equal(q, qw)


def test_quant_group128_f32_equals_bf16_quant_on_bf16_values():
    """On values that are bf16 numbers the float-input quant and the bf16
    quant are one function."""
    x = torch.cat([_edge_tensor(), torch.randn(16, 1024, generator=torch.Generator().manual_seed(3)).bfloat16()])
    for ue8m0 in (True, False):
        q1, s1 = oracle.quant_group128(x.view(torch.int16).numpy().astype(np.uint16), use_ue8m0=ue8m0)
        q2, s2 = oracle.quant_group128_f32(x.float().numpy(), use_ue8m0=ue8m0)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_quant_group128_rejects_ragged_k():
    with pytest.raises(ValueError):
        oracle.quant_group128(np.zeros((2, 100), dtype=np.uint16))


# -------------------------------------------------------------- silu + quant

def test_silu_mul_quant_composition():
    """y = bf16(silu_bf16(gate) * up) then the reference quant; gate/up split
    at N/2 (tasks/baseline/L1/silu_mul_quant_fp8.py:51-60)."""
    g = torch.Generator().manual_seed(3)
    M, Nh = 32, 512
    x = torch.randn(M, 2 * Nh, generator=g)
    x[torch.rand(M, 2 * Nh, generator=g) < 1e-2] *= 50
    x[0, :Nh] = 0.0
    xb = x.bfloat16()
    bits = xb.view(torch.int16).numpy().astype(np.uint16)
    q, s = oracle.silu_mul_quant(bits)
    table = oracle.silu_bf16_table()
    silu = _bf16_tensor(table[bits[:, :Nh]])
    y = (silu.float() * xb[:, Nh:].float()).bfloat16()   # exact product, one RNE
    qw, sw = _torch_reference_quant(y)
    assert np.array_equal(s, sw)
    assert np.array_equal(q, qw)
    # swapping gate and up must change the result (catches a swapped split)
    q2, _ = oracle.silu_mul_quant(np.concatenate([bits[:, Nh:], bits[:, :Nh]], axis=1))
    assert not np.array_equal(q, q2)


# --------------------------------------------------------------------- GEMM

def _rand_fp8(shape, rng, scale=1.0):
    v = np.clip(rng.standard_normal(shape).astype(np.float32) * scale, -448, 448)
    return oracle._encode_fast(v)


def test_gemm_bruteforce_tiny():
    rng = np.random.default_rng(5)
    M, N, K = 3, 130, 256
    A = _rand_fp8((M, K), rng, 4)
    W = _rand_fp8((N, K), rng, 4)
    sA = (2.0 ** rng.integers(-6, 6, (M, K // 128))).astype(np.float32) * np.float32(1.3)
    sW = (2.0 ** rng.integers(-6, 6, (2, K // 128))).astype(np.float32) * np.float32(0.7)
    got = oracle.gemm_nt_sample(A, sA, W, sW)
    a = oracle.e4m3_decode(A).astype(np.float64)
    w = oracle.e4m3_decode(W).astype(np.float64)
    for m in range(M):
        for n in range(N):
            ref = 0.0
            for k in range(K):
                ref += a[m, k] * sA[m, k // 128] * w[n, k] * sW[n // 128, k // 128]
            assert abs(got[m, n] - ref) <= 1e-9 * max(1.0, abs(ref))


def test_gemm_vs_torch_dequant_matmul():
    """The fp32 dequantize-then-matmul form (tasks/reference/L1/fp8_linear.py:
    26-38, 96-104, with A dequantized as well)."""
    g = torch.Generator().manual_seed(0)
    M, N, K = 64, 384, 1024
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02)
    qa, sa = oracle.quant_group128(a.view(torch.int16).numpy().astype(np.uint16))
    qw, sw = oracle.quant_block128(w.numpy())
    got = oracle.gemm_nt_sample(qa, sa, qw, sw)
    A = torch.from_numpy(qa).view(torch.float8_e4m3fn).float() * torch.from_numpy(sa).repeat_interleave(128, 1)
    sWx = torch.from_numpy(sw).repeat_interleave(128, 0).repeat_interleave(128, 1)[:N, :K]
    W = torch.from_numpy(qw).view(torch.float8_e4m3fn).float() * sWx
    ref = (A.double() @ W.double().T).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-9 * np.max(np.abs(ref))
    ref32 = torch.nn.functional.linear(A, W).numpy()
    assert np.max(np.abs(got - ref32)) / np.max(np.abs(ref)) < 1e-5


def test_gemm_special_cases():
    rng = np.random.default_rng(9)
    M, N, K = 4, 256, 384
    A = _rand_fp8((M, K), rng, 8)
    W = np.zeros((N, K), dtype=np.uint8)
    # identity-like weight: W[n, n] = 1.0 (code 0x38) inside the first K block
    for n in range(128):
        W[n, n] = 0x38
    sA = np.full((M, K // 128), 0.5, dtype=np.float32)
    sW = np.full((2, K // 128), 4.0, dtype=np.float32)
    got = oracle.gemm_nt_sample(A, sA, W, sW)
    a = oracle.e4m3_decode(A).astype(np.float64)
    assert np.array_equal(got[:, :128], a[:, :128] * 2.0)
    assert np.all(got[:, 128:] == 0)
    # a single non-zero K block picks up only that block's scales
    W2 = _rand_fp8((N, K), rng, 2)
    W2[:, :128] = 0
    W2[:, 256:] = 0
    sW2 = np.array([[1.0, 8.0, 1e6], [1.0, 0.25, 1e6]], dtype=np.float32)
    got2 = oracle.gemm_nt_sample(A, sA, W2, sW2)
    w2 = oracle.e4m3_decode(W2).astype(np.float64)
    ref = np.empty((M, N))
    ref[:, :128] = (a[:, 128:256] @ w2[:128, 128:256].T) * 0.5 * 8.0
    ref[:, 128:] = (a[:, 128:256] @ w2[128:, 128:256].T) * 0.5 * 0.25
    assert np.allclose(got2, ref, rtol=1e-12, atol=1e-12)


def test_gemm_ue8m0_contract_rounds_scales_up():
    rng = np.random.default_rng(11)
    A = _rand_fp8((2, 128), rng)
    W = _rand_fp8((128, 128), rng)
    sA = np.array([[0.3], [0.25]], dtype=np.float32)
    sW = np.array([[3.0]], dtype=np.float32)
    got = oracle.gemm_nt_sample(A, sA, W, sW, ue8m0=True)
    ref = oracle.gemm_nt_sample(A, np.array([[0.5], [0.25]], np.float32), W, np.array([[4.0]], np.float32))
    assert np.array_equal(got, ref)


def test_grouped_gemm_matches_dense_per_expert():
    rng = np.random.default_rng(2)
    E, N, K, M_sum = 3, 256, 256, 512
    A = _rand_fp8((M_sum, K), rng)
    sA = (2.0 ** rng.integers(-3, 3, (M_sum, K // 128))).astype(np.float32)
    B = _rand_fp8((E, N, K), rng)
    sB = (2.0 ** rng.integers(-3, 3, (E, 2, K // 128))).astype(np.float32)
    ids = np.repeat(np.array([2, 0, -1, 1], dtype=np.int32), 128)
    got = oracle.grouped_gemm_nt_sample(A, sA, B, sB, ids)
    for blk, e in enumerate([2, 0, -1, 1]):
        sl = slice(blk * 128, (blk + 1) * 128)
        if e < 0:
            assert np.all(np.isnan(got[sl]))
        else:
            assert np.array_equal(got[sl], oracle.gemm_nt_sample(A[sl], sA[sl], B[e], sB[e]))


# ---------------------------------------------------------------- MoE layout

def test_permute_contiguous_layout():
    rng = np.random.default_rng(0)
    M, k, E, align = 50, 4, 8, 16
    topk = np.stack([rng.choice(E, k, replace=False) for _ in range(M)])
    ids, dest, M_sum = oracle.permute_contiguous(topk, E, align)
    assert M_sum == oracle.compute_aligned_M(M, k, E, align)
    assert M_sum % align == 0 and M_sum >= M * k + E * (align - 1)
    flat = topk.reshape(-1)
    assert len(set(dest.tolist())) == M * k                  # injective
    assert np.array_equal(ids[dest], flat.astype(np.int32))  # row carries its expert
    assert np.sum(ids >= 0) == M * k
    # segments start on alignment boundaries and keep (token, slot) order
    for e in range(E):
        rows_e = dest[flat == e]
        assert rows_e[0] % align == 0
        assert np.all(np.diff(rows_e) == 1)


def test_compute_aligned_M_cfg4():
    assert oracle.compute_aligned_M(4096, 8, 256, 128) == 65280


def _brute_force_layout(topk, E, align):
    """Placement by direct counting, independent of the oracle's sort: walk
    the experts in order, give each its pairs in (token, slot) order, then
    round its row count up to the alignment."""
    M, k = topk.shape
    M_sum = oracle.compute_aligned_M(M, k, E, align)
    dest = np.full(M * k, -1, dtype=np.int64)
    ids = np.full(M_sum, -1, dtype=np.int32)
    row = 0
    for e in range(E):
        n_e = 0
        for m in range(M):
            for j in range(k):
                if topk[m, j] == e:
                    dest[m * k + j] = row + n_e
                    ids[row + n_e] = e
                    n_e += 1
        row += -(-n_e // align) * align
    return ids, dest, M_sum


@pytest.mark.parametrize("M,k,E,align,seed", [(50, 4, 8, 16, 0), (9, 3, 5, 4, 1), (1, 1, 1, 128, 2),
                                              (0, 2, 3, 8, 3), (40, 6, 7, 1, 4)])
def test_permute_contiguous_brute_force(M, k, E, align, seed):
    rng = np.random.default_rng(seed)
    topk = rng.integers(0, E, size=(M, k))
    ids, dest, M_sum = oracle.permute_contiguous(topk, E, align)
    ids_b, dest_b, M_sum_b = _brute_force_layout(topk, E, align)
    assert M_sum == M_sum_b
    assert np.array_equal(ids, ids_b)
    assert np.array_equal(dest, dest_b)


def test_permute_contiguous_drops_out_of_range_ids():
    topk = np.array([[0, 3], [-1, 1], [5, 0], [1, 1]])
    ids, dest, M_sum = oracle.permute_contiguous(topk, 4, 2)
    # valid pairs only: e0 <- (0,0), (2,1); e1 <- (1,1), (3,0), (3,1); e3 <- (0,1)
    # rounded counts 2, 4, 0, 2 -> offsets 0, 2, 6, 6
    assert dest.tolist() == [0, 6, -1, 2, -1, 1, 3, 4]
    assert ids.tolist() == [0, 0, 1, 1, 1, -1, 3, -1, -1, -1, -1, -1]
    assert M_sum == oracle.compute_aligned_M(4, 2, 4, 2)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
def test_unpermute_matches_reference_formula(wdtype):
    """The reference's torch formula (fused_experts.py:130-136) on CPU:
    gather, ``.to(bf16) * weights``, ``.sum(dim=1)``, copy into bf16."""
    g = torch.Generator().manual_seed(7)
    M, k, H, rows = 64, 8, 256, 700
    y = torch.randn(rows, H, generator=g).bfloat16()
    inv = torch.stack([torch.randperm(rows, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    w = torch.softmax(torch.randn(M, k, generator=g), -1).to(wdtype)
    out = torch.empty(M, H, dtype=torch.bfloat16)
    gathered = y[inv.to(torch.int64).view(-1)].view(M, k, H)
    out.copy_((gathered.to(out.dtype) * w.unsqueeze(-1)).sum(dim=1))
    got = oracle.unpermute_and_reduce(oracle.bf16_bits_to_f32(y.view(torch.int16).numpy().view(np.uint16)),
                                      inv.numpy(), w.float().numpy(), bf16_products=wdtype == torch.bfloat16)
    got_bits = oracle.f32_to_bf16_bits(got).astype(np.int32)
    ref_bits = out.view(torch.int16).numpy().view(np.uint16).astype(np.int32)
    # same products; the fp32 sum may differ in order, so allow one bf16 ulp
    assert np.max(np.abs(got_bits - ref_bits)) <= 1
    assert np.mean(got_bits == ref_bits) > 0.99


def test_unpermute_slot_order_and_skips():
    y = np.array([[1.0, 2.0], [3.0, 4.0], [1e8, -1e8]], dtype=np.float32)
    inv = np.array([[2, 0, 2], [1, -1, 5]])
    w = np.array([[1.0, 1.0, -1.0], [0.5, 9.0, 9.0]], dtype=np.float32)
    out = oracle.unpermute_and_reduce(y, inv, w)
    # slot order: (1e8 + 1) - 1e8 = 0 in fp32 (1 is lost), not 1
    assert out[0].tolist() == [0.0, 0.0]
    assert out[1].tolist() == [1.5, 2.0]    # rows -1 and 5 are outside [0, 3)


# ----------------------------------------------------------- golden fixtures

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_golden_quant_edge_fixture():
    """The committed quant fixture (tests/golden/make_fixtures.py) is what
    the oracle computes, and its e4m3 ties carry the known round-half-even
    codes: 1.0625 -> 1.0 (0x38), 1.1875 -> 1.25 (0x3A), 3.125 -> 3.0 (0x44),
    9/1024 -> 4 * 2^-9 (0x04), 448 -> 0x7E, negatives with the sign bit."""
    d = _golden("quant_edge.npz")
    for ue8m0, qk, sk in ((True, "q_ue8m0", "s_ue8m0"), (False, "q_fp32", "s_fp32")):
        q, s = oracle.quant_group128(d["x_bits"], use_ue8m0=ue8m0)
        assert np.array_equal(q, d[qk]) and np.array_equal(s, d[sk])
    assert list(d["q_ue8m0"][2, 256:265]) == [0x38, 0x3A, 0xB8, 0xBA, 0x44, 0xC4, 0x04, 0x84, 0x7E]
    assert d["s_ue8m0"][2, 2] == 1.0 and d["s_ue8m0"][1, 0] == 1.0 and d["s_ue8m0"][1, 1] == 32.0
    assert d["s_ue8m0"][0, 0] == 2.0 ** -42      # all-zero group: eps / 448 rounded up


def test_golden_silu_fixture():
    d = _golden("silu_mul_quant.npz")
    for ue8m0, qk, sk in ((True, "q_ue8m0", "s_ue8m0"), (False, "q_fp32", "s_fp32")):
        q, s = oracle.silu_mul_quant(d["x_bits"], use_ue8m0=ue8m0)
        assert np.array_equal(q, d[qk]) and np.array_equal(s, d[sk])


def test_golden_gemm_cfg1_fixture():
    """BASELINE config 1 regenerated from its seed: same quantized inputs,
    same oracle output (sha256 of the bf16 result and a 16 x 64 slice)."""
    import hashlib

    from tests._util import quantized_gemm_inputs
    d = _golden("gemm_cfg1.npz")
    M, N, K = int(d["M"]), int(d["N"]), int(d["K"])
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=int(d["seed"]))
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert sha(qa) + sha(sa) + sha(qw) + sha(sw) == str(d["inputs_sha256"])
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=True)
    assert sha(oracle.f32_to_bf16_bits(ref.astype(np.float32))) == str(d["out_bf16_sha256"])
    assert np.array_equal(ref[:16, :64], d["out_slice"])


# ------------------------------------------------------ RMSNorm + 1x128 quant
# oracle.rmsnorm_quant restates tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-201
# in the kernel's fixed fp32 order; these pin it independently of that order.

def _bf16(a):
    return oracle.f32_to_bf16_bits(np.asarray(a, dtype=np.float32))


def test_rmsnorm_quant_unit_rows_reduce_to_plain_quant():
    """x = +-1 and eps = 0: sum(x^2) = H exactly, inv = 1, so v = x * w is a
    bf16 value and the codes and scales are the plain 1x128 quant of it."""
    rng = np.random.default_rng(3)
    M, H = 6, 1024
    x = np.where(rng.random((M, H)) < 0.5, -1.0, 1.0).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32) * np.exp2(rng.integers(-6, 6, H))
    wb = _bf16(w)
    q, s = oracle.rmsnorm_quant(_bf16(x), wb, eps=0.0)
    xw = _bf16(x * oracle.bf16_bits_to_f32(wb)[None, :])
    q2, s2 = oracle.quant_group128(xw, use_ue8m0=True)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_rmsnorm_quant_scale_invariance():
    """Scaling a row by 2^k scales every square by 4^k exactly, so with eps=0
    the normalized values, codes and scales do not change."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    w = _bf16(rng.standard_normal(2048))
    q0, s0 = oracle.rmsnorm_quant(_bf16(x), w, eps=0.0)
    for k in (-20, 7):
        qk, sk = oracle.rmsnorm_quant(_bf16(x * np.float32(2.0 ** k)), w, eps=0.0)
        assert np.array_equal(q0, qk) and np.array_equal(s0, sk)


def test_rmsnorm_quant_matches_float64():
    """Against the same math in float64: codes and scales agree except where
    v / s lies within fp32 rounding of an e4m3 tie (adjacent codes only)."""
    rng = np.random.default_rng(5)
    M, H, eps = 64, 7168, 1e-6
    xb = _bf16(rng.standard_normal((M, H)))
    wb = _bf16(rng.standard_normal(H))
    q, s = oracle.rmsnorm_quant(xb, wb, eps=eps)
    x = oracle.bf16_bits_to_f32(xb).astype(np.float64)
    w = oracle.bf16_bits_to_f32(wb).astype(np.float64)
    v = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w[None, :]
    amax = np.maximum(np.abs(v).reshape(M, H // 128, 128).max(axis=2), 1e-10)
    s64 = np.exp2(np.ceil(np.log2(amax / 448.0)))
    assert np.mean(s == s64) > 0.999
    codes64 = oracle.e4m3_encode(np.clip(v / np.repeat(s, 128, axis=1), -448, 448).astype(np.float32))
    dq = oracle.e4m3_decode(q).astype(np.float64)
    d64 = oracle.e4m3_decode(codes64).astype(np.float64)
    same = q == codes64
    assert same.mean() > 0.999
    # where they differ, they are neighbours on the e4m3 grid
    step = np.abs(d64) * 2.0 ** -3 + 2.0 ** -9
    assert np.all(np.abs(dq - d64)[~same] <= step[~same] + 1e-12)


def test_rmsnorm_quant_meets_reference_two_kernel_bar():
    """The reference's own acceptance test (tests/debug/test_fused_norm_quant.py:
    43-76): against RMSNorm to bf16 followed by the 1x128 quant, fewer than 7%
    of codes differ and the scales agree within 0.016."""
    rng = np.random.default_rng(6)
    for H in (3584, 4096, 8192):
        wb = _bf16(rng.standard_normal(H))
        for bs in (1, 8, 32, 128):
            xb = _bf16(rng.standard_normal((bs, H)))
            q, s = oracle.rmsnorm_quant(xb, wb, eps=1e-6)
            x = oracle.bf16_bits_to_f32(xb)
            inv = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)).astype(np.float32)
            norm = _bf16(oracle.bf16_bits_to_f32(_bf16(x * inv)) * oracle.bf16_bits_to_f32(wb)[None, :])
            q2, s2 = oracle.quant_group128(norm, use_ue8m0=True)
            assert np.mean(q != q2) < 0.07
            assert np.max(np.abs(s - s2)) <= 0.016


def test_rmsnorm_quant_residual_variant():
    """Fused add: residual <- bf16(residual + x) exactly; the normalized bf16
    row written back into x re-quantizes to the same codes where it is not a
    tie; and the codes are those of the plain variant on the new residual
    except where the unrounded sum of squares moves a value across a tie."""
    rng = np.random.default_rng(7)
    M, H = 16, 4096
    xb = _bf16(rng.standard_normal((M, H)))
    rb = _bf16(rng.standard_normal((M, H)) * 4)
    wb = _bf16(rng.standard_normal(H))
    q, s, r_out, x_out = oracle.rmsnorm_quant(xb, wb, eps=1e-6, residual_bits=rb)
    assert np.array_equal(r_out, _bf16(oracle.bf16_bits_to_f32(rb) + oracle.bf16_bits_to_f32(xb)))
    q_plain, s_plain = oracle.rmsnorm_quant(r_out, wb, eps=1e-6)
    assert np.mean(q == q_plain) > 0.99 and np.mean(s == s_plain) > 0.99
    xo = oracle.bf16_bits_to_f32(x_out)
    dq = oracle.e4m3_decode(q) * np.repeat(s, 128, axis=1)
    assert np.all(np.abs(xo - dq) <= np.abs(xo) * 2.0 ** -3 + np.repeat(s, 128, axis=1) * 2.0 ** -9 + 1e-30)


def test_f16_rounding_matches_numpy():
    """The oracle's binary16 rounding (nearest even, subnormals, overflow from
    65520) and decoding against numpy's float16 on random fp32 bit patterns,
    the boundaries, and every binary16 value."""
    rng = np.random.default_rng(8)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x477FEFFF, 0x477FF000, 0x477FF001, 0x477FE000, 0x38800000, 0x387FFFFF,
                                     0x33800000, 0x33000000, 0x33000001, 0x32FFFFFF, 0x7F800000, 0xFF800000,
                                     0, 0x80000000], np.uint32)])
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16_bits(f), ref)
    L = oracle.lib()
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dec = np.array([L.orc_f16_to_float(int(h)) for h in allh], np.float32)
    ref = allh.view(np.float16).astype(np.float32)
    assert np.all((dec.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(dec) & np.isnan(ref)))


def test_rmsnorm_quant_values_bf16_equals_bits_oracle():
    """The typed restatement on bf16 rows is the bf16 oracle (plain and fused
    add, H below and above the 8-chunk wavefront switch, and past 16384)."""
    rng = np.random.default_rng(9)
    for H in (1024, 7168, 20480):
        xb, rb, wb = _bf16(rng.standard_normal((5, H))), _bf16(rng.standard_normal((5, H)) * 4), \
            _bf16(rng.standard_normal(H))
        f = oracle.bf16_bits_to_f32
        q1, s1 = oracle.rmsnorm_quant(xb, wb, eps=1e-6)
        q2, s2 = oracle.rmsnorm_quant_values(f(xb), f(wb), "bf16", eps=1e-6)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
        q1, s1, r1, x1 = oracle.rmsnorm_quant(xb, wb, eps=1e-6, residual_bits=rb)
        q2, s2, r2, x2 = oracle.rmsnorm_quant_values(f(xb), f(wb), "bf16", eps=1e-6, residual=f(rb))
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
        assert np.array_equal(f(r1), r2) and np.array_equal(f(x1), x2)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_rmsnorm_quant_values_fp16_fp32_pins(dtype):
    """fp16 / fp32 rows: the reference's two-kernel bar (RMSNorm, then the
    1x128 quant; fewer than 7% of codes differ, scales within 0.016), the
    float64 math (codes equal or adjacent on the e4m3 grid), scale
    invariance, and the fused add's residual = r + x rounded once to the
    type, with the normalized row written back in the type."""
    npt = np.float16 if dtype == "fp16" else np.float32
    rng = np.random.default_rng(10)
    M, H, eps = 32, 4096, 1e-6
    x = rng.standard_normal((M, H)).astype(npt).astype(np.float32)
    w = rng.standard_normal(H).astype(npt).astype(np.float32)
    q, s = oracle.rmsnorm_quant_values(x, w, dtype, eps=eps)
    xd, wd = x.astype(np.float64), w.astype(np.float64)
    v = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + eps) * wd[None, :]
    amax = np.maximum(np.abs(v).reshape(M, H // 128, 128).max(axis=2), 1e-10)
    s64 = np.exp2(np.ceil(np.log2(amax / 448.0)))
    assert np.mean(s == s64) > 0.999
    codes64 = oracle.e4m3_encode(np.clip(v / np.repeat(s, 128, axis=1), -448, 448).astype(np.float32))
    same = q == codes64
    assert same.mean() > 0.999
    dq, d64 = oracle.e4m3_decode(q).astype(np.float64), oracle.e4m3_decode(codes64).astype(np.float64)
    assert np.all(np.abs(dq - d64)[~same] <= (np.abs(d64) * 2.0 ** -3 + 2.0 ** -9)[~same] + 1e-12)
    norm = (x * (1.0 / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + eps)).astype(np.float32))
    norm = norm.astype(npt).astype(np.float32) * w[None, :]
    q2, s2 = oracle.quant_group128_f32(norm.astype(npt).astype(np.float32), use_ue8m0=True)
    assert np.mean(q != q2) < 0.07 and np.max(np.abs(s - s2)) <= 0.016
    for k in (-6, 5):
        qk, sk = oracle.rmsnorm_quant_values(x * np.float32(2.0 ** k), w, dtype, eps=0.0)
        q0, s0 = oracle.rmsnorm_quant_values(x, w, dtype, eps=0.0)
        assert np.array_equal(q0, qk) and np.array_equal(s0, sk)
    r = (rng.standard_normal((M, H)) * 4).astype(npt).astype(np.float32)
    qa, sa, r_out, x_out = oracle.rmsnorm_quant_values(x, w, dtype, eps=eps, residual=r)
    assert np.array_equal(r_out, (r + x).astype(npt).astype(np.float32))
    assert np.array_equal(x_out, x_out.astype(npt).astype(np.float32))
    qp, sp = oracle.rmsnorm_quant_values(r_out, w, dtype, eps=eps)
    assert np.mean(qa == qp) > 0.99 and np.mean(sa == sp) > 0.99


# ------------------------------------------------------- weight block requant

def _torch_per_block_cast(x: torch.Tensor, use_ue8m0: bool):
    """DeepGEMM's per_block_cast_to_fp8 as the reference calls it
    (tasks/baseline/L1/fp8_linear.py:497-499), run by torch on the CPU: zero
    padding to whole blocks, amax clamped at 1e-4, sf = amax/448 (rounded up
    to 2^ceil(log2 sf) under UE8M0), codes = (x * (1/sf)).to(e4m3)."""
    m, n = x.shape
    xp = torch.zeros(-(-m // 128) * 128, -(-n // 128) * 128)
    xp[:m, :n] = x
    xv = xp.view(-1, 128, xp.size(1) // 128, 128)
    amax = xv.abs().float().amax(dim=(1, 3), keepdim=True).clamp(1e-4)
    sf = amax / 448.0
    if use_ue8m0:
        sf = torch.pow(2.0, torch.ceil(torch.log2(sf.abs())))
    q = (xv * (1.0 / sf)).to(torch.float8_e4m3fn)
    return (q.view_as(xp)[:m, :n].contiguous().view(torch.uint8).numpy(),
            sf.view(xv.size(0), xv.size(2)).numpy())


def _checkpoint_weight(N, K, seed):
    """fp8 codes plus arbitrary (non power-of-two) fp32 block scales, as a
    checkpoint stores them."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    q, s = oracle.quant_block128(w, use_ue8m0=False)
    s = (s * rng.uniform(0.5, 3.0, s.shape)).astype(np.float32)
    return q, s


@pytest.mark.parametrize("N,K", [(256, 384), (200, 208), (130, 512), (128, 16)])
@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_block_requant_vs_torch_deepgemm_formula(N, K, use_ue8m0):
    q, s = _checkpoint_weight(N, K, seed=N + K)
    got_q, got_s = oracle.block_requant(q, s, use_ue8m0=use_ue8m0)
    # the reference's dequant (:486): codes to fp32 times the block scale
    sx = torch.from_numpy(s).repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]
    x = torch.from_numpy(q).view(torch.float8_e4m3fn).float() * sx
    ref_q, ref_s = _torch_per_block_cast(x, use_ue8m0)
    assert np.array_equal(got_s, ref_s)
    assert np.array_equal(got_q, ref_q)
    # an fp32 master weight goes through the same cast
    got_q2, got_s2 = oracle.block_requant(x.numpy(), None, use_ue8m0=use_ue8m0)
    assert np.array_equal(got_q2, ref_q) and np.array_equal(got_s2, ref_s)


def test_block_requant_batched_and_special_blocks():
    """Experts requantize independently; an all-zero block gets sf = 1e-4/448
    (2^-22 under UE8M0) and zero codes; a block with a huge entry keeps its
    largest code at 448; ue8m0 with fp32 input equals quant_block128's
    division form at eps 1e-4 (1/sf is exact for a power of two)."""
    rng = np.random.default_rng(3)
    E, N, K = 3, 256, 256
    x = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    x[1, :128, 128:] = 0.0
    x[2, 5, 7] = 3.0e4
    q, s = oracle.block_requant(x, None, use_ue8m0=True)
    for e in range(E):
        qe, se = oracle.block_requant(x[e], None, use_ue8m0=True)
        assert np.array_equal(q[e], qe) and np.array_equal(s[e], se)
        qb, sb = oracle.quant_block128(x[e], eps=1e-4, use_ue8m0=True)
        assert np.array_equal(qe, qb) and np.array_equal(se, sb)
    assert s[1, 0, 1] == np.float32(2.0 ** -22) and not q[1, :128, 128:].any()
    assert oracle.e4m3_decode(q[2, 5, 7]) == 448.0 or s[2, 0, 0] * 448 > 3.0e4
    _, s_plain = oracle.block_requant(x[1], None, use_ue8m0=False)
    assert s_plain[0, 1] == np.float32(np.float32(1e-4) / np.float32(448))


def test_block_requant_identity_on_pow2_checkpoint():
    """Codes whose block maximum is 448 with power-of-two block scales come
    back unchanged under UE8M0: amax = 448 * 2^k gives sf = 2^k exactly."""
    rng = np.random.default_rng(8)
    N, K = 384, 256
    q = oracle._encode_fast(np.clip(rng.standard_normal((N, K)) * 60, -447, 447).astype(np.float32))
    q[::128, ::128] = 0x7E                     # 448 in every block
    s = (2.0 ** rng.integers(-14, -6, (3, 2))).astype(np.float32)
    q2, s2 = oracle.block_requant(q, s, use_ue8m0=True)
    assert np.array_equal(q2, q) and np.array_equal(s2, s)
    # a non power-of-two scale moves the codes: x * (1/sf) is then inexact
    q3, s3 = oracle.block_requant(q, s * np.float32(1.3), use_ue8m0=True)
    assert not np.array_equal(q3, q) and np.array_equal(s3, s * 2)


# ------------------------------------------------------- sorted-token MoE

@pytest.mark.parametrize("M,k,E,block", [(37, 8, 16, 4), (5, 2, 64, 16), (300, 8, 256, 64), (3, 1, 8, 128),
                                         (64, 6, 33, 32)])
def test_moe_align_oracle_layout(M, k, E, block):
    """Each expert's slots hold exactly its pairs (brute force over the flat
    ids), segments are padded to the block size, the rest of the reference's
    buffer is the sentinel numel, and block owners follow the segments."""
    rng = np.random.default_rng(M * 7 + E)
    ids = rng.integers(0, E, size=(M, k))
    if M > 10:
        ids[3, 0] = -1                       # invalid ids are not placed
        ids[4, 0] = E
    sorted_ids, expert_ids, total, cumsum = oracle.moe_align_block_size(ids, E, block)
    flat = ids.reshape(-1)
    numel = flat.size
    bound = numel * block if numel < E else numel + E * (block - 1)
    assert sorted_ids.size == bound and total <= bound and total % block == 0
    assert cumsum[0] == 0 and cumsum[-1] == total
    placed = np.zeros(bound, dtype=bool)
    for e in range(E):
        mine = np.flatnonzero(flat == e)
        seg = sorted_ids[cumsum[e]:cumsum[e + 1]]
        assert cumsum[e + 1] - cumsum[e] == -(-mine.size // block) * block
        assert np.array_equal(seg[:mine.size], mine)
        assert np.all(seg[mine.size:] == numel)
        placed[cumsum[e]:cumsum[e] + mine.size] = True
        assert np.all(expert_ids[cumsum[e] // block:cumsum[e + 1] // block] == e)
    assert np.all(sorted_ids[~placed] == numel)
    assert expert_ids.size == total // block


def test_moe_sum_oracle_orders():
    """Inputs with exact fp32 sums that tell the orders apart: three slots
    where per-add bf16 rounding loses what a single rounding keeps (the
    reference kernel's bf16 accumulator for top_k <= 4), and eight slots
    where round-robin accumulators cancel 2^24 before adding the ones (the
    order of at::sum_out) while a left-to-right fp32 sum absorbs them."""
    def bits(rows):
        return oracle.f32_to_bf16_bits(np.array(rows, dtype=np.float32)[None, :, None])
    one_ulp_half = 2.0 ** -8
    got = oracle.bf16_bits_to_f32(oracle.moe_sum(bits([1.0, one_ulp_half, one_ulp_half])))[0, 0]
    assert got == 1.0                                  # single rounding would give 1 + 2^-7
    got2 = oracle.bf16_bits_to_f32(oracle.moe_sum(bits([1.0, one_ulp_half])))[0, 0]
    assert got2 == 1.0
    v = [2.0 ** 24, 1.0, 1.0, 0.0, -(2.0 ** 24), 0.0, 0.0, 0.0]
    assert oracle.bf16_bits_to_f32(oracle.moe_sum(bits(v)))[0, 0] == 2.0   # left to right would give 0
    v9 = v + [3.0]
    assert oracle.bf16_bits_to_f32(oracle.moe_sum(bits(v9)))[0, 0] == 5.0
    # one slot is the identity; random rows stay within one bf16 rounding of float64
    x = oracle.f32_to_bf16_bits(np.random.default_rng(2).standard_normal((4, 1, 64)).astype(np.float32))
    assert np.array_equal(oracle.moe_sum(x), x[:, 0])
    xr = np.random.default_rng(3).standard_normal((16, 8, 256)).astype(np.float32)
    xb = oracle.f32_to_bf16_bits(xr)
    ref = oracle.bf16_bits_to_f32(xb).astype(np.float64).sum(1)
    got = oracle.bf16_bits_to_f32(oracle.moe_sum(xb)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)


def test_fused_moe_gemm_oracle_bruteforce():
    """Tiny sorted-token GEMM in float64 from the decoded operands, with
    routed weights, an invalid pair and the naive one-pair blocks."""
    rng = np.random.default_rng(11)
    M, k, E, N, K, block = 5, 2, 3, 130, 256, 4
    ids = rng.integers(0, E, size=(M, k))
    ids[2, 1] = -1
    A = _rand_fp8((M, K), rng, 6)
    sA = (2.0 ** rng.integers(-4, 4, (M, K // 128))).astype(np.float32) * np.float32(1.25)
    B = _rand_fp8((E, N, K), rng, 6)
    sB = (2.0 ** rng.integers(-4, 4, (E, 2, K // 128))).astype(np.float32) * np.float32(0.75)
    w = rng.uniform(0.1, 1.0, (M, k)).astype(np.float32)
    sorted_ids, expert_ids, total, _ = oracle.moe_align_block_size(ids, E, block)
    got = oracle.fused_moe_gemm_sample(A, sA, B, sB, sorted_ids, expert_ids, total, block, M * k, k, w)
    a = oracle.e4m3_decode(A).astype(np.float64)
    b = oracle.e4m3_decode(B).astype(np.float64)
    flat = ids.reshape(-1)
    assert sorted(got) == [t for t in range(M * k) if flat[t] >= 0]
    for t, row in got.items():
        e, m = flat[t], t // k
        ref = np.zeros(N)
        for kb in range(K // 128):
            ks = slice(kb * 128, kb * 128 + 128)
            ref += sA[m, kb] * np.repeat(sB[e, :, kb], 128)[:N] * (b[e][:, ks] @ a[m, ks])
        assert np.allclose(row, ref * w.reshape(-1)[t], rtol=1e-12, atol=1e-12)
    # naive: block b holds pair b alone, expert ids are the flat routing
    flat_ok = np.where(flat >= 0, flat, 0).astype(np.int32)
    nv = oracle.fused_moe_gemm_sample(A, sA, B, sB, None, flat_ok, M * k * block, block, M * k, k, None,
                                      naive=True)
    assert sorted(nv) == list(range(M * k))
    t = 3
    assert np.allclose(nv[t], got[t] / w.reshape(-1)[t], rtol=1e-12)


def test_ue8m0_scale_without_division_identity():
    """The kernels' division-free UE8M0 scale (kbn_common.h ue8m0_ceil_div448):
    for amax = m 2^e, ceil_pow2(fl(amax / 448)) is 2^(e-8) when m <= 1.75 and
    2^(e-7) otherwise.  Checked against the definition (float32 division, then
    the oracle's exponent rounding) for every mantissa at a spread of
    exponents, including both sides of 1.75 and the edges of the range the
    kernels use the formula for (biased exponent 10 .. 254)."""
    mant = np.arange(1 << 23, dtype=np.uint32)
    for e in (10, 11, 60, 100, 126, 127, 128, 160, 200, 253, 254):
        u = (np.uint32(e) << np.uint32(23)) | mant
        amax = u.view(np.float32)
        ratio = (amax / np.float32(448.0)).astype(np.float32)
        # definition: exponent bits of the quotient, plus one if its mantissa is not zero
        ru = ratio.view(np.uint32)
        want = ((ru >> 23) & 0xFF) + ((ru & 0x7FFFFF) != 0)
        got = np.uint32(e) - 8 + (mant > 0x600000)
        assert np.array_equal(got, want.astype(np.uint32)), e


def test_torch_restatements_match_the_c_oracle():
    """The torch restatements of the reference CPU path (timed as the bench's
    CPU baseline) agree with the pinned C routines: quant codes and scales
    bit for bit, the dense and grouped GEMMs within the bf16 tolerance."""
    import torch
    from tests._util import bf16_bits, quantized_gemm_inputs, seeded_bf16
    x = seeded_bf16((33, 512), seed=5, outlier_frac=1e-2)
    q, s = oracle.torch_quant_group128(x)
    qo, so = oracle.quant_group128(bf16_bits(x))
    assert np.array_equal(q.view(torch.uint8).numpy(), qo) and np.array_equal(s.numpy(), so)
    M, N, K = 17, 256, 384
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=6)
    a = torch.from_numpy(oracle.e4m3_decode(qa) * np.repeat(sa, 128, axis=1)).bfloat16()
    y = oracle.torch_dense_linear(a, torch.from_numpy(qw).view(torch.float8_e4m3fn), torch.from_numpy(sw))
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw)
    assert np.abs(y.float().numpy() - ref).max() <= 1e-2 * np.abs(ref).max()
    ids = np.array([1] * 10 + [-1] * 6 + [0] * 16, dtype=np.int32)
    qa2, sa2, qw2, sw2 = quantized_gemm_inputs(32, 256, 256, seed=7)
    qb = np.stack([qw2[:128], qw2[128:]])
    sb = np.stack([sw2[:1], sw2[1:]])
    got = oracle.torch_grouped_linear(torch.from_numpy(qa2).view(torch.float8_e4m3fn), torch.from_numpy(sa2),
                                      torch.from_numpy(qb).view(torch.float8_e4m3fn), torch.from_numpy(sb),
                                      torch.from_numpy(ids))
    ref2 = oracle.grouped_gemm_nt_sample(qa2, sa2, qb, sb, ids)
    assert sorted(got) == [r for r in range(32) if ids[r] >= 0]
    for r, row in got.items():
        assert np.abs(row.float().numpy() - ref2[r]).max() <= 1e-2 * np.abs(ref2[r]).max() + 1e-6
