"""GPU parity of the quant kernels against the C oracle: bit-exact codes and
scales (tasks/baseline/L1/fp8_linear.py:181-215,
tasks/baseline/L1/silu_mul_quant_fp8.py:23-143)."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf16_bits, fp8_codes, from_bits, seeded_bf16

pytestmark = pytest.mark.gpu


def _quant_gpu(x, col_major=False, use_ue8m0=True, eps=1e-10):
    from kb_nano_amd import _ops
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=x.device)
    s = _alloc_colmajor_scale(M, K // 128, x.device) if col_major else \
        torch.empty(M, K // 128, dtype=torch.float32, device=x.device)
    _ops.per_token_group_quant_fp8(x, q, s, use_ue8m0=use_ue8m0, eps=eps)
    torch.cuda.synchronize()
    return q, s


def test_e4m3_conversion_exhaustive(gpu_device):
    """Groups whose absmax is exactly 448 get scale 1, so q = e4m3(x): every
    finite bf16 value in [-448, 448] goes through the hardware convert."""
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = oracle.bf16_bits_to_f32(allb)
    keep = np.isfinite(vals) & (np.abs(vals) <= 448.0)
    pool = allb[keep]
    per = 127
    G = -(-len(pool) // per)
    pool = np.concatenate([pool, np.zeros(G * per - len(pool), dtype=np.uint16)])
    x = np.empty((G, 128), dtype=np.uint16)
    x[:, 0] = 0x43E0  # 448.0
    x[:, 1:] = pool.reshape(G, per)
    x = x.reshape(-1, 1024) if G % 8 == 0 else x.reshape(G, 128)
    qo, so = oracle.quant_group128(x)
    assert np.all(so == 1.0)
    q, s = _quant_gpu(from_bits(x, gpu_device))
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)


@pytest.mark.parametrize("M,K", [(1, 128), (3, 2048), (64, 2048), (130, 7168), (257, 1536), (8, 28672)])
@pytest.mark.parametrize("col_major", [False, True])
def test_quant_matches_oracle(gpu_device, M, K, col_major):
    x = seeded_bf16((M, K), seed=M * 7 + K, outlier_frac=1e-3)
    if M > 2:
        x[1, :] = 0            # all-zero groups -> 2^-42
        x[2, :128] = 1e-38     # subnormal-range inputs
    qo, so = oracle.quant_group128(bf16_bits(x))
    q, s = _quant_gpu(x.to(gpu_device), col_major=col_major)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)
    if col_major:
        assert s.stride() == (1, M)


def test_quant_plain_fp32_scales(gpu_device):
    x = seeded_bf16((96, 1024), seed=11, outlier_frac=1e-2)
    qo, so = oracle.quant_group128(bf16_bits(x), use_ue8m0=False)
    q, s = _quant_gpu(x.to(gpu_device), use_ue8m0=False)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)


def test_quant_strided_rows(gpu_device):
    big = seeded_bf16((40, 1024 + 256), seed=3).to(gpu_device)
    x = big[:, 128:1152]
    assert x.stride(0) == 1280
    qo, so = oracle.quant_group128(bf16_bits(x))
    q, s = _quant_gpu(x)
    assert np.array_equal(fp8_codes(q), qo) and np.array_equal(s.cpu().numpy(), so)


def test_quant_module_and_op(gpu_device):
    from kb_nano_amd import PerTokenGroupQuantFp8
    x = seeded_bf16((33, 512), seed=5).to(gpu_device)
    q = torch.empty(33, 512, dtype=torch.float8_e4m3fn, device=gpu_device)
    s = torch.empty(33, 4, dtype=torch.float32, device=gpu_device)
    PerTokenGroupQuantFp8()(x.t().contiguous().t(), q, s)   # non-contiguous input is made contiguous
    torch.cuda.synchronize()
    qo, so = oracle.quant_group128(bf16_bits(x))
    assert np.array_equal(fp8_codes(q), qo) and np.array_equal(s.cpu().numpy(), so)


def test_quant_rejects_bad_args(gpu_device):
    from kb_nano_amd import _ops
    x = torch.zeros(4, 200, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError):
        _ops.per_token_group_quant_fp8(x, torch.empty(4, 200, dtype=torch.float8_e4m3fn, device=gpu_device),
                                       torch.empty(4, 2, device=gpu_device))
    with pytest.raises(RuntimeError):
        _ops.per_token_group_quant_fp8(x.cpu(), torch.empty(4, 200, dtype=torch.float8_e4m3fn),
                                       torch.empty(4, 2))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 128), (3, 2048), (130, 7168), (257, 1536)])
@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_quant_fp16_fp32_inputs_match_oracle(gpu_device, dtype, M, K, use_ue8m0):
    """fp16 and fp32 rows (kbn_per_token_group_quant_fp8_typed): codes and
    scales bit-exact against the oracle's quant of the same values, with
    zero rows, each type's subnormals and values near its max; column-major
    scales on every other shape."""
    print(f"quant {dtype} M={M} K={K} ue8m0={use_ue8m0}", flush=True)
    g = torch.Generator().manual_seed(M * 3 + K)
    x = torch.randn(M, K, generator=g)
    x = torch.where(torch.rand(M, K, generator=g) < 1e-3, x * 50, x)
    if M > 2:
        x[1, :] = 0
        x[2, :128] = torch.randn(128, generator=g) * (3e-7 if dtype == torch.float16 else 1e-39)
        x[2, 128:] = torch.randn(K - 128, generator=g) * (6.0e4 / 8 if dtype == torch.float16 else 3e37)
    x = x.to(dtype)
    qo, so = oracle.quant_group128_f32(x.numpy(), use_ue8m0=use_ue8m0)
    q, s = _quant_gpu(x.to(gpu_device), col_major=(M % 2 == 1), use_ue8m0=use_ue8m0)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quant_fp16_fp32_nonfinite_groups(gpu_device, dtype):
    """fp16 / fp32 groups holding +-inf or NaN follow the bf16 kernel's rules
    (NaN ignored by the absmax, an infinite absmax gives an infinite scale,
    finite values then code to +-0): equal to the oracle up to the NaN
    code's sign bit, and to the bf16 kernel on the same (bf16) values."""
    x = seeded_bf16((16, 1024), seed=22).float().numpy()
    x[0, 5] = np.inf
    x[1, 130] = -np.inf
    x[2, 300] = np.nan
    x[3, :128] = np.nan
    x[4, 513] = np.inf
    x[4, 514] = np.nan
    x[5, 640:768] = np.inf
    xt = torch.from_numpy(x).to(dtype)
    qo, so = oracle.quant_group128_f32(xt.numpy())
    q, s = _quant_gpu(xt.to(gpu_device))
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(_canon_nan(fp8_codes(q)), _canon_nan(qo))
    qb, sb = _quant_gpu(torch.from_numpy(x).bfloat16().to(gpu_device))
    assert np.array_equal(fp8_codes(q), fp8_codes(qb)) and torch.equal(s, sb)


def test_quant_module_and_op_fp16_fp32(gpu_device):
    """The module and the registered op take fp16 / fp32 input as the
    reference's do; a dtype outside bf16 / fp16 / fp32 is rejected."""
    from kb_nano_amd import PerTokenGroupQuantFp8, _ops
    for dtype in (torch.float16, torch.float32):
        x = torch.randn(40, 384, generator=torch.Generator().manual_seed(6)).to(dtype)
        qo, so = oracle.quant_group128_f32(x.numpy())
        for call in (lambda xx, qq, ss: PerTokenGroupQuantFp8()(xx, qq, ss),
                     lambda xx, qq, ss: torch.ops.kb_nano_fp8.per_token_group_quant_fp8(xx, qq, ss, False)):
            q = torch.empty(40, 384, dtype=torch.float8_e4m3fn, device=gpu_device)
            s = torch.empty(40, 3, dtype=torch.float32, device=gpu_device)
            call(x.to(gpu_device), q, s)
            torch.cuda.synchronize()
            assert np.array_equal(fp8_codes(q), qo) and np.array_equal(s.cpu().numpy(), so)
    with pytest.raises(TypeError):
        _ops.per_token_group_quant_fp8(torch.zeros(4, 128, dtype=torch.float64, device=gpu_device),
                                       torch.empty(4, 128, dtype=torch.float8_e4m3fn, device=gpu_device),
                                       torch.empty(4, 1, device=gpu_device))


def test_quant_empty(gpu_device):
    q, s = _quant_gpu(torch.empty(0, 256, dtype=torch.bfloat16, device=gpu_device))
    assert q.shape == (0, 256) and s.shape == (0, 2)


# ------------------------------------------------------------ SiLU + quant

@pytest.mark.parametrize("path", [0, 1])
def test_silu_exhaustive(gpu_device, path):
    """All 65,536 bf16 gate values through the kernels' silu vs the oracle's
    correctly rounded table (itself pinned against 50-digit decimal): path 0
    the table as the SiLU*Mul + quant kernels read it, path 1 at the symbol
    address the grouped GEMM's SiLU*Mul epilogue reads (every pattern,
    infinities and NaNs included, the same bits)."""
    from kb_nano_amd import _ops
    g = torch.arange(65536, dtype=torch.int32).to(torch.int16).to(gpu_device)
    out = torch.empty_like(g)
    _ops.debug_silu_bf16(g, out, path=path)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.uint16)
    want = oracle.silu_bf16_table()
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (allb & 0x7F80) != 0x7F80
    mism = np.nonzero((got != want) & finite)[0]
    assert mism.size == 0, [(hex(i), hex(got[i]), hex(want[i])) for i in mism[:10]]
    if path == 1:
        table = torch.empty_like(g)
        _ops.debug_silu_bf16(g, table, path=0)
        torch.cuda.synchronize()
        assert torch.equal(out, table)


def _silu_gpu(inp, col_major=True, use_ue8m0=True):
    from kb_nano_amd import _ops
    M, N = inp.shape
    q = torch.empty(M, N // 2, dtype=torch.float8_e4m3fn, device=inp.device)
    s = torch.empty(N // 256, M, dtype=torch.float32, device=inp.device).t() if col_major else \
        torch.empty(M, N // 256, dtype=torch.float32, device=inp.device)
    _ops.silu_mul_quant_fp8(inp, q, s, use_ue8m0=use_ue8m0)
    torch.cuda.synchronize()
    return q, s


@pytest.mark.parametrize("M,Nh", [(8, 128), (128, 1024), (136, 2048), (256, 4608)])
@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_silu_mul_quant_matches_oracle(gpu_device, M, Nh, use_ue8m0):
    x = seeded_bf16((M, 2 * Nh), seed=M + Nh, outlier_frac=1e-3)
    x[0, :Nh] = 0.0
    # tiny gate and up values: fp32-subnormal products must round like IEEE
    x[1] = (x[1].float() * 1e-19).bfloat16()
    if M > 2:
        x[2, Nh:] = (x[2, Nh:].float() * 3e-38).bfloat16()
    qo, so = oracle.silu_mul_quant(bf16_bits(x), use_ue8m0=use_ue8m0)
    q, s = _silu_gpu(x.to(gpu_device), use_ue8m0=use_ue8m0)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)


def test_silu_mul_quant_module(gpu_device):
    from kb_nano_amd import SiluMulQuantFp8
    x = seeded_bf16((128, 1024), seed=21, outlier_frac=1e-3).to(gpu_device)
    out = torch.empty(128, 512, dtype=torch.float8_e4m3fn, device=gpu_device)
    q, s = SiluMulQuantFp8()(x, output=out)
    torch.cuda.synchronize()
    assert q.data_ptr() == out.data_ptr()
    assert s.shape == (128, 4) and s.stride() == (1, 128)
    qo, so = oracle.silu_mul_quant(bf16_bits(x))
    assert np.array_equal(fp8_codes(q), qo) and np.array_equal(s.cpu().numpy(), so)
    with pytest.raises(AssertionError):
        SiluMulQuantFp8()(x[:100])   # M % 128 != 0, as the reference asserts


@pytest.mark.parametrize("M,Nh,tail", [(384, 512, 0.0), (1000, 384, 0.3), (4096, 2048, 0.25)])
def test_silu_mul_quant_skips_rows_with_negative_ids(gpu_device, M, Nh, tail):
    """Row ids (the contiguous MoE layout's expert ids, as FusedExperts
    passes them): rows whose id is negative are neither read nor written
    (their codes and scales keep a sentinel); every other row is bit-exact
    against the oracle.  Ragged M (not a multiple of the 32-row blocks the
    rows are dealt in) and a skipped tail, as the layout's unused rows."""
    from kb_nano_amd import _ops
    x = seeded_bf16((M, 2 * Nh), seed=M + 3, outlier_frac=1e-3)
    g = torch.Generator().manual_seed(M)
    ids = torch.randint(0, 256, (M,), generator=g, dtype=torch.int32)
    ids[torch.rand(M, generator=g) < 0.45] = -1
    ids[:3] = -1   # a run at the start, and the last row too
    ids[-1] = -1
    ids[M - int(tail * M):] = -1
    keep = (ids >= 0).numpy()
    qo, so = oracle.silu_mul_quant(bf16_bits(x))
    xd, idd = x.to(gpu_device), ids.to(gpu_device)
    q = torch.full((M, Nh), 0x55, dtype=torch.uint8, device=gpu_device).view(torch.float8_e4m3fn)
    s = torch.full((Nh // 128, M), -3.0, device=gpu_device).t()
    _ops.silu_mul_quant_fp8(xd, q, s, row_ids=idd)
    torch.cuda.synchronize()
    qc, sc = fp8_codes(q), s.cpu().numpy()
    assert np.array_equal(qc[keep], qo[keep])
    assert np.array_equal(sc[keep], so[keep])
    assert (qc[~keep] == 0x55).all(), "a skipped row was written"
    assert (sc[~keep] == -3.0).all(), "a skipped row's scales were written"


def test_silu_mul_quant_cfg2_full(gpu_device):
    """BASELINE config 2 at full size: [8192, 36864] bf16 with 0.1% x50
    outliers, checked bit-exact against the oracle on every row."""
    M, Nh = 8192, 18432
    x = seeded_bf16((M, 2 * Nh), seed=1, outlier_frac=1e-3)
    xb = bf16_bits(x)
    q, s = _silu_gpu(x.to(gpu_device))
    del x
    qo, so = oracle.silu_mul_quant(xb)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(fp8_codes(q), qo)


# ------------------------------------------------------------ golden fixtures

def test_quant_golden_fixture(gpu_device):
    """The committed edge-case fixture (tests/golden/quant_edge.npz), both
    scale contracts, bit-exact."""
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_edge.npz"), allow_pickle=False)
    x = from_bits(d["x_bits"], gpu_device)
    for ue8m0, qk, sk in ((True, "q_ue8m0", "s_ue8m0"), (False, "q_fp32", "s_fp32")):
        q, s = _quant_gpu(x, col_major=True, use_ue8m0=ue8m0)
        assert np.array_equal(fp8_codes(q), d[qk]) and np.array_equal(s.cpu().numpy(), d[sk])


def test_silu_mul_quant_golden_fixture(gpu_device):
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "silu_mul_quant.npz"), allow_pickle=False)
    x = from_bits(d["x_bits"], gpu_device)
    for ue8m0, qk, sk in ((True, "q_ue8m0", "s_ue8m0"), (False, "q_fp32", "s_fp32")):
        q, s = _silu_gpu(x, use_ue8m0=ue8m0)
        assert np.array_equal(fp8_codes(q), d[qk]) and np.array_equal(s.cpu().numpy(), d[sk])


def _canon_nan(codes: np.ndarray) -> np.ndarray:
    """e4m3fn has two NaN codes (0x7F, 0xFF); gfx950's conversion always
    gives 0xFF, the oracle keeps the sign.  Both mean NaN."""
    c = codes.copy()
    c[(c & 0x7F) == 0x7F] = 0xFF
    return c


def test_quant_nonfinite_groups(gpu_device):
    """Groups holding +-inf or NaN: the absmax ignores NaN (the reference's
    max), an infinite absmax gives an infinite scale and then codes +-0 for
    the group's finite values (x / inf) and NaN for the rest; a group of
    only NaN gets the eps scale.  Codes equal the oracle's up to the NaN
    code's sign bit."""
    x = seeded_bf16((16, 1024), seed=21).float().numpy()
    x[0, 5] = np.inf
    x[1, 130] = -np.inf
    x[2, 300] = np.nan
    x[3, :128] = np.nan
    x[4, 513] = np.inf
    x[4, 514] = np.nan
    x[5, 640:768] = np.inf
    x[6, 900] = -np.inf
    x[6, 901] = np.inf
    bits = oracle.f32_to_bf16_bits(x)
    qo, so = oracle.quant_group128(bits)
    q, s = _quant_gpu(from_bits(bits, gpu_device))
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(_canon_nan(fp8_codes(q)), _canon_nan(qo))
    assert np.isinf(so[0, 0]) and np.all(qo[0, :128][np.isfinite(x[0, :128])] & 0x7F == 0)


def test_silu_mul_quant_nonfinite(gpu_device):
    """SiLU*Mul + quant with infinite and NaN gates and ups (silu(inf) = inf,
    silu(-inf) = -0, inf * 0 = NaN): codes equal the oracle's up to the NaN
    code's sign bit, scales exactly."""
    from kb_nano_amd import _ops
    M, Nh = 8, 512
    x = seeded_bf16((M, 2 * Nh), seed=23).float().numpy()
    x[0, 3] = np.inf                 # gate inf, up finite
    x[1, 200] = -np.inf              # gate -inf -> silu -0
    x[2, 7] = np.inf
    x[2, Nh + 7] = 0.0               # inf * 0 -> NaN
    x[3, Nh + 100] = np.nan          # up NaN
    x[4, 260] = np.nan               # gate NaN
    x[5, Nh + 400] = -np.inf         # up -inf
    bits = oracle.f32_to_bf16_bits(x)
    qo, so = oracle.silu_mul_quant(bits)
    inp = from_bits(bits, gpu_device)
    q = torch.empty(M, Nh, dtype=torch.float8_e4m3fn, device=gpu_device)
    s = torch.empty(Nh // 128, M, device=gpu_device).t()
    _ops.silu_mul_quant_fp8(inp, q, s)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(_canon_nan(fp8_codes(q)), _canon_nan(qo))
