"""GPU parity of the fused RMSNorm (+ residual add) + 1x128 FP8 quant
(tasks/baseline/L1/rmsnorm_quant.py, csrc/rmsnorm_quant.cu:21-201) against the
oracle, which evaluates the same fp32 operations in the kernel's order: codes,
scales, the updated residual and the normalized row are compared bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf16_bits, fp8_codes, from_bits

pytestmark = pytest.mark.gpu


def _inputs(M, H, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, H, generator=g) * scale).bfloat16()
    w = torch.randn(H, generator=g).bfloat16()
    r = (torch.randn(M, H, generator=g) * 4).bfloat16()
    return x, w, r


@pytest.mark.parametrize("M,H", [(1, 7168), (7, 4096), (128, 3584), (300, 8192), (5, 200), (64, 16384),
                                 (33, 1024), (4096, 7168)])
def test_rmsnorm_quant_matches_oracle(gpu_device, M, H):
    from kb_nano_amd import RMSNormFP8Quant
    dev = gpu_device
    print(f"rmsnorm_quant M={M} H={H}", flush=True)
    x, w, _ = _inputs(M, H, seed=M + H)
    q, s = RMSNormFP8Quant()(x.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    G = -(-H // 128)
    assert q.shape == (M, H) and s.shape == (M, G) and s.stride() == (1, M)
    q_ref, s_ref = oracle.rmsnorm_quant(bf16_bits(x), bf16_bits(w), eps=1e-6)
    assert np.array_equal(fp8_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("M,H", [(1, 7168), (9, 4096), (128, 8192), (3, 200), (256, 2048)])
def test_fused_add_rmsnorm_quant_matches_oracle(gpu_device, M, H):
    from kb_nano_amd import FusedAddRMSNormFP8Quant
    dev = gpu_device
    print(f"fused_add_rmsnorm_quant M={M} H={H}", flush=True)
    x, w, r = _inputs(M, H, seed=2 * M + H)
    xd, rd = x.to(dev), r.to(dev)
    q, s, r_ret = FusedAddRMSNormFP8Quant()(xd, rd, w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert r_ret is rd
    q_ref, s_ref, r_ref, x_ref = oracle.rmsnorm_quant(bf16_bits(x), bf16_bits(w), eps=1e-6,
                                                      residual_bits=bf16_bits(r))
    assert np.array_equal(bf16_bits(rd), r_ref)        # residual <- residual + input
    assert np.array_equal(bf16_bits(xd), x_ref)        # input <- normalized row
    assert np.array_equal(fp8_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


def test_rmsnorm_quant_edge_rows(gpu_device):
    """Zero rows (inv = 1/sqrt(eps), every group at the 1e-10 floor), huge and
    tiny magnitudes, a row with a single non-zero element, and rows with a NaN
    or an infinity (inv becomes NaN or 0; the reference's fminf/fmaxf clamp
    sends NaN quotients to -448, as the kernel's v_med3_f32 does)."""
    dev = gpu_device
    H = 1024
    nan_row = np.linspace(-3, 3, H).astype(np.float32)
    nan_row[5] = np.nan
    inf_row = np.linspace(-3, 3, H).astype(np.float32)
    inf_row[700] = np.inf
    rows = [np.zeros(H, np.float32),
            np.full(H, 1e30, np.float32),            # squares overflow: inv = 0
            np.full(H, 1e-30, np.float32),           # squares underflow: inv = 1/sqrt(eps)
            np.eye(1, H, 77, dtype=np.float32)[0] * 5.0,
            nan_row, inf_row]
    xb = oracle.f32_to_bf16_bits(np.stack(rows))
    wb = oracle.f32_to_bf16_bits(np.linspace(-2, 2, H).astype(np.float32))
    q = torch.empty(len(rows), H, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(H // 128, len(rows), device=dev).t()
    torch.ops.kb_nano_norm.rmsnorm_fp8_quant(q, s, from_bits(xb, dev), from_bits(wb, dev), 1e-6)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.rmsnorm_quant(xb, wb, eps=1e-6)
    assert np.array_equal(fp8_codes(q), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_rmsnorm_quant_op_on_3d_input(gpu_device):
    """The ops take [..., H] inputs (tokens = numel / H), as the reference does."""
    dev = gpu_device
    x, w, _ = _inputs(24, 2048, seed=9)
    x3 = x.view(2, 12, 2048).to(dev)
    q = torch.empty(24, 2048, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(16, 24, device=dev).t()
    torch.ops.kb_nano_norm.rmsnorm_fp8_quant(q, s, x3, w.to(dev), 1e-5)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.rmsnorm_quant(bf16_bits(x), bf16_bits(w), eps=1e-5)
    assert np.array_equal(fp8_codes(q), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_rmsnorm_quant_rejects_off_path_inputs(gpu_device):
    from kb_nano_amd import RMSNormFP8Quant
    from kb_nano_amd._lib import KbnError
    dev = gpu_device
    with pytest.raises(TypeError):   # float64 is not a type the reference dispatches
        RMSNormFP8Quant()(torch.zeros(4, 256, dtype=torch.float64, device=dev),
                          torch.ones(256, dtype=torch.float64, device=dev))
    with pytest.raises(TypeError, match="dtype"):   # weight of another type than the input
        RMSNormFP8Quant()(torch.zeros(4, 256, dtype=torch.float16, device=dev),
                          torch.ones(256, dtype=torch.bfloat16, device=dev))
    with pytest.raises(KbnError, match="multiple of 8"):
        RMSNormFP8Quant()(torch.zeros(4, 260, dtype=torch.bfloat16, device=dev),
                          torch.ones(260, dtype=torch.bfloat16, device=dev))


_NP = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _check_typed(x, w, r, dev, eps=1e-6):
    """Run the module (fused add when r is given) on x, w (and r) of one
    dtype and compare codes, scales, the residual and the normalized row
    bit for bit with the typed oracle."""
    from kb_nano_amd import FusedAddRMSNormFP8Quant, RMSNormFP8Quant
    dt = _NP[x.dtype]
    f = lambda t: t.float().numpy()
    if r is None:
        q, s = RMSNormFP8Quant()(x.to(dev), w.to(dev), eps)
        torch.cuda.synchronize()
        q_ref, s_ref = oracle.rmsnorm_quant_values(f(x), f(w), dt, eps=eps)
    else:
        xd, rd = x.to(dev), r.to(dev)
        q, s, _ = FusedAddRMSNormFP8Quant()(xd, rd, w.to(dev), eps)
        torch.cuda.synchronize()
        q_ref, s_ref, r_ref, x_ref = oracle.rmsnorm_quant_values(f(x), f(w), dt, eps=eps, residual=f(r))
        assert rd.dtype == x.dtype and xd.dtype == x.dtype
        assert np.array_equal(f(rd.cpu()), r_ref, equal_nan=True)
        assert np.array_equal(f(xd.cpu()), x_ref, equal_nan=True)
    assert np.array_equal(fp8_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,H", [(3, 200), (17, 4096), (64, 7168), (5, 20480), (4, 8200), (2, 16392)])
@pytest.mark.parametrize("add", [False, True])
def test_rmsnorm_quant_any_dtype_and_size(gpu_device, dtype, M, H, add):
    """fp16 / fp32 rows and rows longer than the register-resident kernel's
    (bf16 past 16384 columns, or 8192 with the residual add) take the
    two-pass kernel: bit for bit against the typed oracle, in the same
    summation order as the bf16 kernel (whose cases below 8192 / 16384
    columns this also runs)."""
    print(f"rmsnorm typed {dtype} M={M} H={H} add={add}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + H + add)
    x = torch.randn(M, H, generator=g).to(dtype)
    w = torch.randn(H, generator=g).to(dtype)
    r = (torch.randn(M, H, generator=g) * 4).to(dtype) if add else None
    _check_typed(x, w, r, gpu_device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_rmsnorm_quant_typed_edge_rows(gpu_device, dtype):
    """Zero rows, squares that overflow or underflow fp32, a single non-zero
    element, NaN and infinity rows, and weights so large that a group's
    absmax overflows (an infinite scale: finite values code to +-0, as the
    reference's v / inf; the bf16 case runs the register-resident kernel)."""
    H = 1024
    rows = [np.zeros(H, np.float32), np.full(H, 1e30 if dtype != torch.float16 else 6e4, np.float32),
            np.full(H, 1e-30 if dtype != torch.float16 else 1e-7, np.float32),
            np.eye(1, H, 77, dtype=np.float32)[0] * 5.0]
    nan_row = np.linspace(-3, 3, H).astype(np.float32)
    nan_row[5] = np.nan
    inf_row = np.linspace(-3, 3, H).astype(np.float32)
    inf_row[700] = np.inf
    rows += [nan_row, inf_row, np.linspace(-3, 3, H).astype(np.float32)]
    x = torch.from_numpy(np.stack(rows)).to(dtype)
    w = np.linspace(-2, 2, H).astype(np.float32)
    w[130] = 6e4 if dtype == torch.float16 else 3e38      # group 1's absmax overflows where x is not small
    _check_typed(x, torch.from_numpy(w).to(dtype), None, gpu_device)




def test_fused_add_rounding_edge_cases(gpu_device):
    """The residual sums r + x are rounded to bf16 once (nearest even) and the
    rounded values are what gets normalized: ties at 1 + k 2^-8 (odd k ties,
    even k exact), sums k 2^-133 that are fp32 denormals (kept, not flushed),
    sums just below and above the bf16 overflow threshold, and a random row.  Residual, normalized row, codes and scales
    equal the oracle bit for bit."""
    from kb_nano_amd import FusedAddRMSNormFP8Quant
    dev = gpu_device
    H = 1024
    rng = np.random.default_rng(5)
    f32 = np.float32
    rows_x, rows_r = [], []
    k = np.arange(H) % 16
    sign = np.where(rng.random(H) < 0.5, f32(-1), f32(1))
    rows_r.append(sign * f32(1.0))
    rows_x.append(sign * (k * f32(2.0 ** -8)).astype(np.float32))
    tiny = f32(2.0 ** -126)
    kk = (np.arange(H) % 8).astype(np.float32)
    rows_r.append(sign * tiny)
    rows_x.append(-sign * (tiny - kk * f32(2.0 ** -133)))   # sums k 2^-133: fp32 denormals, exact in bf16
    bf = lambda a: torch.from_numpy(np.asarray(a, np.float32)).bfloat16().float().numpy()
    big = bf(np.full(H, 1.69e38))   # sums 3.38e38 (finite) to 3.44e38 (fp32 overflow)
    rows_r.append(big * sign)
    rows_x.append(bf(1.69e38 + (np.arange(H) % 4) * 0.01e38) * sign)
    rows_r.append(bf(rng.standard_normal(H) * 4))
    rows_x.append(bf(rng.standard_normal(H)))
    to_bits = lambda a: torch.from_numpy(np.stack(a)).bfloat16()
    x, r = to_bits(rows_x), to_bits(rows_r)
    # the inputs must themselves be exact bf16 values (the sums are what is tested)
    assert torch.equal(x.float(), torch.from_numpy(np.stack(rows_x)))
    w = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).bfloat16()
    xd, rd = x.to(dev), r.to(dev)
    q, s, _ = FusedAddRMSNormFP8Quant()(xd, rd, w.to(dev), 1e-6)
    torch.cuda.synchronize()
    q_ref, s_ref, r_ref, x_ref = oracle.rmsnorm_quant(bf16_bits(x), bf16_bits(w), eps=1e-6,
                                                      residual_bits=bf16_bits(r))
    assert np.array_equal(bf16_bits(rd), r_ref)
    assert np.array_equal(bf16_bits(xd), x_ref)
    assert np.array_equal(fp8_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref, equal_nan=True)
