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
    from kb_nano_amd import FusedAddRMSNormFP8Quant, RMSNormFP8Quant
    from kb_nano_amd._lib import KbnError
    dev = gpu_device
    with pytest.raises(TypeError):   # fp16 activations are not on this path
        RMSNormFP8Quant()(torch.zeros(4, 256, dtype=torch.float16, device=dev),
                          torch.ones(256, dtype=torch.float16, device=dev))
    with pytest.raises(KbnError, match="multiple of 8"):
        RMSNormFP8Quant()(torch.zeros(4, 260, dtype=torch.bfloat16, device=dev),
                          torch.ones(260, dtype=torch.bfloat16, device=dev))
    with pytest.raises(KbnError, match="at most 8192"):
        FusedAddRMSNormFP8Quant()(torch.zeros(2, 8200, dtype=torch.bfloat16, device=dev),
                                  torch.zeros(2, 8200, dtype=torch.bfloat16, device=dev),
                                  torch.ones(8200, dtype=torch.bfloat16, device=dev))
