"""GPU parity of the load-time weight requant (postprocess_fp8_weights[_batched],
tasks/baseline/L1/fp8_linear.py:453-554) against the oracle's restatement of
the reference's dequant + DeepGEMM per_block_cast_to_fp8: codes and block
scales bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import fp8_codes, to_fp8

pytestmark = pytest.mark.gpu


def _checkpoint(E, N, K, seed):
    rng = np.random.default_rng(seed)
    q = np.empty((E, N, K), np.uint8)
    NB, KB = -(-N // 128), -(-K // 128)
    s = np.empty((E, NB, KB), np.float32)
    for e in range(E):
        w = (rng.standard_normal((N, K)) * rng.uniform(0.005, 0.1)).astype(np.float32)
        q[e], s[e] = oracle.quant_block128(w, use_ue8m0=False)
    s = (s * rng.uniform(0.5, 3.0, s.shape)).astype(np.float32)   # arbitrary fp32 scales
    return q, s


@pytest.mark.parametrize("N,K", [(512, 7168), (200, 208), (130, 512), (4096, 128), (7, 16)])
@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_postprocess_weights_matches_oracle(gpu_device, monkeypatch, N, K, use_ue8m0):
    from kb_nano_amd import fp8_linear, postprocess_fp8_weights
    monkeypatch.setattr(fp8_linear, "is_e8m0_used", lambda: use_ue8m0)
    print(f"postprocess_fp8_weights N={N} K={K} ue8m0={use_ue8m0}", flush=True)
    q, s = _checkpoint(1, N, K, seed=N * 7 + K)
    W, sW = to_fp8(q[0], gpu_device), torch.from_numpy(s[0]).to(gpu_device)
    W2, sW2 = postprocess_fp8_weights(W, sW)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.block_requant(q[0], s[0], use_ue8m0=use_ue8m0)
    assert np.array_equal(sW2.cpu().numpy(), s_ref)
    assert np.array_equal(fp8_codes(W2), q_ref)
    assert np.array_equal(fp8_codes(W), q[0])             # the input is left alone


def test_postprocess_weights_batched_in_place(gpu_device):
    """All experts in one launch, in place, with a scale tensor wider than
    the blocks (the reference slices scale_inv[idx, :rows, :cols]); the extra
    entries are left alone."""
    from kb_nano_amd import postprocess_fp8_weights_batched
    from kb_nano_amd.fp8_linear import is_e8m0_used
    E, N, K = 5, 384, 320
    print(f"postprocess_fp8_weights_batched E={E} N={N} K={K}", flush=True)
    q, s = _checkpoint(E, N, K, seed=11)
    s_wide = np.full((E, 4, 5), 7.0, np.float32)
    s_wide[:, :3, :3] = s
    W = to_fp8(q, gpu_device)
    sW = torch.from_numpy(s_wide).to(gpu_device)
    postprocess_fp8_weights_batched(W, sW)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.block_requant(q, s, use_ue8m0=is_e8m0_used())
    got_s = sW.cpu().numpy()
    assert np.array_equal(got_s[:, :3, :3], s_ref)
    assert np.all(got_s[:, 3:, :] == 7.0) and np.all(got_s[:, :, 3:] == 7.0)
    assert np.array_equal(fp8_codes(W), q_ref)


@pytest.mark.parametrize("use_ue8m0", [True, False])
def test_block_requant_fp32_master_weight(gpu_device, use_ue8m0):
    """fp32 input (the benchmark and test weight builder), with an all-zero
    block, a block holding one huge entry and a block of tiny values."""
    from kb_nano_amd.fp8_linear import _block_requant
    rng = np.random.default_rng(4)
    E, N, K = 2, 300, 272
    x = (rng.standard_normal((E, N, K)) * 0.02).astype(np.float32)
    x[0, 128:256, :128] = 0.0
    x[1, 3, 260] = 5.0e5
    x[1, 256:, :128] *= np.float32(1e-12)
    print(f"block_requant fp32 E={E} N={N} K={K} ue8m0={use_ue8m0}", flush=True)
    q, s = _block_requant(torch.from_numpy(x).to(gpu_device), use_ue8m0=use_ue8m0, eps=1e-4)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.block_requant(x, None, use_ue8m0=use_ue8m0, eps=1e-4)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(fp8_codes(q), q_ref)


def test_block_requant_rejects_bad_shapes(gpu_device):
    from kb_nano_amd import _ops
    from kb_nano_amd._lib import KbnError
    dev = gpu_device
    w = torch.zeros(128, 120, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.ones(1, 1, device=dev)
    with pytest.raises(KbnError, match="multiple of 16"):
        _ops.fp8_block_requant(w, s, w, s, True, 1e-4)
    w = torch.zeros(256, 128, dtype=torch.float8_e4m3fn, device=dev)
    with pytest.raises(ValueError, match=">= 2"):
        _ops.fp8_block_requant(w, s, w, s, True, 1e-4)
