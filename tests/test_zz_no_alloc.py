"""GPU check of the allocation-free GEMM entry point kbn_fp8_gemm_nt_noalloc
(no reference counterpart): its split-K slabs live in the library's static
per-GPU scratch instead of a caller workspace.  Two calls in a row, the
second on a smaller input, each compared bit for bit with
kbn_fp8_gemm_nt_ws (same kernels and plan, caller workspace) and with the
float64 oracle to the GEMM tolerance (max relative error <= 1e-2, cosine
>= 0.9999, atol = rtol = 1e-2)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_gemm_close, bf16_bits, quantized_gemm_inputs, to_fp8

pytestmark = pytest.mark.gpu


def _call(L, fn, A, sA, W, sW, D, M, N, K, ws=None):
    args = [A.data_ptr(), K, sA.data_ptr(), 1, M, W.data_ptr(), K, sW.data_ptr(), K // 128,
            D.data_ptr(), N, M, N, K, 1]
    if ws is not None:
        args += [ctypes.c_void_p(ws.data_ptr()) if ws.numel() else None, ws.numel()]
    rc = fn(*args, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.kbn_last_error().decode()


def _inputs(M, N, K, dev, seed):
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=seed)
    A = to_fp8(qa, dev)
    sA = _alloc_colmajor_scale(M, K // 128, dev)
    sA.copy_(torch.from_numpy(sa))
    return qa, sa, qw, sw, A, sA, to_fp8(qw, dev), torch.from_numpy(sw).to(dev)


def test_gemm_noalloc_under_graph_capture(gpu_device):
    """Collected first in this file, so in a fresh process (and after the
    other test files, which never call this entry point) the scratch address
    is looked up inside the capture.  Two split plans (summed in the split
    launch, M = 8; by the separate reduction, M = 64) captured into one graph
    and replayed four times with eager work in between: every replay equals
    the workspace entry point's eager result bit for bit."""
    from kb_nano_amd._lib import lib
    L = lib()
    cases = []
    for M, N, K in ((8, 8192, 8192), (64, 10240, 8192)):
        qa, sa, qw, sw, A, sA, W, sW = _inputs(M, N, K, gpu_device, seed=M + 11)
        ws = torch.empty(L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1), dtype=torch.uint8, device=gpu_device)
        ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        _call(L, L.kbn_fp8_gemm_nt_ws, A, sA, W, sW, ref, M, N, K, ws)
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        cases.append((M, N, K, A, sA, W, sW, ref, out))
    torch.cuda.synchronize()
    print("noalloc GEMM: capturing two split plans", flush=True)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for M, N, K, A, sA, W, sW, ref, out in cases:
                _call(L, L.kbn_fp8_gemm_nt_noalloc, A, sA, W, sW, out, M, N, K)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(4):
        for c in cases:
            c[8].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for M, N, K, A, sA, W, sW, ref, out in cases:
            assert np.array_equal(bf16_bits(out), bf16_bits(ref)), f"replay {rep}: noalloc graph != ws at M={M}"
        # eager calls of the same entry point between replays share the scratch
        M, N, K, A, sA, W, sW, ref, _ = cases[1]
        tmp = torch.empty(M, N, dtype=torch.bfloat16, device=gpu_device)
        _call(L, L.kbn_fp8_gemm_nt_noalloc, A, sA, W, sW, tmp, M, N, K)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(tmp), bf16_bits(ref)), f"eager noalloc after replay {rep}"


def test_gemm_noalloc_matches_workspace_entry_point(gpu_device):
    from kb_nano_amd._lib import lib
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    L = lib()
    assert L.kbn_fp8_gemm_nt_noalloc_scratch_bytes() == 64 << 20
    # first a split tail summed by the separate reduction launch (M = 64),
    # then a smaller one summed inside the split launch (M = 8)
    for M, N, K in ((64, 10240, 8192), (8, 8192, 8192)):
        ws_bytes = L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1)
        assert 0 < ws_bytes <= L.kbn_fp8_gemm_nt_noalloc_scratch_bytes(), (M, N, K, ws_bytes)
        print(f"noalloc GEMM M={M} N={N} K={K} (workspace {ws_bytes} B)", flush=True)
        qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=M + 7)
        A = to_fp8(qa, gpu_device)
        sA = _alloc_colmajor_scale(M, K // 128, gpu_device)
        sA.copy_(torch.from_numpy(sa))
        W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
        D_ws = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        D_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu_device)
        _call(L, L.kbn_fp8_gemm_nt_ws, A, sA, W, sW, D_ws, M, N, K, ws)
        _call(L, L.kbn_fp8_gemm_nt_noalloc, A, sA, W, sW, D_na, M, N, K)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(D_na), bf16_bits(D_ws)), f"noalloc != ws at M={M}"
        cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(M).integers(0, N, 94)]))
        ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=True, cols=cols)
        assert_gemm_close(D_na[:, torch.from_numpy(cols).to(gpu_device)], ref, f"noalloc M={M}")
