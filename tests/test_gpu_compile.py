"""The swappable modules inside a compiled graph.

kb_nano's kernel_swapper requires candidates that sit inside a
``torch.compile`` graph to compile without graph breaks
(infra/kernel_swapper.py:503-513).  Each module is compiled with
``fullgraph=True`` (a graph break raises) on the ``aot_eager`` backend, which
traces the opaque custom ops through their Meta implementations and then runs
the same gfx950 kernels, so the outputs must equal eager execution bit for
bit."""
import numpy as np
import pytest
import torch

from tests._util import bf16_bits, fp8_codes, quantized_gemm_inputs, to_fp8

pytestmark = pytest.mark.gpu


def _compiled(fn):
    torch._dynamo.reset()
    return torch.compile(fn, fullgraph=True, backend="aot_eager")


@pytest.mark.parametrize("M", [8, 256])
def test_fp8_linear_compiles_without_graph_breaks(gpu_device, M):
    from kb_nano_amd import Fp8Linear
    print(f"compile Fp8Linear M={M}", flush=True)
    N, K = 512, 1024
    _, _, qw, sw = quantized_gemm_inputs(M, N, K, seed=M)
    W, sW = to_fp8(qw, gpu_device), torch.from_numpy(sw).to(gpu_device)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(2, M // 2, K, generator=g).bfloat16().to(gpu_device)
    bias = torch.randn(N, generator=g).bfloat16().to(gpu_device)
    lin = Fp8Linear()
    ref = lin(x, W, sW, bias).clone()
    got = _compiled(lambda a: lin(a, W, sW, bias))(x)
    torch.cuda.synchronize()
    assert got.shape == (2, M // 2, N)
    assert np.array_equal(bf16_bits(got), bf16_bits(ref))


def test_quant_modules_compile_without_graph_breaks(gpu_device):
    from kb_nano_amd import PerTokenGroupQuantFp8, SiluMulQuantFp8
    from kb_nano_amd.fp8_linear import _alloc_colmajor_scale
    print("compile quant modules", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(128, 1024, generator=g).bfloat16().to(gpu_device)
    silu = SiluMulQuantFp8()
    q0, s0 = silu(x)
    q1, s1 = _compiled(lambda a: silu(a))(x)
    torch.cuda.synchronize()
    assert np.array_equal(fp8_codes(q1), fp8_codes(q0)) and torch.equal(s1, s0)
    assert s1.stride() == s0.stride()

    quant = PerTokenGroupQuantFp8()
    qa, sa = torch.empty(128, 1024, dtype=torch.float8_e4m3fn, device=gpu_device), _alloc_colmajor_scale(128, 8, gpu_device)
    qb, sb = torch.empty_like(qa), _alloc_colmajor_scale(128, 8, gpu_device)
    quant(x, qa, sa)

    def run(a):
        quant(a, qb, sb)
        return qb, sb
    _compiled(run)(x)
    torch.cuda.synchronize()
    assert np.array_equal(fp8_codes(qb), fp8_codes(qa)) and torch.equal(sb, sa)


def test_grouped_gemm_and_norm_compile_without_graph_breaks(gpu_device):
    from kb_nano_amd import Fp8GroupedGemmContiguous, RMSNormFP8Quant
    print("compile grouped gemm and rmsnorm", flush=True)
    E, N, K, rows = 2, 768, 512, 256
    qa, sa, _, _ = quantized_gemm_inputs(rows, N, K, seed=11)
    A, sA = to_fp8(qa, gpu_device), torch.from_numpy(sa).to(gpu_device)
    ws, ss = [], []
    for e in range(E):
        _, _, qw, sw = quantized_gemm_inputs(1, N, K, seed=20 + e)
        ws.append(to_fp8(qw, gpu_device))
        ss.append(torch.from_numpy(sw).to(gpu_device))
    B, sB = torch.stack(ws), torch.stack(ss)
    ids = torch.tensor([0] * 128 + [1] * 100 + [-1] * 28, dtype=torch.int32, device=gpu_device)
    mod = Fp8GroupedGemmContiguous()
    c0 = torch.zeros(rows, N, dtype=torch.bfloat16, device=gpu_device)
    c1 = torch.zeros_like(c0)
    mod(A, sA, B, sB, c0, ids)

    def run(a):
        mod(a, sA, B, sB, c1, ids)
        return c1
    _compiled(run)(A)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(c1), bf16_bits(c0))

    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 7168, generator=g).bfloat16().to(gpu_device)
    w = torch.randn(7168, generator=g).bfloat16().to(gpu_device)
    norm = RMSNormFP8Quant()
    q0, s0 = norm(x, w, 1e-6)
    q1, s1 = _compiled(lambda a: norm(a, w, 1e-6))(x)
    torch.cuda.synchronize()
    assert np.array_equal(fp8_codes(q1), fp8_codes(q0)) and torch.equal(s1, s0)


def test_fused_add_norm_compiles_and_mutates_in_place(gpu_device):
    """The fused residual-add variant writes its two bf16 inputs in place; under
    the compiled graph the same buffers must end up with the same bits."""
    from kb_nano_amd import FusedAddRMSNormFP8Quant
    print("compile fused add rmsnorm", flush=True)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(64, 7168, generator=g).bfloat16().to(gpu_device)
    r = (torch.randn(64, 7168, generator=g) * 4).bfloat16().to(gpu_device)
    w = torch.randn(7168, generator=g).bfloat16().to(gpu_device)
    norm = FusedAddRMSNormFP8Quant()
    x0, r0 = x.clone(), r.clone()
    q0, s0, _ = norm(x0, r0, w, 1e-6)
    x1, r1 = x.clone(), r.clone()
    q1, s1, r_ret = _compiled(lambda a, b: norm(a, b, w, 1e-6))(x1, r1)
    torch.cuda.synchronize()
    assert np.array_equal(fp8_codes(q1), fp8_codes(q0)) and torch.equal(s1, s0)
    assert np.array_equal(bf16_bits(x1), bf16_bits(x0)) and np.array_equal(bf16_bits(r1), bf16_bits(r0))
    assert np.array_equal(bf16_bits(r_ret), bf16_bits(r0))
