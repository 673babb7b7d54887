"""CPU-side checks of the C-ABI library and the host layer (no GPU needed):
the library loads, exports every symbol include/kbn_fp8.h declares, and
rejects bad arguments with an error code and message before touching a
device."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kbn_fp8.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(kbn_\w+)\s*\(", text)))


def test_header_declares_the_path():
    names = _declared()
    for n in ("kbn_per_token_group_quant_fp8", "kbn_silu_mul_quant_fp8", "kbn_fp8_gemm_nt",
              "kbn_fp8_grouped_gemm_nt_contiguous", "kbn_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from kb_nano_amd._lib import SIGNATURES, lib
    L = lib()
    for name in _declared():
        assert hasattr(L, name), name
        assert name in SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version():
    from kb_nano_amd._lib import ABI_VERSION, lib
    assert lib().kbn_abi_version() == ABI_VERSION


def _err():
    from kb_nano_amd._lib import lib
    return lib().kbn_last_error().decode()


def test_quant_rejects_ragged_k_without_device():
    from kb_nano_amd._lib import lib
    rc = lib().kbn_per_token_group_quant_fp8(None, 4, 100, 100, None, 100, None, 1, 1, 1e-10, 1, None)
    assert rc == 1 and "multiple of 128" in _err()


def test_typed_quant_rejects_bad_arguments_without_device():
    """The fp16 / fp32 quant entry validates before any device call: an
    unknown dtype code, a ragged K, misaligned rows; empty input is a no-op."""
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert L.kbn_per_token_group_quant_fp8_typed(p, 3, 4, 128, 128, p, 128, p, 1, 1, 1e-10, 1, None) == 1
    assert "dtype code 3" in _err()
    assert L.kbn_per_token_group_quant_fp8_typed(p, 2, 4, 100, 100, p, 100, p, 1, 1, 1e-10, 1, None) == 1
    assert "multiple of 128" in _err()
    assert L.kbn_per_token_group_quant_fp8_typed(p, 1, 4, 128, 132, p, 128, p, 1, 1, 1e-10, 1, None) == 1
    assert "16-byte" in _err()
    assert L.kbn_per_token_group_quant_fp8_typed(None, 2, 0, 128, 128, None, 128, None, 1, 1, 1e-10, 1, None) == 0


def test_silu_rows_rejects_null_row_ids():
    from kb_nano_amd._lib import lib
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert lib().kbn_silu_mul_quant_fp8_rows(p, 128, 256, 512, p, 256, p, 1, 128, 1e-10, 1, None, None) == 1
    assert "row ids" in _err()


def test_silu_rejects_ragged_n():
    from kb_nano_amd._lib import lib
    rc = lib().kbn_silu_mul_quant_fp8(None, 8, 100, 200, None, 100, None, 1, 1, 1e-10, 1, None)
    assert rc == 1 and "multiple of 128" in _err()


def test_gemm_rejects_bad_shapes():
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_fp8_gemm_nt(None, 128, None, 1, 1, None, 128, None, 1, None, 128, 8, 128, 100, 1, None) == 1
    assert "multiple of 128" in _err()
    assert L.kbn_fp8_gemm_nt(None, 64, None, 1, 1, None, 128, None, 1, None, 128, 8, 128, 128, 1, None) == 1
    assert "leading dimension" in _err()
    # misaligned A pointer
    assert L.kbn_fp8_gemm_nt(ctypes.c_void_p(8), 128, None, 1, 1, None, 128, None, 1, None, 128,
                             8, 128, 128, 1, None) == 1
    assert "aligned" in _err()


def test_gemm_workspace_query():
    """A workspace is only asked for when the last wave of tiles would be
    partly empty and splitting its K pays off; it then holds one fp32
    BM x BN slab per (split, tail tile)."""
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_fp8_gemm_nt_workspace_bytes(4096, 36864, 7168, 1) == 0   # 2304 tiles = 9 full waves
    assert L.kbn_fp8_gemm_nt_workspace_bytes(8, 8192, 100, 1) == 0        # K not a multiple of 128
    assert L.kbn_fp8_gemm_nt_workspace_bytes(0, 8192, 8192, 1) == 0
    assert L.kbn_fp8_gemm_nt_workspace_bytes(24, 512, 512, 1) == 0        # too little K to split
    for M, N, K in ((128, 7168, 18432), (1, 8192, 28672), (77, 203, 65536)):
        n = L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1)
        assert n > 0 and n % (64 * 128 * 4) == 0, (M, N, K, n)


def test_gemm_split_plan_choices():
    """The tail planner's choices on a 256-CU device (the planner's default
    when no device is visible), pinned to what split-count sweeps measured
    fastest on MI355X: 12 K blocks stay data-parallel (a split's fixed cost
    exceeds the six blocks it saves), long K splits, and a deep split is
    capped where the per-split reduction cost overtakes the shorter K run.
    The workspace is one fp32 BM x BN slab per (split, tail tile)."""
    from kb_nano_amd._lib import lib
    L = lib()
    if torch.cuda.device_count() > 0 and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the plan depends on the device's CU count; pinned for 256 CUs")

    def splits(M, N, K, bm, bn):
        tiles = -(-M // bm) * -(-N // bn)
        return L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1) // (tiles % 256 * bm * bn * 4) or 1

    # 12 K blocks: data-parallel (measured 10.3 us against 20.1 us split in two)
    assert splits(128, 12288, 1536, 128, 128) == 1
    assert splits(128, 4096, 1536, 128, 128) == 1
    assert splits(64, 12288, 1536, 64, 128) == 1
    assert splits(8, 12288, 1536, 64, 128) == 1
    # long K: split, and not deeper than the sweep's best
    assert splits(128, 12288, 7168, 128, 128) == 2
    assert splits(128, 7168, 18432, 128, 128) == 4
    assert splits(8, 10240, 8192, 64, 128) == 3
    assert splits(64, 8192, 28672, 64, 128) == 4
    assert 6 <= splits(32, 2048, 7168, 64, 128) <= 8
    assert splits(512, 4096, 7168, 256, 256) == 4


def test_gemm_ws_rejects_bad_shapes():
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_fp8_gemm_nt_ws(None, 128, None, 1, 1, None, 128, None, 1, None, 128, 8, 128, 100, 1,
                                None, 0, None) == 1
    assert "multiple of 128" in _err()


def test_bf16a_gemm_rejects_bad_shapes_and_plans_like_the_dense_gemm():
    """The bf16-activation GEMM covers M <= 64 and K in whole 128-blocks;
    its split plan is the 64x128 tiles' (one fp32 slab per split and tail
    tile), asked for only where the dense GEMM's plan splits too."""
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert L.kbn_fp8_gemm_bf16a(p, 256, 1e-10, p, 256, p, 2, p, 128, 65, 128, 256, None, 0, None) == 1
    assert "M <= 64" in _err()
    assert L.kbn_fp8_gemm_bf16a(p, 256, 1e-10, p, 256, p, 2, p, 128, 8, 128, 200, None, 0, None) == 1
    assert "multiple of 128" in _err()
    assert L.kbn_fp8_gemm_bf16a(ctypes.c_void_p(8), 256, 1e-10, p, 256, p, 2, p, 128, 8, 128, 256, None, 0,
                                None) == 1
    assert "aligned" in _err()
    assert L.kbn_fp8_gemm_bf16a(None, 256, 1e-10, None, 256, None, 2, None, 128, 0, 128, 256, None, 0, None) == 0
    assert L.kbn_fp8_gemm_bf16a_workspace_bytes(65, 8192, 8192) == 0
    assert L.kbn_fp8_gemm_bf16a_workspace_bytes(8, 8192, 100) == 0
    assert L.kbn_fp8_gemm_bf16a_workspace_bytes(8, 12288, 1536) == 0      # 12 K blocks stay data-parallel
    for M, N, K in ((1, 10240, 8192), (64, 8192, 28672), (8, 8192, 8192)):
        n = L.kbn_fp8_gemm_bf16a_workspace_bytes(M, N, K)
        assert n > 0 and n % (64 * 128 * 4) == 0, (M, N, K, n)


def test_bf16a_routing_rule():
    """Fp8Linear takes the bf16-activation GEMM for every shape up to 32 rows
    (measured faster than quant + GEMM on MI355X on all Llama-70B decode
    shapes), and at 33-64 rows only where its plan splits K into workgroups
    of at most 16 blocks within one wave of tiles (2048 x 2048, o); long K per
    workgroup (qkv, down), more tiles than CUs (gate_up), unsplit plans and
    M > 64 stay with quant + GEMM."""
    from kb_nano_amd._lib import lib
    L = lib()
    if torch.cuda.device_count() > 0 and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the plan depends on the device's CU count; pinned for 256 CUs")
    yes = [(1, 10240, 8192), (32, 57344, 8192), (16, 8192, 28672), (64, 2048, 2048), (64, 8192, 8192)]
    no = [(64, 10240, 8192), (64, 8192, 28672), (64, 57344, 8192), (64, 7168, 2048), (65, 2048, 2048),
          (8, 2048, 200)]
    for M, N, K in yes:
        assert L.kbn_fp8_gemm_bf16a_preferred(M, N, K) == 1, (M, N, K)
    for M, N, K in no:
        assert L.kbn_fp8_gemm_bf16a_preferred(M, N, K) == 0, (M, N, K)


def test_grouped_rejects_unaligned_m_sum():
    from kb_nano_amd._lib import lib
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    rc = lib().kbn_fp8_grouped_gemm_nt_contiguous(p, 128, p, 1, 1, p, p, p, 256, p,
                                                  100, 256, 128, 4, 1, None)
    assert rc == 1 and "128-row alignment" in _err()


def test_empty_shapes_are_noops():
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_per_token_group_quant_fp8(None, 0, 256, 256, None, 256, None, 1, 1, 1e-10, 1, None) == 0
    assert L.kbn_fp8_gemm_nt(None, 128, None, 1, 1, None, 128, None, 1, None, 128, 0, 128, 128, 1, None) == 0


def test_host_layer_refuses_cpu_tensors():
    from kb_nano_amd import _ops
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        _ops.per_token_group_quant_fp8(x, torch.empty(4, 256, dtype=torch.float8_e4m3fn), torch.empty(4, 2))


def test_ops_registered_with_reference_schemas():
    import kb_nano_amd  # noqa: F401
    s = str(torch.ops.kb_nano_fp8.fp8_gemm_nt.default._schema)
    assert "fp8_gemm_nt(Tensor q_input, Tensor input_scale, Tensor weight, Tensor weight_scale, Tensor(" in s
    assert "!" in s.split("weight_scale,")[1]  # output is declared mutated
    s = str(torch.ops.kb_nano_fp8.flashinfer_blockscale_gemm.default._schema)
    assert "flashinfer_blockscale_gemm(Tensor input_bf16, Tensor weight_fp8, Tensor weight_scale, Tensor(" in s
    assert "!" in s.split("weight_scale,")[1]
    s = str(torch.ops.kb_nano_fp8.per_token_group_quant_fp8.default._schema)
    assert "bool column_major_scales=False" in s
    s = str(torch.ops.kb_nano_fp8_moe.m_grouped_gemm_nt_contiguous.default._schema)
    assert "Tensor expert_ids, bool disable_ue8m0_cast" in s


def test_meta_impls_allow_fake_tracing():
    """The ops have Meta impls, so shape propagation never runs a kernel."""
    import kb_nano_amd  # noqa: F401
    M, N, K = 16, 256, 512
    dev = "meta"
    torch.ops.kb_nano_fp8.fp8_gemm_nt(
        torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev), torch.empty(M, K // 128, device=dev),
        torch.empty(N, K, dtype=torch.float8_e4m3fn, device=dev), torch.empty(2, 4, device=dev),
        torch.empty(M, N, dtype=torch.bfloat16, device=dev))


def test_module_api_matches_reference_surface():
    from kb_nano_amd import Fp8GroupedGemmContiguous, Fp8Linear, SiluMulQuantFp8, _Fp8PrefillBufs
    lin = Fp8Linear()
    assert lin.BLOCK_SIZE == 128 and lin._FLASHINFER_M_THRESHOLD == 32
    assert lin._a_buf is None and lin._s_buf is None and lin._o_buf is None and lin._pf is None
    assert _Fp8PrefillBufs.__slots__ == ("a", "s", "o")
    import inspect
    assert list(inspect.signature(Fp8Linear.forward).parameters) == [
        "self", "input_bf16", "weight_fp8", "weight_scale_inv", "bias"]
    assert list(inspect.signature(SiluMulQuantFp8.forward).parameters) == [
        "self", "input", "output", "use_ue8m0", "eps"]
    assert list(inspect.signature(Fp8GroupedGemmContiguous.forward).parameters) == [
        "self", "a_fp8", "a_scale", "b_fp8", "b_scale", "c_bf16", "expert_ids"]


def test_candidate_slot_files_load_standalone():
    """kernel_swapper loads tasks/candidate/L1/<name>.py with
    spec_from_file_location and picks the baseline class name
    (infra/kernel_swapper.py:328-355)."""
    import importlib.util
    for fname, cls in [("fp8_linear", "Fp8Linear"), ("silu_mul_quant_fp8", "SiluMulQuantFp8"),
                       ("fp8_grouped_gemm_contiguous", "Fp8GroupedGemmContiguous")]:
        path = os.path.join(ROOT, "kb_nano_amd", "candidate", "L1", fname + ".py")
        spec = importlib.util.spec_from_file_location(f"_cand_{fname}", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        assert isinstance(getattr(mod, cls), type)


def test_colmajor_scale_layout():
    from kb_nano_amd import _alloc_colmajor_scale
    s = _alloc_colmajor_scale(64, 16, torch.device("cpu"))
    assert s.shape == (64, 16) and s.stride() == (1, 64)


def test_compute_aligned_m():
    from kb_nano_amd.moe_layout import _compute_aligned_M
    import oracle
    for args in [(4096, 8, 256, 128), (7, 2, 3, 128), (128, 1, 1, 128)]:
        assert _compute_aligned_M(*args) == oracle.compute_aligned_M(*args)


def test_moe_layout_has_no_cpu_path():
    """The permute and the unpermute run only in the HIP kernels."""
    from kb_nano_amd.moe_layout import _deepgemm_permute, _deepgemm_unpermute_and_reduce
    topk = torch.zeros(4, 2, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="no CPU path"):
        _deepgemm_permute(torch.zeros(4, 256, dtype=torch.float8_e4m3fn), torch.ones(4, 2), topk, 8, 128)
    with pytest.raises(RuntimeError, match="no CPU path"):
        _deepgemm_unpermute_and_reduce(torch.zeros(1024, 256, dtype=torch.bfloat16), topk, torch.ones(4, 2),
                                       torch.zeros(4, 2, dtype=torch.int32), torch.empty(4, 256, dtype=torch.bfloat16))


def test_moe_permute_workspace_query():
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_moe_permute_workspace_bytes(32768, 0) == -1
    assert L.kbn_moe_permute_workspace_bytes(32768, 1025) == -1
    assert L.kbn_moe_permute_workspace_bytes(-1, 8) == -1
    # no pairs: counts and offsets only
    assert L.kbn_moe_permute_workspace_bytes(0, 256) == 1024 + 1040
    # cfg4: 64 chunks x 256 experts of histograms, a rank per pair, counts, offsets
    assert L.kbn_moe_permute_workspace_bytes(32768, 256) == 64 * 256 * 4 + 32768 * 4 + 1024 + 1040
    # chunks grow past 256 x 512 pairs so the scan stays short
    n = 1 << 20
    assert L.kbn_moe_permute_workspace_bytes(n, 64) == 256 * 64 * 4 + n * 4 + 256 + 272


def test_moe_permute_rejects_bad_arguments():
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first

    def call(ids_bytes=8, M=4, k=2, E=8, align=128, ld=256, row=256, M_sum=None, ws=1 << 20, sp=(2, 1)):
        M_sum = (M * k + E * (align - 1) + align - 1) // align * align if M_sum is None else M_sum
        return L.kbn_moe_permute_contiguous(p, ids_bytes, M, k, E, align, p, ld, row, p, 2, 1, 2, M_sum,
                                            p, p, sp[0], sp[1], p, p, 1, p, ws, None)
    assert call(ids_bytes=2) == 1 and "ids_bytes" in _err()
    assert call(E=2000) == 1 and "num_experts" in _err()
    assert call(M_sum=1152) == 1 and "M_sum" in _err()   # the right value is 1024
    assert call(row=100, ld=100) == 1 and "multiple of 16" in _err()
    assert call(ld=128) == 1 and "row stride" in _err()
    assert call(ws=16) == 1 and "workspace" in _err()
    assert call(sp=(1, 100)) == 1 and "column-major" in _err()    # columns would overlap rows (M_sum 1024)
    assert call(sp=(1, 1)) == 1 and "strides" in _err()


def test_moe_permute_quant_rejects_bad_arguments():
    """The quantizing permute refuses what the copy permute refuses, plus its
    own limits (bf16 rows: K a multiple of 128, ld_x >= K with 16-byte rows,
    top_k <= 64), before any launch."""
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first

    def call(M=4, k=2, E=8, ld=256, K=256, M_sum=None, x=p, ws=1 << 20, sp=(2, 1)):
        M_sum = (M * k + E * 127 + 127) // 128 * 128 if M_sum is None else M_sum
        return L.kbn_moe_permute_quant_contiguous(p, 8, M, k, E, 128, x, ld, K, 1e-10, 1, M_sum, p, p, sp[0], sp[1],
                                                  p, p, 0, p, ws, None)
    assert call(K=200, ld=200) == 1 and "multiple of 128" in _err()
    assert call(k=65, E=128) == 1 and "top_k" in _err()
    assert call(ld=128) == 1 and "ld_x" in _err()
    assert call(ld=260) == 1 and "16-byte aligned" in _err()
    assert call(x=ctypes.c_void_p(4098)) == 1 and "16-byte aligned" in _err()
    assert call(M_sum=1152) == 1 and "M_sum" in _err()
    assert call(ws=16) == 1 and "workspace" in _err()
    assert call(sp=(1, 1)) == 1 and "strides" in _err()


def test_grouped_gemm_silu_quant_rejects_bad_arguments():
    """The grouped GEMM with the SiLU*Mul + quant epilogue refuses shapes it
    cannot tile (N2 not a multiple of 256, M_sum not a multiple of 128),
    unaligned outputs and negative scale strides, before any launch."""
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)

    def call(M_sum=256, N2=512, K=256, q=p, ldq=256, qs=p, qs_sm=1, qs_sg=256):
        return L.kbn_fp8_grouped_gemm_silu_quant(p, K, p, 1, M_sum, p, p, p, M_sum, N2, K, 4, 1, q, ldq, qs,
                                                 qs_sm, qs_sg, 1e-10, 1, None)
    assert call(N2=384, ldq=192) == 1 and "multiple of 256" in _err()
    assert call(M_sum=200) == 1 and "128-row alignment" in _err()
    assert call(q=ctypes.c_void_p(4100)) == 1 and "8-byte aligned" in _err()
    assert call(ldq=260) == 1 and "8-byte aligned" in _err()
    assert call(qs_sm=-1) == 1 and "scale strides" in _err()
    assert call(qs=ctypes.c_void_p(4098)) == 1 and "scale strides" in _err()
    assert call(K=200) == 1 and "multiple of 128" in _err()
    assert call(M_sum=0) == 0                                   # nothing to do


def test_moe_unpermute_rejects_bad_arguments():
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)
    assert L.kbn_moe_unpermute_reduce(p, 1024, 100, 100, p, 4, 2, p, 0, p, 100, None) == 1
    assert "multiple of 8" in _err()
    assert L.kbn_moe_unpermute_reduce(p, 1024, 256, 256, p, 4, 2, p, 0, ctypes.c_void_p(4100), 256, None) == 1
    assert "aligned" in _err()
    assert L.kbn_moe_unpermute_reduce(None, 1024, 256, 256, None, 0, 2, None, 0, None, 256, None) == 0  # M = 0


def test_fused_experts_surface():
    """FusedExperts keeps the reference forward's argument names and order
    (tasks/baseline/L2/fused_experts.py:190-205)."""
    import inspect

    from kb_nano_amd import FusedExperts
    names = list(inspect.signature(FusedExperts.forward).parameters)
    assert names == ["self", "hidden_states", "w13", "w2", "topk_weights", "topk_ids", "num_experts", "w13_scale",
                     "w2_scale", "w13_scale_dg", "w2_scale_dg", "use_fp8_w8a8", "block_shape"]


def test_rmsnorm_quant_rejects_bad_arguments():
    """Validation before any device call: hidden sizes that are not a
    multiple of 8, an unknown dtype code, misaligned rows; empty input is a
    no-op (any H that is a multiple of 8 is accepted)."""
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    assert L.kbn_rmsnorm_fp8_quant(p, 4, 100, 100, p, None, 0, p, 104, p, 1, 4, 1e-6, None) == 1
    assert "multiple of 8" in _err()
    assert L.kbn_rmsnorm_fp8_quant_typed(p, 3, 4, 1024, 1024, p, None, 0, p, 1024, p, 1, 4, 1e-6, None) == 1
    assert "dtype code 3" in _err()
    assert L.kbn_rmsnorm_fp8_quant_typed(p, 2, 4, 1028, 1028, p, None, 0, p, 1032, p, 1, 4, 1e-6, None) == 1
    assert "multiple of 8" in _err()
    assert L.kbn_rmsnorm_fp8_quant_typed(p, 1, 4, 1024, 1020, p, None, 0, p, 1024, p, 1, 4, 1e-6, None) == 1
    assert "row stride" in _err()
    assert L.kbn_rmsnorm_fp8_quant(None, 0, 1024, 1024, None, None, 0, None, 1024, None, 1, 0, 1e-6, None) == 0
    assert L.kbn_rmsnorm_fp8_quant_typed(None, 2, 0, 40960, 40960, None, None, 0, None, 40960, None, 1, 0, 1e-6,
                                         None) == 0


def test_rmsnorm_quant_surface_matches_reference():
    """Module names, forward arguments and op schemas of
    tasks/baseline/L1/rmsnorm_quant.py:27-134."""
    import inspect
    from kb_nano_amd import FusedAddRMSNormFP8Quant, RMSNormFP8Quant
    assert list(inspect.signature(RMSNormFP8Quant.forward).parameters) == ["self", "input", "weight", "eps"]
    assert list(inspect.signature(FusedAddRMSNormFP8Quant.forward).parameters) == [
        "self", "input", "residual", "weight", "eps"]
    def args(op):
        sch = op.default._schema
        return [(a.name, bool(a.alias_info and a.alias_info.is_write)) for a in sch.arguments]
    assert args(torch.ops.kb_nano_norm.rmsnorm_fp8_quant) == [
        ("output_fp8", True), ("output_scales", True), ("input", False), ("weight", False), ("eps", False)]
    assert args(torch.ops.kb_nano_norm.fused_add_rmsnorm_fp8_quant) == [
        ("output_fp8", True), ("output_scales", True), ("input", True), ("residual", True), ("weight", False),
        ("eps", False)]


def test_sorted_moe_entry_points_reject_bad_arguments():
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    # moe_align_block_size: 100 pairs, 16 experts, blocks of 64 need 100 + 16*63 slots
    assert L.kbn_moe_align_block_size(p, 4, 100, 16, 64, p, 1000, p, 100, p, None, p, 1 << 20, None) == 1
    assert "sorted_token_ids holds 1000" in _err()
    assert L.kbn_moe_align_block_size(p, 4, 100, 16, 64, p, 1108, p, 10, p, None, p, 1 << 20, None) == 1
    assert "expert_ids holds 10" in _err()
    assert L.kbn_moe_align_block_size(p, 2, 100, 16, 64, p, 1108, p, 18, p, None, p, 1 << 20, None) == 1
    assert "ids_bytes" in _err()
    assert L.kbn_moe_align_block_size(p, 4, 100, 16, 64, p, 1108, p, 18, p, None, p, 16, None) == 1
    assert "workspace" in _err()
    # fused MoE GEMM
    args = dict(lda=256, rows=8, N=512, K=256, E=4, block=64, nv=16, topk=2)

    def gemm(**kw):
        a = {**args, **kw}
        return L.kbn_fp8_fused_moe_gemm(p, a["lda"], a["rows"], p, 2, 1, p, p, p, a["N"], p, p, p, 1024,
                                        a["block"], a["nv"], a["topk"], None, a["N"], a["K"], a["E"],
                                        a.get("ws"), a.get("ws_bytes", 0), None)
    assert gemm(K=200, lda=208) == 1 and "multiple of 128" in _err()
    assert gemm(block=32) == 1 and "multiple of 64" in _err()
    assert gemm(rows=4) == 1 and "A rows" in _err()
    assert gemm(lda=250) == 1 and "16-byte" in _err()
    assert L.kbn_fp8_fused_moe_gemm_workspace_bytes(1024, 256) == 1024 * 2 * 4
    assert gemm(ws=p, ws_bytes=100) == 1 and "workspace" in _err()
    # moe_sum
    assert L.kbn_moe_sum(p, 4, 0, 128, 128, p, 128, None) == 1 and "top_k" in _err()
    assert L.kbn_moe_sum(p, 4, 2, 128, 100, p, 128, None) == 1 and "strides" in _err()
    assert L.kbn_moe_sum(None, 0, 2, 128, 128, None, 128, None) == 0


def test_sorted_moe_surface_matches_reference():
    """Argument names and order of the sorted-token modules
    (tasks/baseline/L1/moe_align.py:71-77, moe_sum.py:25-29,
    moe_grouped_gemm.py:308-324, tasks/baseline/L2/vllm_fused_experts.py:116-127)."""
    import importlib.util
    import inspect

    from kb_nano_amd import MoeAlign, MoeGroupedGemm, MoeSum, VllmFusedExperts
    assert list(inspect.signature(MoeAlign.forward).parameters) == ["self", "topk_ids", "block_size",
                                                                    "num_experts", "naive"]
    assert list(inspect.signature(MoeSum.forward).parameters) == ["self", "input", "topk"]
    assert list(inspect.signature(MoeGroupedGemm.forward).parameters) == [
        "self", "A", "B", "C", "topk_weights", "sorted_token_ids", "expert_ids", "num_tokens_post_padded",
        "mul_routed_weight", "top_k", "config", "a_scale", "b_scale", "use_fp8_w8a8", "block_shape"]
    assert list(inspect.signature(VllmFusedExperts.forward).parameters) == [
        "self", "hidden_states", "w13", "w2", "topk_weights", "topk_ids", "num_experts", "w13_scale", "w2_scale",
        "block_shape"]
    for fname, cls in [("moe_align", "MoeAlign"), ("moe_sum", "MoeSum"), ("moe_grouped_gemm", "MoeGroupedGemm")]:
        path = os.path.join(ROOT, "kb_nano_amd", "candidate", "L1", fname + ".py")
        spec = importlib.util.spec_from_file_location(f"_cand_{fname}", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        assert isinstance(getattr(mod, cls), type)


def test_sorted_moe_config_block_sizes():
    from kb_nano_amd.moe_grouped_gemm import MoeGroupedGemm, get_triton_config
    assert get_triton_config(4, (256, 4096, 7168), (256, 7168, 2048), 8, True, [128, 128])["BLOCK_SIZE_M"] == 64
    assert get_triton_config(4096, (256, 4096, 7168), (256, 7168, 2048), 8, True, [128, 128])["BLOCK_SIZE_M"] == 128
    with pytest.raises(NotImplementedError):
        MoeGroupedGemm()(torch.zeros(4, 256), torch.zeros(2, 256, 256), torch.zeros(8, 256), None, None,
                         torch.zeros(8, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), False, 2)


def test_requant_rejects_unsafe_aliasing():
    """In-place requant is allowed only for fp8 codes over the same layout:
    fp32 input (4 bytes per element) under an fp8 output, a shifted fp8
    output, or scales aliased with other strides are rejected before any
    launch (the pointers are never dereferenced)."""
    from kb_nano_amd._lib import lib
    L = lib()
    E, N, K = 2, 256, 256
    base = 1 << 20
    w, s = ctypes.c_void_p(base), ctypes.c_void_p(base + (1 << 24))
    # fp32 input, fp8 output at the same address
    assert L.kbn_fp8_block_requant(w, 1, None, 0, 0, E, N, K, w, s, 4, 2, 1, 1e-4, None) == 1
    assert "in place" in _err()
    # fp32 input, fp8 output inside its second half
    w2 = ctypes.c_void_p(base + E * N * K * 2)
    assert L.kbn_fp8_block_requant(w, 1, None, 0, 0, E, N, K, w2, s, 4, 2, 1, 1e-4, None) == 1
    # fp8 input, output shifted by one row
    w3 = ctypes.c_void_p(base + K)
    assert L.kbn_fp8_block_requant(w, 0, s, 4, 2, E, N, K, w3, ctypes.c_void_p(base + (1 << 25)), 4, 2, 1, 1e-4,
                                   None) == 1
    assert "w_out == w_in" in _err()
    # fp8 input in place, but the output scales alias the input scales with other strides
    assert L.kbn_fp8_block_requant(w, 0, s, 4, 2, E, N, K, w, s, 8, 2, 1, 1e-4, None) == 1
    assert "different layout" in _err()


def test_gemm_noalloc_validates_before_touching_a_device():
    """The allocation-free GEMM reports its fixed scratch size and rejects
    bad shapes like the other GEMM entry points, before any device call."""
    from kb_nano_amd._lib import lib
    L = lib()
    assert L.kbn_fp8_gemm_nt_noalloc_scratch_bytes() == 64 << 20
    assert L.kbn_fp8_gemm_nt_noalloc(None, 128, None, 1, 1, None, 128, None, 1, None, 128, 8, 128, 100, 1,
                                     None) == 1
    assert "multiple of 128" in _err()
    assert L.kbn_fp8_gemm_nt_noalloc(None, 128, None, 1, 1, None, 128, None, 1, None, 128, 0, 128, 128, 1,
                                     None) == 0


def test_splitk_counter_regions_exhaust_and_fall_back():
    """The region table behind the fused split-K sums (no GPU): every new
    stream takes the next region until all 1024 are taken, later streams get
    none and are counted as fallbacks (their launches take the separate
    reduction kernel), and a stream that holds a region keeps it."""
    import numpy as np
    from kb_nano_amd._lib import lib
    L = lib()
    used, total, fb = ctypes.c_int64(-1), ctypes.c_int64(-1), ctypes.c_int64(-1)
    assert L.kbn_splitk_counter_stats(ctypes.byref(used), ctypes.byref(total), ctypes.byref(fb)) == 0
    assert total.value == 1024 and used.value >= 0 and fb.value >= 0
    for n in (1, 1023, 1024, 1030):
        out = np.full(n + 1, -7, dtype=np.int32)
        nfb = ctypes.c_int64(-1)
        assert L.kbn_debug_splitk_regions(n, out.ctypes.data, ctypes.byref(nfb)) == 0, _err()
        k = min(n, 1024)
        assert np.array_equal(out[:k], np.arange(k)), n
        assert np.all(out[k:n] == -1), n
        assert out[n] == 0, "a stream keeps its region"
        assert nfb.value == n - k
    assert L.kbn_debug_splitk_regions(0, None, None) == 1
    from kb_nano_amd import _ops
    st = _ops.splitk_counter_stats()
    assert st["regions_total"] == 1024 and st["fallbacks"] == fb.value


def test_fused_experts_direct_silu_call_respects_hooks():
    """The experts layer launches its SiLU*Mul+quant kernel directly only
    when no forward hook would see the reference's module call."""
    from torch import nn

    from kb_nano_amd.fused_experts import _direct_call_ok
    from kb_nano_amd.silu_mul_quant_fp8 import SiluMulQuantFp8
    m = SiluMulQuantFp8()
    assert _direct_call_ok(m)
    h = m.register_forward_hook(lambda *a: None)
    assert not _direct_call_ok(m)
    h.remove()
    h = m.register_forward_pre_hook(lambda *a: None)
    assert not _direct_call_ok(m)
    h.remove()
    h = nn.modules.module.register_module_forward_hook(lambda *a: None)
    assert not _direct_call_ok(m)
    h.remove()
    assert _direct_call_ok(m)

    class Other(SiluMulQuantFp8):
        pass
    assert not _direct_call_ok(Other())


def test_release_workspaces_drops_cached_buffers():
    from kb_nano_amd import _ops
    saved = dict(_ops._WS_BUFS)
    try:
        _ops._WS_BUFS.clear()
        _ops._WS_BUFS[(0, 1)] = torch.empty(4, dtype=torch.uint8)
        _ops._WS_BUFS[(1, 1)] = torch.empty(4, dtype=torch.uint8)
        assert _ops.release_workspaces(device=1) == 1 and list(_ops._WS_BUFS) == [(0, 1)]
        assert _ops.release_workspaces() == 1 and not _ops._WS_BUFS
    finally:
        _ops._WS_BUFS.clear()
        _ops._WS_BUFS.update(saved)


def test_pack_ue8m0_weight_scales_layout():
    """The packed per-row UE8M0 layout: byte j of word (n, i) is the rounded-up
    exponent of row n's block scale for K block 4i + j, MN-major storage."""
    import numpy as np

    from kb_nano_amd import _ops
    N, K = 300, 1408                      # 3 row blocks (the last partial), 11 K blocks, 3 words
    rng = np.random.default_rng(0)
    s = (2.0 ** rng.integers(-12, 3, size=(3, 11)) * rng.choice([1.0, 1.37], size=(3, 11))).astype(np.float32)
    p = _ops.pack_ue8m0_weight_scales(torch.from_numpy(s), N, K)
    assert p.shape == (N, 3) and p.dtype == torch.int32 and p.stride() == (1, 300)
    words = p.numpy().view(np.uint32)
    for n in (0, 127, 128, 255, 256, 299):
        for kb in range(11):
            e = (words[n, kb // 4] >> (8 * (kb % 4))) & 0xFF
            v = float(s[n // 128, kb])
            assert 2.0 ** (int(e) - 127) == 2.0 ** np.ceil(np.log2(v)), (n, kb)
        assert (words[n, 2] >> 24) == 0   # K block 11 does not exist


def test_packed_gemm_rejects_bad_scales_without_device():
    from kb_nano_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4098)
    rc = L.kbn_fp8_gemm_nt_packed_ws(p, 256, p, 1, 64, p, 256, odd, 1, 64, p, 128, 64, 128, 256, None, 0, None)
    assert rc == 1 and "4-byte aligned" in _err()
    rc = L.kbn_fp8_gemm_nt_packed_ws(p, 256, p, 1, 64, p, 256, p, 0, 64, p, 128, 64, 128, 256, None, 0, None)
    assert rc == 1 and "strides" in _err()
    rc = L.kbn_fp8_gemm_nt_packed_ws(p, 256, None, 1, 64, p, 256, p, 1, 128, p, 128, 64, 128, 256, None, 0, None)
    assert rc == 1 and "null scale" in _err()


def _plan(L, M, N, K, ue8m0=1, bf16a=0):
    import numpy as np
    out = np.zeros(9, dtype=np.int64)
    assert L.kbn_debug_gemm_plan(M, N, K, ue8m0, bf16a, out.ctypes.data) == 0, _err()
    return out


def test_weight_stream_plans_narrow_and_wide():
    """The tile planner (no GPU: 256 CUs assumed).  Weight-streaming shapes
    (M <= 64) with narrow weights (N <= 4096) take 64x64 tiles with K split
    and summed in the split launch; wider weights keep the 64x128 tiles
    (Llama-70B decode shapes: qkv 3 splits, o and down 4, gate_up
    data-parallel); the bf16-activation GEMM plans exactly as the fp8 GEMM
    (its results are bit-identical to quant + GEMM); the FP32 contract keeps
    64x128; the workspace the plan writes is what the entry point asks for."""
    import numpy as np
    from kb_nano_amd._lib import lib
    L = lib()
    for M in (1, 8, 32, 48, 64):
        for N, K in ((2048, 2048), (1024, 7168), (4096, 7168), (200, 1152), (4032, 2048)):
            p = _plan(L, M, N, K)
            assert (p[0], p[1], p[2]) == (64, 64, 4) and p[5] > 1 and p[7] == 1, (M, N, K, p)
            assert p[3] == -(-N // 64) and p[4] == 0 and p[5] * p[6] >= K // 128 > (p[5] - 1) * p[6]
            assert p[8] == p[5] * p[3] * 64 * 64 * 4 == L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, 1)
            assert np.array_equal(p, _plan(L, M, N, K, bf16a=1))
            assert _plan(L, M, N, K, ue8m0=0)[1] == 128
        for N, K, splits in ((10240, 8192, 3), (8192, 8192, 4), (8192, 28672, 4), (57344, 8192, 1)):
            p = _plan(L, M, N, K)
            assert (p[0], p[1], p[5]) == (64, 128, splits), (M, N, K, p)
            assert np.array_equal(p, _plan(L, M, N, K, bf16a=1))
    # config 1 takes the one-launch bf16-activation GEMM at 64 rows; long K on
    # 64x64 tiles does not (quant + GEMM measured faster there)
    assert L.kbn_fp8_gemm_bf16a_preferred(64, 2048, 2048) == 1
    assert L.kbn_fp8_gemm_bf16a_preferred(64, 4096, 7168) == 0
    assert L.kbn_fp8_gemm_bf16a_preferred(32, 4096, 7168) == 1
    # larger M: the 128x128 and 256x256 tiles, unchanged
    assert tuple(_plan(L, 128, 24576, 1536)[:2]) == (128, 128)
    assert tuple(_plan(L, 4096, 7168, 18432)[:2]) == (256, 256)
    assert L.kbn_debug_gemm_plan(65, 2048, 2048, 1, 1, np.zeros(9, np.int64).ctypes.data) == 1
    assert "bad arguments" in _err()


def test_scales_are_pow2_predicate_and_cache():
    """The check that lets the MoE layers run the UE8M0 kernels under the
    FP32 contract: true only when every scale is a positive, finite, normal
    power of two; its per-tensor answer is recomputed after an in-place change
    (through the tensor or a view of it) and after this package's raw-pointer
    scale writer bumps the version."""
    import torch
    from kb_nano_amd import _ops
    s = torch.tensor([[1.0, 0.5, 2.0 ** -100], [2.0 ** 100, 4.0, 2.0 ** -126]])
    assert _ops.scales_are_pow2(s)
    for bad in (1.1, 0.0, -2.0, float("inf"), float("nan"), 1e-40, 3.0):
        t = s.clone()
        t[1, 1] = bad
        assert not _ops.scales_are_pow2(t), bad
    s[0, 0] = 1.5                      # in place: the version moves, the answer follows
    assert not _ops.scales_are_pow2(s)
    s[0, 0] = 8.0
    assert _ops.scales_are_pow2(s)
    s[1:].fill_(0.75)                  # through a view: the base's version moves too
    assert not _ops.scales_are_pow2(s)
    assert not _ops.scales_are_pow2(torch.ones(2, 2, dtype=torch.float64))
    u = torch.ones(3, 3)
    assert _ops.scales_are_pow2(u)
    v0 = u._version
    torch.autograd.graph.increment_version(u)   # what fp8_block_requant does after writing
    assert u._version == v0 + 1 and u._kbn_pow2[0][0] == v0
    assert _ops.scales_are_pow2(u) and u._kbn_pow2[0][0] == v0 + 1
    # inference tensors have no version counter: checked once, again after
    # this package's in-place scale writes (the generation fp8_block_requant bumps)
    with torch.inference_mode():
        w = torch.ones(2, 3)
    assert _ops.scales_are_pow2(w)
    with torch.inference_mode():
        w[0, 0] = 3.0
        assert _ops.scales_are_pow2(w)          # not seen: documented
        _ops._SCALE_WRITES[0] += 1
        assert not _ops.scales_are_pow2(w)
