"""Fused MoE experts over the FP8 contiguous-layout path.

Mirrors ``FusedExperts`` of ``tasks/baseline/L2/fused_experts.py:139-283``
(kb_nano) for FP8 W8A8 block-scaled expert weights, the path its
``_forward_deep_gemm`` takes (:246-283):

    1x128 quant (row-major scales) -> contiguous permute -> grouped GEMM1 (w13)
    -> fused SiLU*Mul + 1x128 quant -> grouped GEMM2 (w2) -> unpermute-and-reduce

Every step runs in this package's gfx950 kernels: ``PerTokenGroupQuantFp8``,
the permute and unpermute-and-reduce of ``moe_layout``,
``m_grouped_fp8_gemm_nt_contiguous`` and ``SiluMulQuantFp8``.  When the
SiLU*Mul+quant module is this package's own and unhooked, GEMM1 and that
step are one launch (``_ops.grouped_gemm_silu_quant``: the GEMM's epilogue
applies SiLU*Mul and the 1x128 quant to its bf16 tile, the same bits as the
two launches, with no bf16 intermediate); likewise the quant of the hidden
states runs inside the permute (``_deepgemm_permute_quant``) when the quant
module is this package's own.  Where every block scale is a power of two the
grouped GEMMs run their UE8M0 kernels, which give the bits of the reference's
scales-as-given contract there.  Scratch buffers are shared by all layers, as
in the reference (layers run one after another).

The reference falls back to its Triton ``fused_moe_kernel`` for BF16 weights,
for shapes DeepGEMM does not take and while a CUDA graph is being captured
(:228-244).  Here nothing on the path synchronises with the host, so the
layer is captured as it runs eagerly.  The Triton kernel family is not part
of this path: BF16 experts and off-gate shapes raise ``NotImplementedError``
instead of running something else.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch.nn.modules import module as _module

from . import _ops
from .fp8_linear import PerTokenGroupQuantFp8
from .moe_grouped_gemm import _valid_deep_gemm, m_grouped_fp8_gemm_nt_contiguous
from .moe_layout import _compute_aligned_M, _deepgemm_permute, _deepgemm_permute_quant, _deepgemm_unpermute_and_reduce
from .silu_mul_quant_fp8 import SiluMulQuantFp8

__all__ = ["FusedExperts", "_compute_aligned_M", "_deepgemm_permute", "_deepgemm_unpermute_and_reduce"]

_FP8_GROUP_SIZE = 128


class _SharedBuf:
    """Scratch buffers shared by every FusedExperts layer (reference :139-153).

    ``captured`` keeps every buffer a HIP graph was captured with alive for
    the life of the process: a later, larger call replaces the buffer here,
    but the graph's kernels still address the old one."""
    __slots__ = ("a_fp8_1", "a_scale_1", "dg_ws1", "dg_ws2", "captured")

    def __init__(self):
        self.a_fp8_1 = None
        self.a_scale_1 = None
        self.dg_ws1 = None
        self.dg_ws2 = None
        self.captured = {}

    def hold_for_graph(self):
        for t in (self.a_fp8_1, self.a_scale_1, self.dg_ws1, self.dg_ws2):
            if t is not None:
                self.captured.setdefault(id(t), t)


_SHARED_BUF = _SharedBuf()


def _own_module(mod: nn.Module, cls) -> bool:
    """Whether ``mod`` is this package's ``cls`` with no forward hook or
    pre-hook (its own or a global one) and no compiler trace running: its
    outputs are then known (e.g. power-of-two scales)."""
    return (type(mod) is cls and not torch.compiler.is_compiling()
            and not mod._forward_hooks and not mod._forward_pre_hooks
            and not _module._global_forward_hooks and not _module._global_forward_pre_hooks)


def _direct_call_ok(mod: nn.Module) -> bool:
    """Whether the experts layer may launch the SiLU*Mul+quant kernel itself
    (over the rows with an expert id only) instead of calling the submodule:
    only for this package's own module, outside a compiler trace, and when
    no forward hook or pre-hook (the module's own or a global one) would see
    the call the reference makes (tasks/baseline/L2/fused_experts.py:272)."""
    return _own_module(mod, SiluMulQuantFp8)


class FusedExperts(nn.Module):
    """Fused MoE experts: two grouped FP8 GEMMs with SiLU*Mul+quant between.

    ``forward(hidden_states, w13, w2, topk_weights, topk_ids, num_experts,
    w13_scale, w2_scale, w13_scale_dg, w2_scale_dg, use_fp8_w8a8,
    block_shape)`` takes the reference's arguments: hidden_states bf16 [M, K],
    w13 fp8 [E, 2N, K], w2 fp8 [E, K, N] with 128x128 block scales
    [E, 2N/128, K/128] and [E, K/128, N/128], topk_ids / topk_weights [M, k].
    Returns bf16 [M, K] = sum_j w[m, j] * expert_{ids[m, j]}(x[m]).
    """

    def __init__(self):
        super().__init__()
        self.per_token_group_quant_fp8 = PerTokenGroupQuantFp8()
        self.silu_mul_quant_fp8 = SiluMulQuantFp8()
        self._sb = _SHARED_BUF
        # GEMM1 applies SiLU*Mul + quant in its own epilogue (the same bits as
        # the two launches) when the SiLU module is this package's and unhooked
        self.fuse_gate_up_silu = True
        # the grouped GEMMs run the UE8M0 kernels where they give the FP32
        # contract's bits: weight scales all powers of two, activation scales
        # from this package's quant (which writes powers of two)
        self.ue8m0_when_exact = True
        # the 1x128 quant of the hidden states runs inside the permute (the
        # same codes and scales, no token-order fp8 copy) when the quant
        # module is this package's and unhooked
        self.fuse_quant_permute = True

    def _get_fp8_bufs(self, M: int, K: int, device):
        sb = self._sb
        groups = math.ceil(K / _FP8_GROUP_SIZE)
        if sb.a_fp8_1 is None or sb.a_fp8_1.size(0) < M or sb.a_fp8_1.size(1) < K or sb.a_fp8_1.device != device:
            sb.a_fp8_1 = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=device)
            sb.a_scale_1 = torch.empty(M, groups, dtype=torch.float32, device=device)
        return sb.a_fp8_1[:M, :K], sb.a_scale_1[:M, :groups]

    def _get_dg_workspace(self, buf_id: int, shape, device, dtype):
        """A view of a shared byte buffer (grown when needed) as `shape`/`dtype`
        (reference :175-188)."""
        sb = self._sb
        attr = f"dg_ws{buf_id}"
        need = torch.tensor([], dtype=dtype).element_size() * math.prod(shape)
        raw = getattr(sb, attr)
        if raw is None or raw.numel() < need or raw.device != device:
            raw = torch.empty(need, dtype=torch.uint8, device=device)
            setattr(sb, attr, raw)
        return raw[:need].view(dtype).view(shape)

    def _reserve(self, max_tokens: int, K: int, N2: int, top_k: int, num_experts: int, device) -> None:
        """Size the shared scratch buffers for up to ``max_tokens`` tokens of
        this layer's shape, so later calls (and graph captures) reuse them
        instead of growing them."""
        M_sum = _compute_aligned_M(max_tokens, top_k, num_experts, _FP8_GROUP_SIZE)
        self._get_fp8_bufs(max_tokens, K, device)
        self._get_dg_workspace(1, (M_sum, max(N2, K)), device, torch.bfloat16)
        self._get_dg_workspace(2, (M_sum, N2 // 2), device, torch.float8_e4m3fn)

    def forward(self, hidden_states: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, topk_weights: torch.Tensor,
                topk_ids: torch.Tensor, num_experts: int, w13_scale: torch.Tensor | None = None,
                w2_scale: torch.Tensor | None = None, w13_scale_dg: torch.Tensor | None = None,
                w2_scale_dg: torch.Tensor | None = None, use_fp8_w8a8: bool = False,
                block_shape: list[int] | None = None) -> torch.Tensor:
        M, K = hidden_states.size()
        E, N2, _ = w13.size()
        N = N2 // 2
        top_k = topk_ids.size(1)
        if not use_fp8_w8a8:
            raise NotImplementedError("FusedExperts: only FP8 W8A8 block-scaled experts are on this path "
                                      "(the reference runs BF16 experts through its Triton kernel)")
        if block_shape is not None and list(block_shape) != [_FP8_GROUP_SIZE, _FP8_GROUP_SIZE]:
            raise NotImplementedError(f"FusedExperts: block_shape {block_shape} (only 128x128 blocks)")
        if not _valid_deep_gemm(hidden_states, w13, w2):
            raise NotImplementedError("FusedExperts: shapes outside the contiguous grouped-GEMM gate "
                                      "(the reference falls back to its Triton kernel)")
        s13 = w13_scale_dg if w13_scale_dg is not None else w13_scale
        s2 = w2_scale_dg if w2_scale_dg is not None else w2_scale
        if s13 is None or s2 is None:
            raise ValueError("FusedExperts: FP8 experts need w13_scale and w2_scale")
        return self._forward_deep_gemm(hidden_states, w13, w2, topk_weights, topk_ids, num_experts, s13, s2,
                                       block_shape, M, K, E, N, N2, top_k)

    def _forward_deep_gemm(self, hidden_states, w13, w2, topk_weights, topk_ids, num_experts, w13_scale, w2_scale,
                           block_shape, M, K, E, N, N2, top_k) -> torch.Tensor:
        """quant -> permute -> GEMM1 -> SiLU*Mul+quant -> GEMM2 -> unpermute
        (reference :246-283)."""
        dev = hidden_states.device
        alignment = _FP8_GROUP_SIZE
        M_sum = _compute_aligned_M(M, top_k, num_experts, alignment)

        # padding rows stay unwritten: the grouped GEMM skips them and never
        # writes their output rows, so nothing downstream reads them.  The
        # scales come out column-major, so GEMM1 reads each K block's row
        # scales contiguously (GEMM2's come column-major from SiLU*Mul+quant).
        own_quant = _own_module(self.per_token_group_quant_fp8, PerTokenGroupQuantFp8)
        if self.fuse_quant_permute and own_quant and hidden_states.dtype is torch.bfloat16:
            a1_perm, a1_scale_perm, expert_ids, inv_perm = _deepgemm_permute_quant(
                hidden_states, topk_ids, num_experts, alignment, zero_padding=False, scale_colmajor=True)
        else:
            a_fp8, a_scale = self._get_fp8_bufs(M, K, dev)
            self.per_token_group_quant_fp8(hidden_states, a_fp8, a_scale)
            a1_perm, a1_scale_perm, expert_ids, inv_perm = _deepgemm_permute(a_fp8, a_scale, topk_ids, num_experts,
                                                                            alignment, zero_padding=False,
                                                                            scale_colmajor=True)

        quant_out = self._get_dg_workspace(2, (M_sum, N), dev, torch.float8_e4m3fn)
        # the reference runs both GEMMs under the FP32 contract (its scales as
        # given, disable_ue8m0_cast=True); where every scale is a power of
        # two the UE8M0 kernels give the same bits, and skip the contract's
        # per-block significand bookkeeping
        ue1 = self.ue8m0_when_exact and own_quant and _ops.scales_are_pow2(w13_scale)
        ue2 = self.ue8m0_when_exact and not torch.compiler.is_compiling() and _ops.scales_are_pow2(w2_scale)
        if self.fuse_gate_up_silu and N2 % 256 == 0 and _direct_call_ok(self.silu_mul_quant_fp8):
            # GEMM1 with SiLU*Mul + quant in its epilogue: the codes and
            # column-major scales GEMM1 into a bf16 buffer followed by the
            # row-skipping SiLU*Mul+quant launch below would write, with no
            # bf16 [M_sum, N2] intermediate written or read
            a2_fp8 = quant_out
            a2_scale = torch.empty_strided((M_sum, N // _FP8_GROUP_SIZE), (1, M_sum), dtype=torch.float32,
                                           device=dev)
            _ops.grouped_gemm_silu_quant(a1_perm, a1_scale_perm, w13, w13_scale, expert_ids, not ue1, a2_fp8,
                                         a2_scale, True, 1e-10)
            return self._down_and_unpermute(a2_fp8, a2_scale, w2, w2_scale, expert_ids, topk_ids, topk_weights,
                                            inv_perm, M, K, M_sum, dev, hidden_states.dtype, ue2)

        mm1_out = self._get_dg_workspace(1, (M_sum, N2), dev, hidden_states.dtype)
        if ue1:
            _ops.m_grouped_gemm_nt_contiguous(a1_perm, a1_scale_perm, w13, w13_scale, mm1_out, expert_ids,
                                              disable_ue8m0_cast=False)
        else:
            m_grouped_fp8_gemm_nt_contiguous((a1_perm, a1_scale_perm), (w13, w13_scale), mm1_out, expert_ids)

        if _direct_call_ok(self.silu_mul_quant_fp8):
            # this package's module: the same launch over the rows with an
            # expert id only (padding rows hold nothing GEMM1 wrote, and
            # GEMM2 neither stores their output rows nor lets them touch
            # another row; half of config 4's rows), scales column-major as
            # the module makes them
            a2_fp8 = quant_out
            a2_scale = torch.empty_strided((M_sum, N // _FP8_GROUP_SIZE), (1, M_sum), dtype=torch.float32,
                                           device=dev)
            _ops.silu_mul_quant_fp8(mm1_out, a2_fp8, a2_scale, True, 1e-10, row_ids=expert_ids)
        else:   # a swapped-in or hooked module (or the compiler's trace) keeps the reference's call
            a2_fp8, a2_scale = self.silu_mul_quant_fp8(mm1_out, output=quant_out)
            ue2 = False   # its scales are not known to be powers of two

        return self._down_and_unpermute(a2_fp8, a2_scale, w2, w2_scale, expert_ids, topk_ids, topk_weights,
                                        inv_perm, M, K, M_sum, dev, hidden_states.dtype, ue2)

    def _down_and_unpermute(self, a2_fp8, a2_scale, w2, w2_scale, expert_ids, topk_ids, topk_weights, inv_perm, M, K,
                            M_sum, dev, dtype, ue8m0: bool = False) -> torch.Tensor:
        """GEMM2 and the unpermute-and-reduce (reference :276-283); ``ue8m0``:
        every scale is a power of two, so the UE8M0 kernel gives the FP32
        contract's bits."""
        mm2_out = self._get_dg_workspace(1, (M_sum, K), dev, dtype)
        if ue8m0:
            _ops.m_grouped_gemm_nt_contiguous(a2_fp8, a2_scale, w2, w2_scale, mm2_out, expert_ids,
                                              disable_ue8m0_cast=False)
        else:
            m_grouped_fp8_gemm_nt_contiguous((a2_fp8, a2_scale), (w2, w2_scale), mm2_out, expert_ids)

        output = torch.empty(M, K, dtype=dtype, device=dev)
        _deepgemm_unpermute_and_reduce(mm2_out, topk_ids, topk_weights, inv_perm, output)
        if torch.cuda.is_current_stream_capturing():
            self._sb.hold_for_graph()
        return output
