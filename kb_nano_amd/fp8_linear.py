"""Block-scaled FP8 linear and per-token-group activation quant on MI355X.

Drop-in for ``tasks/baseline/L1/fp8_linear.py`` (kb_nano): same classes,
attributes, helper functions and op names, backed by the gfx950 HIP kernels
of ``libkbn_fp8.so`` instead of Triton + DeepGEMM + FlashInfer.

Reference interface mirrored here:
  * ``PerTokenGroupQuantFp8.forward(x, out_fp8, out_scale) -> None``   (:282-297)
  * ``_alloc_colmajor_scale(M, num_groups, device)``                  (:300-313)
  * ``_Fp8PrefillBufs(max_tokens, K, N, device)`` with ``.a .s .o``    (:316-332)
  * ``Fp8Linear`` (``BLOCK_SIZE``, ``_FLASHINFER_M_THRESHOLD``,
    ``_a_buf/_s_buf/_o_buf/_pf``, ``_ensure_buffers``, ``forward``)   (:335-450)
  * ``postprocess_fp8_weights[_batched]``                            (:453-554)
  * ops ``torch.ops.kb_nano_fp8.{fp8_gemm_nt, per_token_group_quant_fp8,
    flashinfer_blockscale_gemm}`` (:89-178)

The reference sends M < 32 to FlashInfer's Hopper-only swapAB kernel, which
takes bf16 activations and quantizes them itself (:398-417).  Its gfx950
counterpart is ``_ops.fp8_gemm_bf16a`` (op ``flashinfer_blockscale_gemm``):
the block-scaled GEMM quantizes its activations in-kernel, bit-identical to
the quant launch followed by ``fp8_gemm_nt``.  ``Fp8Linear`` takes it for
M <= 64 where the library's plan says one launch beats two.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import _ops
from ._ops import FP8, GROUP, QUANT_EPS, is_e8m0_used

_FP8_INFO = torch.finfo(FP8)
_QUANT_EPS = QUANT_EPS


def _is_deep_gemm_e8m0_used() -> bool:
    """Name kept from the reference (fp8_grouped_gemm_contiguous.py:53-71)."""
    return is_e8m0_used()


def _per_token_group_quant_fp8(x: torch.Tensor, out_fp8: torch.Tensor, out_scale: torch.Tensor,
                               use_ue8m0: bool = True, column_major_scales: bool = False) -> None:
    """In-place 1x128 quant (reference :234-279).  The scale layout comes from
    ``out_scale``'s strides; ``column_major_scales`` only documents the
    caller's intent, as in the reference's Triton path."""
    _ops.per_token_group_quant_fp8(x, out_fp8, out_scale, use_ue8m0=use_ue8m0, eps=_QUANT_EPS)


class PerTokenGroupQuantFp8(nn.Module):
    """In-place per-token-group FP8 quantization (one HIP kernel launch).

    ``forward(x, out_fp8, out_scale)``: x bf16 [M,K] (made contiguous if it is
    not), out_fp8 float8_e4m3fn [M,K], out_scale float32 [M,K/128] with any
    strides (row-major by default, column-major for the dense GEMM)."""

    def forward(self, x: torch.Tensor, out_fp8: torch.Tensor, out_scale: torch.Tensor) -> None:
        x = x if x.is_contiguous() else x.contiguous()
        if torch.compiler.is_compiling():
            torch.ops.kb_nano_fp8.per_token_group_quant_fp8(x, out_fp8, out_scale)
        else:   # eager: the same launch without the dispatcher round trip
            _ops.per_token_group_quant_fp8(x, out_fp8, out_scale)


def _alloc_colmajor_scale(M: int, num_groups: int, device: torch.device) -> torch.Tensor:
    """fp32 scales exposed as [M, num_groups] over [num_groups, M] storage:
    strides (1, M), element (m, g) at g*M + m."""
    return torch.empty_strided((M, num_groups), (1, max(M, 1)), device=device, dtype=torch.float32)


class _Fp8PrefillBufs:
    """One shared set of prefill buffers per (K, N): fp8 activations ``a``,
    column-major scales ``s`` and bf16 output ``o`` for ``max_tokens`` rows."""

    __slots__ = ("a", "s", "o")

    def __init__(self, max_tokens: int, K: int, N: int, device: torch.device):
        self.a = torch.empty(max_tokens, K, dtype=FP8, device=device)
        self.s = _alloc_colmajor_scale(max_tokens, math.ceil(K / GROUP), device)
        self.o = torch.empty(max_tokens, N, dtype=torch.bfloat16, device=device)


def _maybe_get_flashinfer_fp8_gemm():
    """The reference's Hopper-only small-M kernel (:55-82); FlashInfer is
    never present on gfx950.  Its role, a bf16-input GEMM for small M, is
    ``_ops.fp8_gemm_bf16a``, which ``Fp8Linear.forward`` selects itself."""
    return None


class Fp8Linear(nn.Module):
    """Block-scaled FP8 linear: bf16 input, fp8 e4m3 weight [N,K] with fp32
    scales [ceil(N/128), ceil(K/128)], bf16 output [..., N].

    ``forward`` quantizes the input 1x128 with UE8M0 scales into column-major
    scale storage and runs the block-scaled GEMM, or, for M <= 64 where it is
    faster, runs the GEMM that quantizes its bf16 input itself (the same
    output bits; the fp8 buffers are then not written); with buffers
    installed the result is a view into the reused output buffer, exactly as
    the reference returns ``_o_buf[:M]`` / ``_pf.o[:M]``."""

    BLOCK_SIZE = GROUP
    _FLASHINFER_M_THRESHOLD = 32

    def __init__(self):
        super().__init__()
        self._a_buf: torch.Tensor | None = None
        self._s_buf: torch.Tensor | None = None
        self._o_buf: torch.Tensor | None = None
        self._pf: _Fp8PrefillBufs | None = None

    def _ensure_buffers(self, max_tokens: int, K: int, N: int, device: torch.device):
        num_groups = math.ceil(K / self.BLOCK_SIZE)
        self._a_buf = torch.empty(max_tokens, K, dtype=FP8, device=device)
        self._s_buf = _alloc_colmajor_scale(max_tokens, num_groups, device)
        self._o_buf = torch.empty(max_tokens, N, dtype=torch.bfloat16, device=device)

    def forward(self, input_bf16: torch.Tensor, weight_fp8: torch.Tensor,
                weight_scale_inv: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        N, K = weight_fp8.shape
        in_shape = input_bf16.shape
        flat = len(in_shape) == 2 and in_shape[1] == K
        x2 = input_bf16 if flat else input_bf16.reshape(-1, K)
        M = x2.shape[0]
        G = (K + self.BLOCK_SIZE - 1) // self.BLOCK_SIZE

        if torch.compiler.is_compiling():
            # opaque ops for the compiler (the reference's op boundary)
            q_input = torch.empty(M, K, dtype=FP8, device=x2.device)
            input_scale = _alloc_colmajor_scale(M, G, x2.device)
            output = torch.empty(M, N, dtype=torch.bfloat16, device=x2.device)
            torch.ops.kb_nano_fp8.per_token_group_quant_fp8(x2, q_input, input_scale, True)
            torch.ops.kb_nano_fp8.fp8_gemm_nt(q_input, input_scale, weight_fp8, weight_scale_inv, output)
        elif weight_scale_inv.dtype is torch.int32:
            # DeepGEMM's packed per-row UE8M0 scales (the layout the
            # reference's postprocess_fp8_weights returns, :501-510): UE8M0
            # activation quant, then the GEMM that takes the packed exponents
            if self._a_buf is not None and M <= self._a_buf.shape[0]:
                q_buf, s_buf, o_buf = self._a_buf, self._s_buf, self._o_buf
            elif self._pf is not None and M <= self._pf.a.shape[0]:
                q_buf, s_buf, o_buf = self._pf.a, self._pf.s, self._pf.o
            else:
                q_buf = torch.empty(M, K, dtype=FP8, device=x2.device)
                s_buf = _alloc_colmajor_scale(M, G, x2.device)
                o_buf = torch.empty(M, N, dtype=torch.bfloat16, device=x2.device)
            q, s = (q_buf, s_buf) if q_buf.shape[0] == M else (q_buf[:M], s_buf[:M])
            output = o_buf if o_buf.shape[0] == M else o_buf[:M]
            _ops.per_token_group_quant_fp8(x2, q, s, use_ue8m0=True, eps=_QUANT_EPS)
            _ops.fp8_gemm_nt(q, s, weight_fp8, weight_scale_inv, output)
        elif (M <= _ops.BF16A_MAX_M and x2.dtype is torch.bfloat16 and is_e8m0_used()
              and _ops.bf16a_preferred(M, N, K, x2.get_device())):
            # small M (the reference's bf16-input branch, :398-417): one
            # launch of the GEMM that quantizes its bf16 activations itself,
            # the same codes and scales as the quant launch would write, where
            # the library's plan says it is the faster of the two
            if self._o_buf is not None and M <= self._o_buf.shape[0]:
                o_buf = self._o_buf
            elif self._pf is not None and M <= self._pf.o.shape[0]:
                o_buf = self._pf.o
            else:
                o_buf = torch.empty(M, N, dtype=torch.bfloat16, device=x2.device)
            output = o_buf if o_buf.shape[0] == M else o_buf[:M]
            _ops.fp8_gemm_bf16a(x2, weight_fp8, weight_scale_inv, output)
        else:
            # eager: both launches through one library call; the installed
            # decode / prefill buffers (scales included: any row stride works)
            # are written in place without slicing, else fresh ones
            if self._a_buf is not None and M <= self._a_buf.shape[0]:
                q_buf, s_buf, o_buf = self._a_buf, self._s_buf, self._o_buf
            elif self._pf is not None and M <= self._pf.a.shape[0]:
                q_buf, s_buf, o_buf = self._pf.a, self._pf.s, self._pf.o
            else:
                q_buf = torch.empty(M, K, dtype=FP8, device=x2.device)
                s_buf = _alloc_colmajor_scale(M, G, x2.device)
                o_buf = torch.empty(M, N, dtype=torch.bfloat16, device=x2.device)
            output = o_buf if o_buf.shape[0] == M else o_buf[:M]
            if x2.dtype is torch.bfloat16:
                _ops.fp8_linear_forward(x2, q_buf, s_buf, weight_fp8, weight_scale_inv, o_buf)
            else:
                # fp16 / fp32 activations, which the reference's quant also
                # takes (widened to fp32): the quant, then the GEMM
                q, s = (q_buf, s_buf) if q_buf.shape[0] == M else (q_buf[:M], s_buf[:M])
                _ops.per_token_group_quant_fp8(x2, q, s, use_ue8m0=True, eps=_QUANT_EPS)
                _ops.fp8_gemm_nt(q, s, weight_fp8, weight_scale_inv, output)

        if bias is not None:
            output = output + bias
        return output if flat else output.view(*in_shape[:-1], N)


# ---------------------------------------------------------------------------
# Load-time weight processing
# ---------------------------------------------------------------------------

def _block_requant(w_f32: torch.Tensor, use_ue8m0: bool, eps: float = 1e-4):
    """128x128 block quantization of a float32 [N,K] (or [E,N,K]) weight on
    its device, in one gfx950 launch (``kbn_fp8_block_requant``).

    DeepGEMM v2.1.1.post3's ``per_block_cast_to_fp8`` (pyproject.toml:21;
    called at fp8_linear.py:497-499): ragged blocks pad with zeros, amax per
    block clamped to ``eps``, sf = amax/448 rounded up to a power of two under
    UE8M0, codes = fp8(x * (1/sf)).  Returns (fp8, fp32 [(E,) ceil(N/128),
    ceil(K/128)])."""
    N, K = w_f32.shape[-2:]
    NB, KB = math.ceil(N / GROUP), math.ceil(K / GROUP)
    w = w_f32 if w_f32.is_contiguous() else w_f32.contiguous()
    q = torch.empty(w.shape, dtype=FP8, device=w.device)
    s = torch.empty(w.shape[:-2] + (NB, KB), dtype=torch.float32, device=w.device)
    _ops.fp8_block_requant(w, None, q, s, use_ue8m0, eps)
    return q, s


def postprocess_fp8_weights(weight_fp8: torch.Tensor, scale_inv: torch.Tensor):
    """Re-quantize a checkpoint's fp8 weight to the scale format the GEMM
    consumes (reference :453-512): each 128x128 block is dequantized with its
    fp32 scale and re-quantized, with power-of-two scales under the UE8M0
    contract, in one gfx950 launch that reads and writes one byte per element.
    The scale layout stays the canonical fp32 [ceil(N/128), ceil(K/128)] (the
    kernels read it directly, so DeepGEMM's layout transform has no
    counterpart).  Returns new (weight, scale) tensors."""
    N, K = weight_fp8.shape
    NB, KB = math.ceil(N / GROUP), math.ceil(K / GROUP)
    w = torch.empty_like(weight_fp8)
    s = torch.empty(NB, KB, dtype=torch.float32, device=weight_fp8.device)
    _ops.fp8_block_requant(weight_fp8.contiguous(), scale_inv.to(torch.float32), w, s, is_e8m0_used(), 1e-4)
    return w, s


def postprocess_fp8_weights_batched(weight_fp8: torch.Tensor, scale_inv: torch.Tensor) -> None:
    """In-place version for MoE weights [E,N,K] / scales [E, >= ceil(N/128),
    >= ceil(K/128)] (reference :515-554), all experts in one launch."""
    assert weight_fp8.ndim == 3
    if scale_inv.dtype != torch.float32:
        raise TypeError("postprocess_fp8_weights_batched: scale_inv must be float32 to be rewritten in place")
    _ops.fp8_block_requant(weight_fp8, scale_inv, weight_fp8, scale_inv, is_e8m0_used(), 1e-4)