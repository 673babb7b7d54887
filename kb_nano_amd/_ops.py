"""Tensor-level wrappers over the C-ABI and the opaque ``torch.library`` ops.

Every wrapper validates dtype, device, shape and strides on the host, then
launches on the caller's current HIP stream.  Nothing here synchronises or
computes on the CPU; the only device memory taken is kernel workspace from
torch's caching allocator (stream-ordered, and served from the graph's pool
under capture), so the ops are safe inside HIP-graph capture and stay opaque
to ``torch.compile``.

Op schemas follow the reference (tasks/baseline/L1/fp8_linear.py:89-178 and
tasks/baseline/L1/fp8_grouped_gemm_contiguous.py:100-133).  The reference
creates its namespaces with ``Library(..., "DEF")``; this package owns the
same names on ROCm (the reference module cannot import there: it needs
``deep_gemm``), and uses ``FRAGMENT`` so a second registration in one
process is a no-op rather than an error.
"""
from __future__ import annotations

import functools
import os

import torch

from ._lib import check, lib, require_gfx950

FP8 = torch.float8_e4m3fn
GROUP = 128
QUANT_EPS = 1e-10  # tasks/baseline/L1/fp8_linear.py:44


# The per-call host path is kept short (it is paid on every eager launch):
# device indices come from Tensor.get_device() and the launch stream from
# the raw current-stream query, about 0.1 us each where torch.cuda's
# device/stream objects cost about 2 us.
_raw_stream = torch._C._cuda_getCurrentRawStream
_cur_device = torch._C._cuda_getDevice
_capturing = torch._C._cuda_isCurrentStreamCapturing
_GFX950_DEVICES: set = set()
_BF16 = torch.bfloat16
_F32 = torch.float32
# input dtype codes of kbn_per_token_group_quant_fp8_typed
_QUANT_IN = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _stream(t: torch.Tensor) -> int:
    """Raw handle of the current HIP stream of t's device."""
    return _raw_stream(t.get_device())


def _dev_check(what: str, *tensors: torch.Tensor) -> int:
    """All tensors on one gfx950 GPU, the current device; returns its index."""
    idx = tensors[0].get_device()
    if idx < 0:
        raise RuntimeError(f"{what}: tensors must be on a ROCm GPU, got {tensors[0].device} (no CPU path)")
    for t in tensors:
        if t.get_device() != idx:
            raise RuntimeError(f"{what}: all tensors must be on {tensors[0].device}, got {t.device}")
    if idx not in _GFX950_DEVICES:
        require_gfx950(idx)
        _GFX950_DEVICES.add(idx)
    if idx != torch._C._cuda_getDevice():
        raise RuntimeError(f"{what}: tensors are on cuda:{idx} but the current device is "
                           f"cuda:{torch.cuda.current_device()}; wrap the call in torch.cuda.device()")
    return idx


def _dtype_check(what: str, t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{what}: {name} must be {dtype}, got {t.dtype}")


@functools.cache
def is_e8m0_used() -> bool:
    """Whether the GEMM ops treat block scales under the UE8M0 contract.

    Mirrors ``_is_deep_gemm_e8m0_used`` (tasks/baseline/L1/
    fp8_grouped_gemm_contiguous.py:53-71): on by default, switched off by
    ``VLLM_USE_DEEP_GEMM=0`` or ``VLLM_USE_DEEP_GEMM_E8M0=0``.  Under the
    UE8M0 contract each fp32 scale is rounded up to a power of two and applied
    inside the block-scaled MFMA; otherwise scales are used as given."""
    if not bool(int(os.environ.get("VLLM_USE_DEEP_GEMM", "1"))):
        return False
    return bool(int(os.environ.get("VLLM_USE_DEEP_GEMM_E8M0", "1")))


# ---------------------------------------------------------------------------
# Raw launchers
# ---------------------------------------------------------------------------

def per_token_group_quant_fp8(x: torch.Tensor, out_fp8: torch.Tensor, out_scale: torch.Tensor,
                              use_ue8m0: bool = True, eps: float = QUANT_EPS) -> None:
    """1x128 quant of ``x [M,K]`` into ``out_fp8 [M,K]`` and ``out_scale
    [M,K/128]`` (any strides for the scales, e.g. column-major).  ``x`` is
    bf16, or fp16 / fp32 as the reference's kernel also takes (its values
    widened to fp32 exactly, tasks/baseline/L1/fp8_linear.py:197)."""
    what = "per_token_group_quant_fp8"
    idx = x.get_device()
    shape = x.shape
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or out_fp8.get_device() != idx
            or out_scale.get_device() != idx):
        _dev_check(what, x, out_fp8, out_scale)
    if x.dtype is not _BF16 or out_fp8.dtype is not FP8 or out_scale.dtype is not _F32:
        if x.dtype not in _QUANT_IN:
            raise TypeError(f"{what}: input must be bfloat16, float16 or float32, got {x.dtype}")
        _dtype_check(what, out_fp8, FP8, "output_fp8")
        _dtype_check(what, out_scale, torch.float32, "output_scale")
    if len(shape) != 2 or out_fp8.shape != shape:
        raise ValueError(f"{what}: expected 2-D input and matching output, got {tuple(x.shape)} / {tuple(out_fp8.shape)}")
    M, K = shape
    if K % GROUP:
        raise ValueError(f"{what}: K={K} must be a multiple of {GROUP}")
    if out_scale.shape != (M, K // GROUP):
        raise ValueError(f"{what}: output_scale must be {(M, K // GROUP)}, got {tuple(out_scale.shape)}")
    xs, qs, ss = x.stride(), out_fp8.stride(), out_scale.stride()
    if xs[1] != 1 or qs[1] != 1:
        raise ValueError(f"{what}: input and output rows must be contiguous")
    if x.dtype is _BF16:
        rc = lib().kbn_per_token_group_quant_fp8(
            x.data_ptr(), M, K, xs[0], out_fp8.data_ptr(), qs[0], out_scale.data_ptr(), ss[0], ss[1],
            float(eps), 1 if use_ue8m0 else 0, _raw_stream(idx))
    else:
        rc = lib().kbn_per_token_group_quant_fp8_typed(
            x.data_ptr(), _QUANT_IN[x.dtype], M, K, xs[0], out_fp8.data_ptr(), qs[0], out_scale.data_ptr(),
            ss[0], ss[1], float(eps), 1 if use_ue8m0 else 0, _raw_stream(idx))
    if rc:
        check(rc, what)


def silu_mul_quant_fp8(inp: torch.Tensor, out_fp8: torch.Tensor, out_scale: torch.Tensor,
                       use_ue8m0: bool = True, eps: float = QUANT_EPS, row_ids: torch.Tensor | None = None) -> None:
    """y = bf16(silu(gate) * up) for ``inp = [gate | up]`` (bf16 [M, 2N']),
    quantized 1x128 into ``out_fp8 [M,N']`` and ``out_scale [M, N'/128]``.
    With ``row_ids`` (int32 [M], e.g. the contiguous MoE layout's expert ids),
    rows whose id is negative are neither read nor written."""
    what = "silu_mul_quant_fp8"
    idx = inp.get_device()
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or out_fp8.get_device() != idx
            or out_scale.get_device() != idx):
        _dev_check(what, inp, out_fp8, out_scale)
    if inp.dtype is not _BF16 or out_fp8.dtype is not FP8 or out_scale.dtype is not _F32:
        _dtype_check(what, inp, torch.bfloat16, "input")
        _dtype_check(what, out_fp8, FP8, "output")
        _dtype_check(what, out_scale, torch.float32, "output_scales")
    M, N = inp.shape
    Nh = N // 2
    if out_fp8.shape != (M, Nh) or out_scale.shape != (M, Nh // GROUP):
        raise ValueError(f"{what}: bad output shapes {tuple(out_fp8.shape)} / {tuple(out_scale.shape)}")
    xs, qs, ss = inp.stride(), out_fp8.stride(), out_scale.stride()
    if xs[1] != 1 or qs[1] != 1:
        raise ValueError(f"{what}: input and output rows must be contiguous")
    if row_ids is not None:
        if (row_ids.get_device() != idx or row_ids.dtype is not torch.int32 or row_ids.dim() != 1
                or row_ids.shape[0] < M or (M > 1 and row_ids.stride(0) != 1)):
            raise ValueError(f"{what}: row_ids must be a contiguous int32 vector of at least M={M} on the input's device")
        rc = lib().kbn_silu_mul_quant_fp8_rows(
            inp.data_ptr(), M, Nh, xs[0], out_fp8.data_ptr(), qs[0], out_scale.data_ptr(), ss[0], ss[1],
            float(eps), 1 if use_ue8m0 else 0, row_ids.data_ptr(), _raw_stream(idx))
        if rc:
            check(rc, what)
        return
    rc = lib().kbn_silu_mul_quant_fp8(
        inp.data_ptr(), M, Nh, xs[0], out_fp8.data_ptr(), qs[0], out_scale.data_ptr(), ss[0], ss[1],
        float(eps), 1 if use_ue8m0 else 0, _raw_stream(idx))
    if rc:
        check(rc, what)


def fp8_gemm_nt(q_input: torch.Tensor, input_scale: torch.Tensor, weight: torch.Tensor,
                weight_scale: torch.Tensor, output: torch.Tensor, use_ue8m0: bool | None = None) -> None:
    """output[M,N] (bf16) = block-scaled q_input[M,K] x weight[N,K]^T.

    ``weight_scale`` is fp32 [ceil(N/128), ceil(K/128)] block scales, or
    DeepGEMM's packed per-row UE8M0 exponents, int32 [N, ceil(K/512)] (any
    strides), the layout postprocess_fp8_weights hands the reference's GEMM
    (tasks/baseline/L1/fp8_linear.py:501-510); those are UE8M0 by nature."""
    what = "fp8_gemm_nt"
    if weight_scale.dtype is torch.int32:
        _fp8_gemm_nt_packed(q_input, input_scale, weight, weight_scale, output)
        return
    idx = q_input.get_device()
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or input_scale.get_device() != idx
            or weight.get_device() != idx or weight_scale.get_device() != idx or output.get_device() != idx):
        _dev_check(what, q_input, input_scale, weight, weight_scale, output)
    if (q_input.dtype is not FP8 or weight.dtype is not FP8 or input_scale.dtype is not _F32
            or weight_scale.dtype is not _F32 or output.dtype is not _BF16):
        _dtype_check(what, q_input, FP8, "q_input")
        _dtype_check(what, weight, FP8, "weight")
        _dtype_check(what, input_scale, torch.float32, "input_scale")
        _dtype_check(what, weight_scale, torch.float32, "weight_scale")
        _dtype_check(what, output, torch.bfloat16, "output")
    M, K = q_input.shape
    N, K2 = weight.shape
    if K2 != K:
        raise ValueError(f"{what}: K mismatch {K} vs {K2}")
    if output.shape != (M, N):
        raise ValueError(f"{what}: output must be {(M, N)}, got {tuple(output.shape)}")
    KB, NB = -(-K // GROUP), -(-N // GROUP)
    if input_scale.shape != (M, KB):
        raise ValueError(f"{what}: input_scale must be {(M, KB)}, got {tuple(input_scale.shape)}")
    sws = weight_scale.shape
    if len(sws) != 2 or sws[0] < NB or sws[1] < KB:
        raise ValueError(f"{what}: weight_scale must be at least {(NB, KB)}, got {tuple(weight_scale.shape)}")
    qs, ss, ws_, sws_, os_ = q_input.stride(), input_scale.stride(), weight.stride(), weight_scale.stride(), \
        output.stride()
    if qs[1] != 1 or ws_[1] != 1 or os_[1] != 1 or sws_[1] != 1:
        raise ValueError(f"{what}: operands must be contiguous along K (and N for the output)")
    ue8m0 = is_e8m0_used() if use_ue8m0 is None else bool(use_ue8m0)
    if M == 0 or N == 0:
        return
    L = lib()
    # small-M / few-tile shapes split K over more workgroups; the fp32
    # partials live in the launch stream's workspace (_workspace), so
    # concurrent streams never share one
    ws_bytes = _gemm_workspace_bytes(L, idx, M, N, K, ue8m0)
    st = _raw_stream(idx)
    ws = _workspace(ws_bytes, idx, st, output) if ws_bytes else None
    rc = L.kbn_fp8_gemm_nt_ws(
        q_input.data_ptr(), qs[0], input_scale.data_ptr(), ss[0], ss[1], weight.data_ptr(), ws_[0],
        weight_scale.data_ptr(), sws_[0], output.data_ptr(), os_[0], M, N, K, 1 if ue8m0 else 0,
        ws.data_ptr() if ws is not None else None, ws_bytes, st)
    if rc:
        check(rc, what)


def _fp8_gemm_nt_packed(q_input, input_scale, weight, weight_scale, output) -> None:
    """fp8_gemm_nt with packed per-row UE8M0 weight scales (kbn_fp8_gemm_nt_packed_ws)."""
    what = "fp8_gemm_nt"
    idx = _dev_check(what, q_input, input_scale, weight, weight_scale, output)
    _dtype_check(what, q_input, FP8, "q_input")
    _dtype_check(what, weight, FP8, "weight")
    _dtype_check(what, input_scale, torch.float32, "input_scale")
    _dtype_check(what, output, torch.bfloat16, "output")
    M, K = q_input.shape
    N, K2 = weight.shape
    if K2 != K or output.shape != (M, N):
        raise ValueError(f"{what}: shapes q {tuple(q_input.shape)}, W {tuple(weight.shape)}, out {tuple(output.shape)}")
    KB, words = -(-K // GROUP), -(-K // (4 * GROUP))
    if input_scale.shape != (M, KB):
        raise ValueError(f"{what}: input_scale must be {(M, KB)}, got {tuple(input_scale.shape)}")
    if weight_scale.dim() != 2 or weight_scale.shape[0] < N or weight_scale.shape[1] < words:
        raise ValueError(f"{what}: packed int32 weight_scale must be at least {(N, words)} "
                         f"(N, ceil(K/512)), got {tuple(weight_scale.shape)}")
    qs, ss, ws_, os_ = q_input.stride(), input_scale.stride(), weight.stride(), output.stride()
    if qs[1] != 1 or ws_[1] != 1 or os_[1] != 1:
        raise ValueError(f"{what}: operands must be contiguous along K (and N for the output)")
    if M == 0 or N == 0:
        return
    L = lib()
    ws_bytes = _gemm_workspace_bytes(L, idx, M, N, K, True)
    st = _raw_stream(idx)
    ws = _workspace(ws_bytes, idx, st, output) if ws_bytes else None
    wss = weight_scale.stride()
    check(L.kbn_fp8_gemm_nt_packed_ws(
        q_input.data_ptr(), qs[0], input_scale.data_ptr(), ss[0], ss[1], weight.data_ptr(), ws_[0],
        weight_scale.data_ptr(), wss[0], wss[1], output.data_ptr(), os_[0], M, N, K,
        ws.data_ptr() if ws is not None else None, ws_bytes, st), what)


def pack_ue8m0_weight_scales(block_scales: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """DeepGEMM's packed per-row UE8M0 layout of 128x128 block scales (what
    transform_sf_into_required_layout makes of them for the weights,
    tasks/baseline/L1/fp8_linear.py:501-510): int32 [N, ceil(K/512)], byte j of
    word (n, i) the E8M0 exponent of the (power-of-two, else rounded up)
    block scale of row n, K block 4i + j, stored MN-major (strides (1, N')
    with N' = N rounded up to a multiple of 4), as DeepGEMM stores it."""
    KB = -(-K // GROUP)
    words = -(-KB // 4)
    s = block_scales[: -(-N // GROUP), :KB].to(torch.float32)
    bits = s.contiguous().view(torch.int32)
    e = (bits >> 23) & 0xFF
    e = e + ((bits & 0x7FFFFF) != 0).to(torch.int32)          # round up to a power of two
    e = torch.clamp(e, max=254)
    rows = e.repeat_interleave(GROUP, dim=0)[:N]                # [N, KB]
    if KB % 4:
        rows = torch.nn.functional.pad(rows, (0, 4 * words - KB))
    b = rows.to(torch.uint8).view(N, words, 4).to(torch.int32)
    packed = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)
    n_al = -(-N // 4) * 4
    out = torch.empty(words, n_al, dtype=torch.int32, device=block_scales.device)
    out[:, :N] = packed.t()
    if n_al > N:
        out[:, N:] = 0
    return out.t()[:N]


def fp8_linear_forward(x: torch.Tensor, q_buf: torch.Tensor, s_buf: torch.Tensor, weight: torch.Tensor,
                       weight_scale: torch.Tensor, out_buf: torch.Tensor, use_ue8m0: bool | None = None) -> None:
    """Fp8Linear.forward's launches in one library call: the 1x128 UE8M0
    quant of ``x [M, K]`` into rows [0, M) of ``q_buf`` and ``s_buf`` (any
    strides, e.g. a column-major buffer of more rows), then
    ``out_buf[:M] = block-scaled q x weight^T``.  Buffers may hold more than
    M rows; only the first M are written."""
    what = "fp8_linear_forward"
    idx = x.get_device()
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or q_buf.get_device() != idx
            or s_buf.get_device() != idx or weight.get_device() != idx or weight_scale.get_device() != idx
            or out_buf.get_device() != idx):
        _dev_check(what, x, q_buf, s_buf, weight, weight_scale, out_buf)
    if (x.dtype is not _BF16 or q_buf.dtype is not FP8 or weight.dtype is not FP8 or s_buf.dtype is not _F32
            or weight_scale.dtype is not _F32 or out_buf.dtype is not _BF16):
        raise TypeError(f"{what}: expected bf16 x, fp8 q_buf/weight, fp32 scales, bf16 out_buf")
    M, K = x.shape
    N, K2 = weight.shape
    KB, NB = -(-K // GROUP), -(-N // GROUP)
    qsh, ssh, osh, wssh = q_buf.shape, s_buf.shape, out_buf.shape, weight_scale.shape
    if (K2 != K or K % GROUP or qsh[0] < M or qsh[1] != K or ssh[0] < M or ssh[1] != KB or osh[0] < M
            or osh[1] != N or len(wssh) != 2 or wssh[0] < NB or wssh[1] < KB):
        raise ValueError(f"{what}: shapes x {tuple(x.shape)}, q {tuple(q_buf.shape)}, s {tuple(s_buf.shape)}, "
                         f"W {tuple(weight.shape)}, sW {tuple(weight_scale.shape)}, out {tuple(out_buf.shape)}")
    xs, qs, ss, ws_, wss, os_ = x.stride(), q_buf.stride(), s_buf.stride(), weight.stride(), \
        weight_scale.stride(), out_buf.stride()
    if xs[1] != 1 or qs[1] != 1 or ws_[1] != 1 or os_[1] != 1 or wss[1] != 1:
        raise ValueError(f"{what}: rows must be contiguous")
    if M == 0 or N == 0:
        return
    ue8m0 = is_e8m0_used() if use_ue8m0 is None else bool(use_ue8m0)
    L = lib()
    ws_bytes = _gemm_workspace_bytes(L, idx, M, N, K, ue8m0)
    st = _raw_stream(idx)
    ws = _workspace(ws_bytes, idx, st, out_buf) if ws_bytes else None
    rc = L.kbn_fp8_linear_forward(
        x.data_ptr(), M, K, xs[0], q_buf.data_ptr(), qs[0], s_buf.data_ptr(), ss[0], ss[1], QUANT_EPS, 1,
        weight.data_ptr(), ws_[0], weight_scale.data_ptr(), wss[0], out_buf.data_ptr(), os_[0], N,
        1 if ue8m0 else 0, ws.data_ptr() if ws is not None else None, ws_bytes, st)
    if rc:
        check(rc, what)


BF16A_MAX_M = 64   # rows the bf16-activation GEMM covers (its 64-row tiles)


def fp8_gemm_bf16a(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
                   eps: float = QUANT_EPS) -> None:
    """``output[M, N] = block-scaled quant(x) x weight^T`` for bf16 ``x [M, K]``
    with M <= 64, the 1x128 UE8M0 activation quant done inside the GEMM
    kernel (one launch, no fp8 copy of ``x``).  The codes and scales are the
    ones ``per_token_group_quant_fp8`` produces, so the output equals that
    quant followed by ``fp8_gemm_nt`` bit for bit.

    The counterpart of the reference's small-M branch, which hands bf16
    activations to a GEMM that quantizes them itself
    (tasks/baseline/L1/fp8_linear.py:126-148 ``flashinfer_blockscale_gemm``,
    taken at :398-417 for M < 32)."""
    what = "fp8_gemm_bf16a"
    idx = x.get_device()
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or weight.get_device() != idx
            or weight_scale.get_device() != idx or output.get_device() != idx):
        _dev_check(what, x, weight, weight_scale, output)
    if x.dtype is not _BF16 or weight.dtype is not FP8 or weight_scale.dtype is not _F32 or output.dtype is not _BF16:
        raise TypeError(f"{what}: expected bf16 x, fp8 weight, fp32 weight_scale, bf16 output")
    xsh, wsh, wssh, osh = x.shape, weight.shape, weight_scale.shape, output.shape
    if len(xsh) != 2 or len(wsh) != 2 or len(wssh) != 2 or len(osh) != 2:
        raise ValueError(f"{what}: x, weight, weight_scale and output must be 2-D")
    M, K = xsh
    N = wsh[0]
    if (wsh[1] != K or K % GROUP or osh[0] != M or osh[1] != N or wssh[0] * GROUP < N
            or wssh[1] * GROUP < K):
        raise ValueError(f"{what}: shapes x {tuple(xsh)}, W {tuple(wsh)}, sW {tuple(wssh)}, out {tuple(osh)}")
    if M > BF16A_MAX_M:
        raise ValueError(f"{what}: M={M} > {BF16A_MAX_M}; quantize with per_token_group_quant_fp8 and use fp8_gemm_nt")
    xs, ws_, wss, os_ = x.stride(), weight.stride(), weight_scale.stride(), output.stride()
    if xs[1] != 1 or ws_[1] != 1 or os_[1] != 1 or wss[1] != 1:
        raise ValueError(f"{what}: rows must be contiguous")
    if M == 0 or N == 0:
        return
    L = lib()
    key = (idx, "bf16a", M, N, K)
    ws_bytes = _WS_CACHE.get(key)
    if ws_bytes is None:
        with torch.cuda.device(idx):
            ws_bytes = _WS_CACHE[key] = int(L.kbn_fp8_gemm_bf16a_workspace_bytes(M, N, K))
    st = _raw_stream(idx)
    ws = _workspace(ws_bytes, idx, st, output) if ws_bytes else None
    rc = L.kbn_fp8_gemm_bf16a(x.data_ptr(), xs[0], float(eps), weight.data_ptr(), ws_[0], weight_scale.data_ptr(),
                              wss[0], output.data_ptr(), os_[0], M, N, K,
                              ws.data_ptr() if ws is not None else None, ws_bytes, st)
    if rc:
        check(rc, what)


def flashinfer_blockscale_gemm(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                               output: torch.Tensor) -> None:
    """Implementation of the op ``kb_nano_fp8::flashinfer_blockscale_gemm``
    (reference tasks/baseline/L1/fp8_linear.py:126-153): bf16 activations
    ``x [M, K]``, fp8 weight ``[N, K]`` with fp32 block scales, bf16
    ``output [M, N]``, any M.  The reference op uses the weight scales as
    given; here the scale contract of the GEMM ops decides, as for
    ``fp8_gemm_nt``:

    * UE8M0 (``is_e8m0_used()``) and M <= 64: ``fp8_gemm_bf16a``, one launch
      that quantizes the activations itself;
    * otherwise (scales used as given, or more rows than that kernel's
      64-row tiles): the 1x128 quant of ``x`` into fresh buffers (UE8M0 scales
      only under that contract), then ``fp8_gemm_nt`` under the same
      contract, so non-power-of-two weight scales are never rounded unless
      the contract says so."""
    ue8m0 = is_e8m0_used()
    if x.dim() == 2 and ue8m0 and x.shape[0] <= BF16A_MAX_M:
        fp8_gemm_bf16a(x, weight, weight_scale, output)
        return
    if x.dim() != 2:
        raise ValueError(f"flashinfer_blockscale_gemm: x must be 2-D, got {tuple(x.shape)}")
    M, K = x.shape
    q = torch.empty(M, K, dtype=FP8, device=x.device)
    s = torch.empty_strided((M, -(-K // GROUP)), (1, max(M, 1)), dtype=torch.float32, device=x.device)
    per_token_group_quant_fp8(x if x.is_contiguous() else x.contiguous(), q, s, use_ue8m0=ue8m0)
    fp8_gemm_nt(q, s, weight, weight_scale, output, use_ue8m0=ue8m0)


def bf16a_preferred(M: int, N: int, K: int, idx: int) -> bool:
    """Whether ``fp8_gemm_bf16a`` is expected to beat quant + ``fp8_gemm_nt``
    for this shape on device idx (the library's plan-based rule); cached."""
    key = (idx, "bf16a?", M, N, K)
    r = _WS_CACHE.get(key)
    if r is None:
        with torch.cuda.device(idx):
            r = _WS_CACHE[key] = bool(lib().kbn_fp8_gemm_bf16a_preferred(M, N, K))
    return r


_WS_CACHE: dict = {}
_WS_BUFS: dict = {}


_SCALE_WRITES = [0]   # bumped by this package's in-place scale writers


def scales_are_pow2(s: torch.Tensor) -> bool:
    """Whether every element of the fp32 block-scale tensor ``s`` is a
    positive, finite power of two.  The block-scaled GEMMs then give the same
    bits under the UE8M0 and the FP32 scale contracts: the FP32 contract's
    per-block significands are all 1, so it never rescales its running sums.

    Checked on the device (one reduction and a synchronize) once per tensor
    object, storage and version; a view shares its base's version counter,
    and this package's in-place scale writers (``fp8_block_requant``) bump it.
    Inference tensors (``torch.inference_mode``) have no version counter:
    for them the check is redone after this package's in-place scale writes
    only, so a caller that rewrites such a tensor in place by other means
    sets the layer's ``ue8m0_when_exact`` to False.  During graph capture an
    unchecked tensor counts as not all powers of two (nothing synchronizes
    there)."""
    tag = getattr(s, "_kbn_pow2", None)
    key = (-1 if s.is_inference() else s._version, _SCALE_WRITES[0], s.data_ptr(), s.shape, s.stride())
    if tag is not None and tag[0] == key:
        return tag[1]
    if s.dtype is not torch.float32 or (s.is_cuda and _capturing()):
        return False
    b = s.view(torch.int32)
    e = (b >> 23) & 0xFF
    r = bool(((b & -0x7F800001) == 0).logical_and_(e != 0).logical_and_(e != 255).all())
    try:
        s._kbn_pow2 = (key, r)
    except AttributeError:   # a tensor type without attributes: checked again next time
        pass
    return r


def _workspace(nbytes: int, idx: int, stream: int, like: torch.Tensor) -> torch.Tensor:
    """Scratch for one launch on ``stream``.  Eager launches on a stream reuse
    one buffer per (device, stream), grown as needed: launches on a stream
    run in order, so a buffer is free again when the next launch on that
    stream reads it, and a replaced buffer goes back to the caching allocator,
    which hands it out again only in that stream's order.  Under graph capture
    every launch takes its own buffer from the capture's memory pool, as
    before (a graph keeps what it was captured with).  ``like`` is a tensor
    on the device (its device object is only built when allocating)."""
    if _capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=like.device)
    key = (idx, stream)
    buf = _WS_BUFS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=like.device)
        _WS_BUFS[key] = buf
    return buf


def release_workspaces(device: int | None = None) -> int:
    """Drop the eager split-K workspaces ``_workspace`` keeps per (device,
    stream), all of them or those of one device index; returns how many were
    dropped.  A buffer goes back to torch's caching allocator once no launch
    still uses it (stream-ordered), so a following ``torch.cuda.empty_cache()``
    can return it to the device.  Call it when streams are retired (each
    buffer grows to the largest split plan run on its stream, up to 64 MiB)
    or before measuring free memory; the next eager split launch on a stream
    allocates afresh.  Graph-captured launches hold their own buffers and
    are not affected."""
    keys = [k for k in _WS_BUFS if device is None or k[0] == device]
    for k in keys:
        del _WS_BUFS[k]
    return len(keys)


def splitk_counter_stats() -> dict:
    """State of the split-K arrival-counter regions (``kbn_splitk_counter_stats``):
    ``regions_used`` on the busiest device, ``regions_total`` per device and
    ``fallbacks``, the small-M split launches that ran the separate reduction
    kernel because every region was taken (one region per eager stream and
    per captured stream, held for the life of the process).  A non-zero
    ``fallbacks`` means results as usual but one launch more per such call:
    an engine that re-captures graphs many times should reuse its graphs
    instead."""
    import ctypes
    used, total, fb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(lib().kbn_splitk_counter_stats(ctypes.byref(used), ctypes.byref(total), ctypes.byref(fb)),
          "splitk_counter_stats")
    return {"regions_used": used.value, "regions_total": total.value, "fallbacks": fb.value}


def _gemm_workspace_bytes(L, idx: int, M, N, K, ue8m0) -> int:
    """Split-K workspace of a shape on device idx (the plan depends on the
    device's CU count); cached per (device, shape)."""
    key = (idx, M, N, K, ue8m0)
    n = _WS_CACHE.get(key)
    if n is None:
        with torch.cuda.device(idx):
            n = int(L.kbn_fp8_gemm_nt_workspace_bytes(M, N, K, int(ue8m0)))
        _WS_CACHE[key] = n
    return n


def m_grouped_gemm_nt_contiguous(a_fp8: torch.Tensor, a_scale: torch.Tensor, b_fp8: torch.Tensor,
                                 b_scale: torch.Tensor, c_bf16: torch.Tensor, expert_ids: torch.Tensor,
                                 disable_ue8m0_cast: bool) -> None:
    """Contiguous-layout grouped GEMM: row r of ``a_fp8`` multiplies expert
    ``expert_ids[r]`` of ``b_fp8``; rows with id -1 are left unwritten."""
    what = "m_grouped_gemm_nt_contiguous"
    _dev_check(what, a_fp8, a_scale, b_fp8, b_scale, c_bf16, expert_ids)
    _dtype_check(what, a_fp8, FP8, "a_fp8")
    _dtype_check(what, b_fp8, FP8, "b_fp8")
    _dtype_check(what, a_scale, torch.float32, "a_scale")
    _dtype_check(what, b_scale, torch.float32, "b_scale")
    _dtype_check(what, c_bf16, torch.bfloat16, "c_bf16")
    _dtype_check(what, expert_ids, torch.int32, "expert_ids")
    M_sum, K = a_fp8.shape
    E, N, K2 = b_fp8.shape
    if K2 != K:
        raise ValueError(f"{what}: K mismatch {K} vs {K2}")
    KB, NB = -(-K // GROUP), -(-N // GROUP)
    if tuple(c_bf16.shape) != (M_sum, N) or tuple(expert_ids.shape) != (M_sum,):
        raise ValueError(f"{what}: c_bf16 must be {(M_sum, N)} and expert_ids {(M_sum,)}")
    if tuple(a_scale.shape) != (M_sum, KB) or tuple(b_scale.shape) != (E, NB, KB):
        raise ValueError(f"{what}: scales must be {(M_sum, KB)} and {(E, NB, KB)}, got "
                         f"{tuple(a_scale.shape)} / {tuple(b_scale.shape)}")
    if not (b_fp8.is_contiguous() and b_scale.is_contiguous() and expert_ids.is_contiguous()):
        raise ValueError(f"{what}: b_fp8, b_scale and expert_ids must be contiguous")
    if a_fp8.stride(1) != 1 or c_bf16.stride(1) != 1:
        raise ValueError(f"{what}: a_fp8 and c_bf16 rows must be contiguous")
    check(lib().kbn_fp8_grouped_gemm_nt_contiguous(
        a_fp8.data_ptr(), a_fp8.stride(0), a_scale.data_ptr(), a_scale.stride(0), a_scale.stride(1),
        b_fp8.data_ptr(), b_scale.data_ptr(), c_bf16.data_ptr(), c_bf16.stride(0), expert_ids.data_ptr(),
        M_sum, N, K, E, int(not disable_ue8m0_cast), _stream(c_bf16)), what)


def grouped_gemm_silu_quant(a_fp8: torch.Tensor, a_scale: torch.Tensor, b_fp8: torch.Tensor, b_scale: torch.Tensor,
                            expert_ids: torch.Tensor, disable_ue8m0_cast: bool, out_fp8: torch.Tensor,
                            out_scale: torch.Tensor, use_ue8m0: bool = True, eps: float = QUANT_EPS) -> None:
    """The contiguous grouped GEMM of ``b_fp8 [E, N2, K]`` (rows [0, N2/2) the
    gate, [N2/2, N2) the up projection) with SiLU*Mul + 1x128 quant in its
    epilogue: ``out_fp8 [M_sum, N2/2]`` and ``out_scale [M_sum, N2/256]`` get
    exactly what ``m_grouped_gemm_nt_contiguous`` into a bf16 buffer followed
    by ``silu_mul_quant_fp8(buffer, row_ids=expert_ids)`` writes; rows with id
    -1 are not written."""
    what = "grouped_gemm_silu_quant"
    _dev_check(what, a_fp8, a_scale, b_fp8, b_scale, expert_ids, out_fp8, out_scale)
    _dtype_check(what, a_fp8, FP8, "a_fp8")
    _dtype_check(what, b_fp8, FP8, "b_fp8")
    _dtype_check(what, a_scale, torch.float32, "a_scale")
    _dtype_check(what, b_scale, torch.float32, "b_scale")
    _dtype_check(what, expert_ids, torch.int32, "expert_ids")
    _dtype_check(what, out_fp8, FP8, "out_fp8")
    _dtype_check(what, out_scale, torch.float32, "out_scale")
    M_sum, K = a_fp8.shape
    E, N2, K2 = b_fp8.shape
    if K2 != K or N2 % 256:
        raise ValueError(f"{what}: K mismatch {K} vs {K2} or N2={N2} not a multiple of 256")
    KB, NB = -(-K // GROUP), N2 // GROUP
    if tuple(out_fp8.shape) != (M_sum, N2 // 2) or tuple(out_scale.shape) != (M_sum, N2 // 2 // GROUP):
        raise ValueError(f"{what}: outputs must be {(M_sum, N2 // 2)} and {(M_sum, N2 // 2 // GROUP)}")
    if tuple(expert_ids.shape) != (M_sum,):
        raise ValueError(f"{what}: expert_ids must be {(M_sum,)}")
    if tuple(a_scale.shape) != (M_sum, KB) or tuple(b_scale.shape) != (E, NB, KB):
        raise ValueError(f"{what}: scales must be {(M_sum, KB)} and {(E, NB, KB)}, got "
                         f"{tuple(a_scale.shape)} / {tuple(b_scale.shape)}")
    if not (b_fp8.is_contiguous() and b_scale.is_contiguous() and expert_ids.is_contiguous()):
        raise ValueError(f"{what}: b_fp8, b_scale and expert_ids must be contiguous")
    if a_fp8.stride(1) != 1 or out_fp8.stride(1) != 1:
        raise ValueError(f"{what}: a_fp8 and out_fp8 rows must be contiguous")
    check(lib().kbn_fp8_grouped_gemm_silu_quant(
        a_fp8.data_ptr(), a_fp8.stride(0), a_scale.data_ptr(), a_scale.stride(0), a_scale.stride(1),
        b_fp8.data_ptr(), b_scale.data_ptr(), expert_ids.data_ptr(), M_sum, N2, K, E, int(not disable_ue8m0_cast),
        out_fp8.data_ptr(), out_fp8.stride(0), out_scale.data_ptr(), out_scale.stride(0), out_scale.stride(1),
        float(eps), int(use_ue8m0), _stream(out_fp8)), what)


def moe_permute_contiguous(x: torch.Tensor, x_scale: torch.Tensor, topk_ids: torch.Tensor, num_experts: int,
                           alignment: int, M_sum: int, x_perm: torch.Tensor, scale_perm: torch.Tensor,
                           expert_ids: torch.Tensor, inv_perm: torch.Tensor, zero_padding: bool = True) -> None:
    """Scatter the rows of ``x [M, K]`` and ``x_scale [M, K/128]`` into the
    expert-contiguous layout ``x_perm [M_sum, K]`` / ``scale_perm`` (row- or
    column-major), writing ``expert_ids [M_sum]`` and ``inv_perm [M, top_k]``
    (int32)."""
    what = "moe_permute_contiguous"
    _dev_check(what, x, x_scale, topk_ids, x_perm, scale_perm, expert_ids, inv_perm)
    _dtype_check(what, x_scale, torch.float32, "x_scale")
    _dtype_check(what, scale_perm, torch.float32, "scale_perm")
    _dtype_check(what, expert_ids, torch.int32, "expert_ids")
    _dtype_check(what, inv_perm, torch.int32, "inv_perm")
    if x_perm.dtype != x.dtype:
        raise TypeError(f"{what}: x_perm must be {x.dtype}, got {x_perm.dtype}")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{what}: topk_ids must be int32 or int64, got {topk_ids.dtype}")
    if x.dim() != 2 or topk_ids.dim() != 2 or topk_ids.shape[0] != x.shape[0]:
        raise ValueError(f"{what}: x [M, K] and topk_ids [M, top_k] expected, got {tuple(x.shape)} and "
                         f"{tuple(topk_ids.shape)}")
    M, K = x.shape
    top_k = topk_ids.shape[1]
    cols = K // GROUP
    if tuple(x_scale.shape) != (M, cols):
        raise ValueError(f"{what}: x_scale must be {(M, cols)}, got {tuple(x_scale.shape)}")
    if tuple(x_perm.shape) != (M_sum, K) or tuple(scale_perm.shape) != (M_sum, cols):
        raise ValueError(f"{what}: outputs must be {(M_sum, K)} and {(M_sum, cols)}")
    if tuple(expert_ids.shape) != (M_sum,) or tuple(inv_perm.shape) != (M, top_k):
        raise ValueError(f"{what}: expert_ids must be {(M_sum,)} and inv_perm {(M, top_k)}")
    for t, name in ((topk_ids, "topk_ids"), (x_perm, "x_perm"), (expert_ids, "expert_ids"), (inv_perm, "inv_perm")):
        if not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be contiguous")
    esz = x.element_size()
    if x.stride(1) != 1 and M > 1:
        raise ValueError(f"{what}: rows of x must be contiguous")
    L = lib()
    ws_bytes = int(L.kbn_moe_permute_workspace_bytes(M * top_k, num_experts))
    if ws_bytes < 0:
        raise ValueError(f"{what}: num_experts={num_experts} outside [1, 1024] or too many pairs")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    check(L.kbn_moe_permute_contiguous(
        topk_ids.data_ptr(), topk_ids.element_size(), M, top_k, num_experts, alignment,
        x.data_ptr() if M else None, x.stride(0) * esz, K * esz, x_scale.data_ptr() if M else None,
        x_scale.stride(0), x_scale.stride(1), cols, M_sum, x_perm.data_ptr(), scale_perm.data_ptr(),
        scale_perm.stride(0), scale_perm.stride(1), expert_ids.data_ptr(), inv_perm.data_ptr(), int(zero_padding),
        ws.data_ptr(), ws_bytes,
        _stream(x_perm)), what)


def moe_permute_quant_contiguous(x: torch.Tensor, topk_ids: torch.Tensor, num_experts: int, alignment: int,
                                 M_sum: int, x_perm: torch.Tensor, scale_perm: torch.Tensor,
                                 expert_ids: torch.Tensor, inv_perm: torch.Tensor, zero_padding: bool = True,
                                 use_ue8m0: bool = True, eps: float = QUANT_EPS) -> None:
    """``per_token_group_quant_fp8(x)`` followed by ``moe_permute_contiguous``
    in one launch: each bf16 row of ``x [M, K]`` is quantized 1x128 once and
    its codes and scales are written to the expert-contiguous rows of all the
    token's routed pairs (``x_perm`` fp8 [M_sum, K], ``scale_perm`` fp32
    [M_sum, K/128], row- or column-major), with ``expert_ids`` and
    ``inv_perm`` as the permute writes them; the same bytes as the two
    launches."""
    what = "moe_permute_quant_contiguous"
    _dev_check(what, x, topk_ids, x_perm, scale_perm, expert_ids, inv_perm)
    _dtype_check(what, x, _BF16, "x")
    _dtype_check(what, x_perm, FP8, "x_perm")
    _dtype_check(what, scale_perm, torch.float32, "scale_perm")
    _dtype_check(what, expert_ids, torch.int32, "expert_ids")
    _dtype_check(what, inv_perm, torch.int32, "inv_perm")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{what}: topk_ids must be int32 or int64, got {topk_ids.dtype}")
    if x.dim() != 2 or topk_ids.dim() != 2 or topk_ids.shape[0] != x.shape[0]:
        raise ValueError(f"{what}: x [M, K] and topk_ids [M, top_k] expected, got {tuple(x.shape)} and "
                         f"{tuple(topk_ids.shape)}")
    M, K = x.shape
    top_k = topk_ids.shape[1]
    cols = K // GROUP
    if K % GROUP:
        raise ValueError(f"{what}: K={K} must be a multiple of {GROUP}")
    if tuple(x_perm.shape) != (M_sum, K) or tuple(scale_perm.shape) != (M_sum, cols):
        raise ValueError(f"{what}: outputs must be {(M_sum, K)} and {(M_sum, cols)}")
    if tuple(expert_ids.shape) != (M_sum,) or tuple(inv_perm.shape) != (M, top_k):
        raise ValueError(f"{what}: expert_ids must be {(M_sum,)} and inv_perm {(M, top_k)}")
    for t, name in ((topk_ids, "topk_ids"), (x_perm, "x_perm"), (expert_ids, "expert_ids"), (inv_perm, "inv_perm")):
        if not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be contiguous")
    if x.stride(1) != 1 and M > 1:
        raise ValueError(f"{what}: rows of x must be contiguous")
    L = lib()
    ws_bytes = int(L.kbn_moe_permute_workspace_bytes(M * top_k, num_experts))
    if ws_bytes < 0:
        raise ValueError(f"{what}: num_experts={num_experts} outside [1, 1024] or too many pairs")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    check(L.kbn_moe_permute_quant_contiguous(
        topk_ids.data_ptr(), topk_ids.element_size(), M, top_k, num_experts, alignment,
        x.data_ptr() if M else None, x.stride(0) if M else K, K, float(eps), int(bool(use_ue8m0)), M_sum,
        x_perm.data_ptr(), scale_perm.data_ptr(), scale_perm.stride(0), scale_perm.stride(1), expert_ids.data_ptr(),
        inv_perm.data_ptr(), int(zero_padding), ws.data_ptr(), ws_bytes, _stream(x_perm)), what)


def moe_unpermute_reduce(y: torch.Tensor, inv_perm: torch.Tensor, topk_weights: torch.Tensor,
                         out: torch.Tensor) -> None:
    """``out[m] = sum_j topk_weights[m, j] * y[inv_perm[m, j]]`` (bf16 rows,
    fp32 sum in slot order)."""
    what = "moe_unpermute_reduce"
    _dev_check(what, y, inv_perm, topk_weights, out)
    _dtype_check(what, y, torch.bfloat16, "mm2_out")
    _dtype_check(what, out, torch.bfloat16, "output")
    _dtype_check(what, inv_perm, torch.int32, "inv_perm")
    if topk_weights.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"{what}: topk_weights must be float32 or bfloat16, got {topk_weights.dtype}")
    M, H = out.shape
    if tuple(inv_perm.shape) != tuple(topk_weights.shape) or inv_perm.dim() != 2 or inv_perm.shape[0] != M:
        raise ValueError(f"{what}: inv_perm and topk_weights must both be [{M}, top_k], got "
                         f"{tuple(inv_perm.shape)} and {tuple(topk_weights.shape)}")
    if y.dim() != 2 or y.shape[1] != H:
        raise ValueError(f"{what}: mm2_out must be [M_sum, {H}], got {tuple(y.shape)}")
    if not (inv_perm.is_contiguous() and topk_weights.is_contiguous()):
        raise ValueError(f"{what}: inv_perm and topk_weights must be contiguous")
    if (y.stride(1) != 1 and y.shape[0] > 1) or (out.stride(1) != 1 and M > 1):
        raise ValueError(f"{what}: rows of mm2_out and output must be contiguous")
    check(lib().kbn_moe_unpermute_reduce(
        y.data_ptr(), y.shape[0], H, y.stride(0), inv_perm.data_ptr(), M, inv_perm.shape[1],
        topk_weights.data_ptr(), int(topk_weights.dtype == torch.bfloat16), out.data_ptr(), out.stride(0),
        _stream(out)), what)


def rmsnorm_fp8_quant(output_fp8: torch.Tensor, output_scales: torch.Tensor, input: torch.Tensor,
                      weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None) -> None:
    """RMSNorm of ``input [..., H]`` (of ``residual + input`` when ``residual``
    is given, updating both in place as the reference does) quantized 1x128
    into ``output_fp8 [T, H]`` and ``output_scales [T, ceil(H/128)]`` (any
    strides; the reference allocates them column-major).  ``input``,
    ``weight`` and ``residual`` share one dtype: bfloat16, float16 or
    float32, as the reference's kernel dispatches (rmsnorm_quant.cu:111)."""
    idx = input.get_device()
    add = residual is not None
    if (idx not in _GFX950_DEVICES or idx != _cur_device() or output_fp8.get_device() != idx
            or output_scales.get_device() != idx or weight.get_device() != idx
            or (add and residual.get_device() != idx)):
        _dev_check("fused_add_rmsnorm_fp8_quant" if add else "rmsnorm_fp8_quant",
                   *((output_fp8, output_scales, input, weight) + ((residual,) if add else ())))
    if (output_fp8.dtype is not FP8 or output_scales.dtype is not _F32 or input.dtype is not _BF16
            or weight.dtype is not _BF16 or (add and residual.dtype is not _BF16)):
        what = "fused_add_rmsnorm_fp8_quant" if add else "rmsnorm_fp8_quant"
        _dtype_check(what, output_fp8, FP8, "output_fp8")
        _dtype_check(what, output_scales, torch.float32, "output_scales")
        if input.dtype not in _QUANT_IN:
            raise TypeError(f"{what}: input must be bfloat16, float16 or float32, got {input.dtype}")
        for t, name in ((weight, "weight"),) + (((residual, "residual"),) if add else ()):
            if t.dtype != input.dtype:
                raise TypeError(f"{what}: {name} must have the input's dtype {input.dtype}, got {t.dtype}")
    shape = input.shape
    H = shape[-1] if len(shape) else 1
    T = input.numel() // H if H else 0
    G = -(-H // GROUP)
    qs, ss = output_fp8.stride(), output_scales.stride()
    if (not input.is_contiguous() or (add and (not residual.is_contiguous() or residual.shape != shape))
            or weight.shape != (H,) or not weight.is_contiguous() or output_fp8.shape != (T, H) or qs[1] != 1
            or output_scales.shape != (T, G)):
        what = "fused_add_rmsnorm_fp8_quant" if add else "rmsnorm_fp8_quant"
        if not input.is_contiguous() or (add and not residual.is_contiguous()):
            raise ValueError(f"{what}: input and residual must be contiguous")
        if add and residual.shape != shape:
            raise ValueError(f"{what}: residual must match input {tuple(shape)}, got {tuple(residual.shape)}")
        if weight.shape != (H,) or not weight.is_contiguous():
            raise ValueError(f"{what}: weight must be a contiguous [{H}] vector, got {tuple(weight.shape)}")
        if output_fp8.shape != (T, H) or qs[1] != 1:
            raise ValueError(f"{what}: output_fp8 must be [{T}, {H}] with contiguous rows")
        raise ValueError(f"{what}: output_scales must be [{T}, {G}], got {tuple(output_scales.shape)}")
    if input.dtype is _BF16:
        rc = lib().kbn_rmsnorm_fp8_quant(
            input.data_ptr(), T, H, H, weight.data_ptr(), residual.data_ptr() if add else None, H,
            output_fp8.data_ptr(), qs[0], output_scales.data_ptr(), ss[0], ss[1], float(eps), _raw_stream(idx))
    else:
        rc = lib().kbn_rmsnorm_fp8_quant_typed(
            input.data_ptr(), _QUANT_IN[input.dtype], T, H, H, weight.data_ptr(),
            residual.data_ptr() if add else None, H, output_fp8.data_ptr(), qs[0], output_scales.data_ptr(), ss[0],
            ss[1], float(eps), _raw_stream(idx))
    if rc:
        check(rc, "fused_add_rmsnorm_fp8_quant" if add else "rmsnorm_fp8_quant")


def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int, sorted_token_ids: torch.Tensor,
                         expert_ids: torch.Tensor, num_tokens_post_pad: torch.Tensor,
                         cumsum: torch.Tensor | None = None) -> None:
    """Sorted-token layout of ``topk_ids`` (any shape, int32/int64): slots of
    each expert padded to ``block_size``, sentinel ``numel`` elsewhere, one
    expert id per block, the padded total in ``num_tokens_post_pad[0]``."""
    what = "moe_align_block_size"
    _dev_check(what, topk_ids, sorted_token_ids, expert_ids, num_tokens_post_pad,
               *([cumsum] if cumsum is not None else []))
    for t, name in ((sorted_token_ids, "sorted_token_ids"), (expert_ids, "expert_ids"),
                    (num_tokens_post_pad, "num_tokens_post_pad")) + (((cumsum, "cumsum"),) if cumsum is not None else ()):
        _dtype_check(what, t, torch.int32, name)
        if not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be contiguous")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{what}: topk_ids must be int32 or int64, got {topk_ids.dtype}")
    if not topk_ids.is_contiguous():
        raise ValueError(f"{what}: topk_ids must be contiguous")
    if cumsum is not None and cumsum.numel() < num_experts + 1:
        raise ValueError(f"{what}: cumsum needs {num_experts + 1} entries")
    numel = topk_ids.numel()
    L = lib()
    ws_bytes = int(L.kbn_moe_permute_workspace_bytes(numel, num_experts))
    if ws_bytes < 0:
        raise ValueError(f"{what}: num_experts={num_experts} outside [1, 1024] or too many pairs")
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=topk_ids.device)
    check(L.kbn_moe_align_block_size(
        topk_ids.data_ptr() if numel else None, topk_ids.element_size(), numel, num_experts, block_size,
        sorted_token_ids.data_ptr(), sorted_token_ids.numel(), expert_ids.data_ptr(), expert_ids.numel(),
        num_tokens_post_pad.data_ptr(), cumsum.data_ptr() if cumsum is not None else None,
        ws.data_ptr(), ws.numel(), _stream(sorted_token_ids)), what)


def fused_moe_gemm(a: torch.Tensor, a_scale: torch.Tensor, b: torch.Tensor, b_scale: torch.Tensor, c: torch.Tensor,
                   sorted_token_ids: torch.Tensor | None, expert_ids: torch.Tensor,
                   num_tokens_post_padded: torch.Tensor, EM: int, block_m: int, top_k: int,
                   topk_weights: torch.Tensor | None = None) -> None:
    """Sorted-token FP8 GEMM: ``c[t] = (a[t // top_k] . b[e]^T)`` with 1x128
    activation and 128x128 weight block scales, for every routed pair t
    (``c`` is [num_valid, N], num_valid = c rows), times ``topk_weights[t]``
    when given."""
    what = "fused_moe_gemm"
    tensors = [a, a_scale, b, b_scale, c, expert_ids, num_tokens_post_padded]
    if sorted_token_ids is not None:
        tensors.append(sorted_token_ids)
    if topk_weights is not None:
        tensors.append(topk_weights)
    _dev_check(what, *tensors)
    _dtype_check(what, a, FP8, "A")
    _dtype_check(what, b, FP8, "B")
    _dtype_check(what, a_scale, torch.float32, "a_scale")
    _dtype_check(what, b_scale, torch.float32, "b_scale")
    _dtype_check(what, c, torch.bfloat16, "C")
    for t, name in ((expert_ids, "expert_ids"), (num_tokens_post_padded, "num_tokens_post_padded")) + \
            (((sorted_token_ids, "sorted_token_ids"),) if sorted_token_ids is not None else ()):
        _dtype_check(what, t, torch.int32, name)
        if not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be contiguous")
    if a.dim() != 2 or b.dim() != 3 or c.dim() != 2:
        raise ValueError(f"{what}: A [rows, K], B [E, N, K] and C [pairs, N] expected")
    E, N, K = b.shape
    rows_A = a.shape[0]
    if a.shape[1] != K or c.shape[1] != N:
        raise ValueError(f"{what}: K or N mismatch: A {tuple(a.shape)}, B {tuple(b.shape)}, C {tuple(c.shape)}")
    KB, NB = -(-K // GROUP), -(-N // GROUP)
    if tuple(a_scale.shape) != (rows_A, KB):
        raise ValueError(f"{what}: a_scale must be {(rows_A, KB)}, got {tuple(a_scale.shape)}")
    if tuple(b_scale.shape) != (E, NB, KB) or not b_scale.is_contiguous() or not b.is_contiguous():
        raise ValueError(f"{what}: B and b_scale must be contiguous [E, N, K] and [E, {NB}, {KB}]")
    if a.stride(1) != 1 or c.stride(1) != 1:
        raise ValueError(f"{what}: rows of A and C must be contiguous")
    num_valid = c.shape[0]
    if topk_weights is not None:
        _dtype_check(what, topk_weights, torch.float32, "topk_weights")
        if topk_weights.numel() != num_valid or not topk_weights.is_contiguous():
            raise ValueError(f"{what}: topk_weights must hold one contiguous fp32 weight per pair ({num_valid})")
    if sorted_token_ids is not None and sorted_token_ids.numel() < EM:
        raise ValueError(f"{what}: sorted_token_ids holds {sorted_token_ids.numel()} rows, EM = {EM}")
    if expert_ids.numel() * block_m < EM:
        raise ValueError(f"{what}: expert_ids holds {expert_ids.numel()} blocks of {block_m}, EM = {EM}")
    L = lib()
    # the scales are gathered into sorted-row order in a workspace from the
    # caching allocator (stream-ordered on the launch stream)
    ws_bytes = int(L.kbn_fp8_fused_moe_gemm_workspace_bytes(EM, K))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=c.device) if ws_bytes > 0 else None
    check(L.kbn_fp8_fused_moe_gemm(
        a.data_ptr(), a.stride(0), rows_A, a_scale.data_ptr(), a_scale.stride(0), a_scale.stride(1),
        b.data_ptr(), b_scale.data_ptr(), c.data_ptr(), c.stride(0),
        sorted_token_ids.data_ptr() if sorted_token_ids is not None else None, expert_ids.data_ptr(),
        num_tokens_post_padded.data_ptr(), EM, block_m, num_valid, top_k,
        topk_weights.data_ptr() if topk_weights is not None else None, N, K, E,
        ws.data_ptr() if ws is not None else None, ws_bytes if ws is not None else 0, _stream(c)), what)


def moe_sum(x: torch.Tensor, out: torch.Tensor) -> None:
    """``out[m] = sum_j x[m, j]`` over the top-k rows of each token: ``x``
    bf16 [M, top_k, H] (or [M * top_k, H] viewed so), ``out`` bf16 [M, H]."""
    what = "moe_sum"
    _dev_check(what, x, out)
    _dtype_check(what, x, torch.bfloat16, "input")
    _dtype_check(what, out, torch.bfloat16, "output")
    if x.dim() != 3 or out.dim() != 2 or x.shape[0] != out.shape[0] or x.shape[2] != out.shape[1]:
        raise ValueError(f"{what}: input [M, top_k, H] and output [M, H] expected, got {tuple(x.shape)} and "
                         f"{tuple(out.shape)}")
    M, top_k, H = x.shape
    if x.stride(2) != 1 or out.stride(1) != 1 or (M > 1 and x.stride(0) != top_k * x.stride(1)):
        raise ValueError(f"{what}: rows of input and output must be contiguous, slots of a token adjacent")
    check(lib().kbn_moe_sum(x.data_ptr(), M, top_k, H, x.stride(1), out.data_ptr(), out.stride(0), _stream(out)),
          what)


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether the storage byte ranges spanned by two tensors intersect."""
    def span(t):
        lo = t.data_ptr()
        return lo, lo + (sum((n - 1) * st for n, st in zip(t.shape, t.stride())) + 1) * t.element_size()
    (a0, a1), (b0, b1) = span(a), span(b)
    return a.numel() > 0 and b.numel() > 0 and a0 < b1 and b0 < a1


def fp8_block_requant(w_in: torch.Tensor, s_in: torch.Tensor | None, w_out: torch.Tensor, s_out: torch.Tensor,
                      use_ue8m0: bool, eps: float) -> None:
    """128x128 block quantization of ``w_in`` ([N, K] or [E, N, K]; fp8 codes
    dequantized with the block scales ``s_in``, or fp32) into ``w_out`` (fp8,
    same shape) and ``s_out`` ([(E,) ceil(N/128), >= ceil(K/128)]).  fp8 codes
    may be requantized in place (``w_out`` is ``w_in``, ``s_out`` is ``s_in``);
    any other overlap, and every overlap of fp32 input, is rejected."""
    what = "fp8_block_requant"
    _dev_check(what, *[t for t in (w_in, s_in, w_out, s_out) if t is not None])
    in_f32 = w_in.dtype == torch.float32
    if not in_f32:
        _dtype_check(what, w_in, FP8, "w_in")
        if s_in is None:
            raise ValueError(f"{what}: fp8 input needs its block scales")
        _dtype_check(what, s_in, torch.float32, "s_in")
    _dtype_check(what, w_out, FP8, "w_out")
    _dtype_check(what, s_out, torch.float32, "s_out")
    if w_in.shape != w_out.shape or w_in.dim() not in (2, 3):
        raise ValueError(f"{what}: w_in and w_out must both be [N, K] or [E, N, K]")
    if not (w_in.is_contiguous() and w_out.is_contiguous()):
        raise ValueError(f"{what}: weights must be contiguous")
    E = w_in.shape[0] if w_in.dim() == 3 else 1
    N, K = w_in.shape[-2:]
    NB, KB = -(-N // GROUP), -(-K // GROUP)

    def strides(s, name):
        if s.dim() != w_in.dim() or s.shape[-2] < NB or s.shape[-1] < KB or s.stride(-1) != 1:
            raise ValueError(f"{what}: {name} must be [..., >= {NB}, >= {KB}] with unit column stride")
        return (s.stride(0) if s.dim() == 3 else NB * s.stride(-2)), s.stride(-2)

    so_e, so_ld = strides(s_out, "s_out")
    si_e, si_ld = strides(s_in, "s_in") if not in_f32 else (0, 0)
    if _overlaps(w_in, w_out) and (in_f32 or w_in.data_ptr() != w_out.data_ptr()):
        raise ValueError(f"{what}: w_out overlaps w_in (only fp8 codes requantized exactly in place are allowed)")
    if not in_f32 and _overlaps(s_in, s_out) and (s_in.data_ptr() != s_out.data_ptr() or (si_e, si_ld) != (so_e, so_ld)):
        raise ValueError(f"{what}: s_out overlaps s_in with a different layout")
    check(lib().kbn_fp8_block_requant(
        w_in.data_ptr(), int(in_f32), s_in.data_ptr() if not in_f32 else None, si_e, si_ld, E, N, K,
        w_out.data_ptr(), s_out.data_ptr(), so_e, so_ld, int(bool(use_ue8m0)), float(eps), _stream(w_out)), what)
    # written through raw pointers: tell torch (and scales_are_pow2's cache)
    # that both tensors changed
    torch.autograd.graph.increment_version(w_out)
    torch.autograd.graph.increment_version(s_out)
    _SCALE_WRITES[0] += 1


def debug_silu_bf16(g_bits: torch.Tensor, out_bits: torch.Tensor, path: int = 0) -> None:
    """Test hook: the kernels' silu (bf16 in, bf16 out) on int16 bit patterns;
    path 0 reads the table as the SiLU kernels do, path 1 at the symbol
    address the grouped GEMM's SiLU*Mul epilogue is given."""
    _dev_check("debug_silu_bf16", g_bits, out_bits)
    if g_bits.dtype != torch.int16 or out_bits.dtype != torch.int16 or not g_bits.is_contiguous():
        raise TypeError("debug_silu_bf16: contiguous int16 bit patterns expected")
    check(lib().kbn_debug_silu_bf16(g_bits.data_ptr(), out_bits.data_ptr(), g_bits.numel(), int(path),
                                   _stream(g_bits)),
          "debug_silu_bf16")


# ---------------------------------------------------------------------------
# torch.library registration (opaque custom ops with Meta impls)
# ---------------------------------------------------------------------------

_fp8_lib = torch.library.Library("kb_nano_fp8", "FRAGMENT")
_moe_lib = torch.library.Library("kb_nano_fp8_moe", "FRAGMENT")
_norm_lib = torch.library.Library("kb_nano_norm", "FRAGMENT")


def _has_op(ns: str, name: str) -> bool:
    try:
        getattr(getattr(torch.ops, ns), name)
        return True
    except (AttributeError, RuntimeError):
        return False


def _meta_noop(*args, **kwargs):
    return None


def _register():
    if not _has_op("kb_nano_fp8", "fp8_gemm_nt"):
        _fp8_lib.define("fp8_gemm_nt(Tensor q_input, Tensor input_scale, "
                        "Tensor weight, Tensor weight_scale, Tensor! output) -> ()")
        _fp8_lib.impl("fp8_gemm_nt", lambda q, s, w, ws, o: fp8_gemm_nt(q, s, w, ws, o), "CUDA")
        _fp8_lib.impl("fp8_gemm_nt", _meta_noop, "Meta")
    if not _has_op("kb_nano_fp8", "flashinfer_blockscale_gemm"):
        # the reference's bf16-input GEMM op (fp8_linear.py:126-153): the
        # gfx950 kernel that quantizes its activations itself where the scale
        # contract and M allow, else quant + fp8_gemm_nt
        _fp8_lib.define("flashinfer_blockscale_gemm(Tensor input_bf16, Tensor weight_fp8, "
                        "Tensor weight_scale, Tensor! output) -> ()")
        _fp8_lib.impl("flashinfer_blockscale_gemm", lambda x, w, ws, o: flashinfer_blockscale_gemm(x, w, ws, o),
                      "CUDA")
        _fp8_lib.impl("flashinfer_blockscale_gemm", _meta_noop, "Meta")
    if not _has_op("kb_nano_fp8", "per_token_group_quant_fp8"):
        _fp8_lib.define("per_token_group_quant_fp8(Tensor input, Tensor! output_fp8, "
                        "Tensor! output_scale, bool column_major_scales=False) -> ()")
        # the scale layout is read from the output's strides, so the
        # column-major flag needs no separate code path
        _fp8_lib.impl("per_token_group_quant_fp8",
                      lambda x, q, s, column_major_scales=False: per_token_group_quant_fp8(x, q, s), "CUDA")
        _fp8_lib.impl("per_token_group_quant_fp8", _meta_noop, "Meta")
    if not _has_op("kb_nano_fp8", "silu_mul_quant_fp8"):
        _fp8_lib.define("silu_mul_quant_fp8(Tensor input, Tensor! output, Tensor! output_scales, "
                        "bool use_ue8m0=True, float eps=1e-10) -> ()")
        _fp8_lib.impl("silu_mul_quant_fp8",
                      lambda x, q, s, use_ue8m0=True, eps=QUANT_EPS: silu_mul_quant_fp8(x, q, s, use_ue8m0, eps),
                      "CUDA")
        _fp8_lib.impl("silu_mul_quant_fp8", _meta_noop, "Meta")
    if not _has_op("kb_nano_fp8_moe", "m_grouped_gemm_nt_contiguous"):
        _moe_lib.define("m_grouped_gemm_nt_contiguous(Tensor a_fp8, Tensor a_scale, "
                        "Tensor b_fp8, Tensor b_scale, Tensor! c_bf16, Tensor expert_ids, "
                        "bool disable_ue8m0_cast) -> ()")
        _moe_lib.impl("m_grouped_gemm_nt_contiguous", m_grouped_gemm_nt_contiguous, "CUDA")
        _moe_lib.impl("m_grouped_gemm_nt_contiguous", _meta_noop, "Meta")
    # schemas of tasks/baseline/L1/rmsnorm_quant.py:27-55
    if not _has_op("kb_nano_norm", "rmsnorm_fp8_quant"):
        _norm_lib.define("rmsnorm_fp8_quant(Tensor! output_fp8, Tensor! output_scales, "
                         "Tensor input, Tensor weight, float eps) -> ()")
        _norm_lib.impl("rmsnorm_fp8_quant", lambda q, s, x, w, eps: rmsnorm_fp8_quant(q, s, x, w, eps), "CUDA")
        _norm_lib.impl("rmsnorm_fp8_quant", _meta_noop, "Meta")
    if not _has_op("kb_nano_norm", "fused_add_rmsnorm_fp8_quant"):
        _norm_lib.define("fused_add_rmsnorm_fp8_quant(Tensor! output_fp8, Tensor! output_scales, "
                         "Tensor(a!) input, Tensor(b!) residual, Tensor weight, float eps) -> ()")
        _norm_lib.impl("fused_add_rmsnorm_fp8_quant",
                       lambda q, s, x, r, w, eps: rmsnorm_fp8_quant(q, s, x, w, eps, residual=r), "CUDA")
        _norm_lib.impl("fused_add_rmsnorm_fp8_quant", _meta_noop, "Meta")


_register()
