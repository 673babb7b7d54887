"""ctypes binding of ``libkbn_fp8.so`` (the C-ABI declared in include/kbn_fp8.h).

The library is loaded once per process.  There is no fallback: if the built
library is missing, or the visible GPU is not gfx950, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB_PATH

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int

# name -> argtypes, in the order of include/kbn_fp8.h
SIGNATURES = {
    "kbn_last_error": ([], ctypes.c_char_p),
    "kbn_abi_version": ([], _I),
    "kbn_device_arch": ([_I, ctypes.c_char_p, _I], _I),
    "kbn_per_token_group_quant_fp8": ([_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _F, _I, _P], _I),
    "kbn_per_token_group_quant_fp8_typed": ([_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _F, _I, _P], _I),
    "kbn_silu_mul_quant_fp8": ([_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _F, _I, _P], _I),
    "kbn_silu_mul_quant_fp8_rows": ([_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _F, _I, _P, _P], _I),
    "kbn_fp8_gemm_nt": ([_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P], _I),
    "kbn_fp8_gemm_nt_workspace_bytes": ([_I64, _I64, _I64, _I], _I64),
    "kbn_fp8_gemm_nt_ws": (
        [_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P], _I),
    "kbn_fp8_gemm_nt_packed_ws": (
        [_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "kbn_fp8_linear_forward": ([_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _F, _I, _P, _I64, _P, _I64, _P,
                                _I64, _I64, _I, _P, _I64, _P], _I),
    "kbn_fp8_gemm_bf16a_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "kbn_fp8_gemm_bf16a_preferred": ([_I64, _I64, _I64], _I),
    "kbn_fp8_gemm_bf16a": ([_P, _I64, _F, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "kbn_fp8_gemm_nt_noalloc_scratch_bytes": ([], _I64),
    "kbn_fp8_gemm_nt_noalloc": ([_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P], _I),
    "kbn_fp8_grouped_gemm_nt_contiguous": (
        [_P, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P], _I),
    "kbn_fp8_grouped_gemm_silu_quant": (
        [_P, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _I64, _F, _I, _P],
        _I),
    "kbn_moe_permute_workspace_bytes": ([_I64, _I64], _I64),
    "kbn_moe_permute_contiguous": (
        [_P, _I, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P, _I,
         _P, _I64, _P], _I),
    "kbn_moe_permute_quant_contiguous": (
        [_P, _I, _I64, _I64, _I64, _I64, _P, _I64, _I64, _F, _I, _I64, _P, _P, _I64, _I64, _P, _P, _I, _P, _I64, _P], _I),
    "kbn_moe_unpermute_reduce": ([_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I, _P, _I64, _P], _I),
    "kbn_rmsnorm_fp8_quant": ([_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _F, _P], _I),
    "kbn_rmsnorm_fp8_quant_typed": ([_P, _I, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _F, _P], _I),
    "kbn_moe_align_block_size": ([_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P], _I),
    "kbn_fp8_fused_moe_gemm": ([_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64,
                                _P, _I64, _I64, _I64, _P, _I64, _P], _I),
    "kbn_fp8_fused_moe_gemm_workspace_bytes": ([_I64, _I64], _I64),
    "kbn_moe_sum": ([_P, _I64, _I64, _I64, _I64, _P, _I64, _P], _I),
    "kbn_fp8_block_requant": ([_P, _I, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I, _F, _P], _I),
    "kbn_splitk_counter_stats": ([_P, _P, _P], _I),
    "kbn_debug_splitk_regions": ([_I64, _P, _P], _I),
    "kbn_debug_gemm_plan": ([_I64, _I64, _I64, _I, _I, _P], _I),
    "kbn_debug_silu_bf16": ([_P, _P, _I64, _I, _P], _I),
}

ABI_VERSION = 1

_LOCK = threading.Lock()
_LIB = None


class KbnError(RuntimeError):
    pass


def lib():
    """Load the HIP library (raises if it was never built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise KbnError(
                    f"{LIB_PATH} is missing: build it with `python -m kb_nano_amd._build` "
                    "(or __graft_entry__.build()); kb_nano_amd has no CPU fallback")
            L = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
            if L.kbn_abi_version() != ABI_VERSION:
                raise KbnError(f"{LIB_PATH} has ABI {L.kbn_abi_version()}, expected {ABI_VERSION}; rebuild it")
            _LIB = L
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().kbn_last_error().decode(errors="replace")
        raise KbnError(f"{what}: {msg} (code {rc})")


_ARCH_OK: dict[int, str] = {}


def require_gfx950(device_index: int) -> None:
    """Raise unless device `device_index` is a gfx950 (MI355X-class) GPU."""
    if device_index in _ARCH_OK:
        return
    buf = ctypes.create_string_buffer(128)
    check(lib().kbn_device_arch(device_index, buf, 128), "device_arch")
    arch = buf.value.decode()
    if not arch.startswith("gfx950"):
        raise KbnError(f"kb_nano_amd kernels are built for gfx950; device {device_index} is {arch}")
    _ARCH_OK[device_index] = arch
