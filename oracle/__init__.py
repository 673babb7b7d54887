"""CPU oracle for the block-scaled FP8 linear path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker or the timed CPU baseline.
The product package ``kb_nano_amd`` never imports it.

The arithmetic lives in ``kbn_oracle.c`` (plain C, built by ``oracle/Makefile``
into ``libkbn_oracle.so``); this module wraps it with numpy and restates the
contiguous MoE layout of ``tasks/baseline/L2/fused_experts.py:32-136`` in numpy.
Every function cites the reference lines it follows.

Parity pins (see ``tests/test_oracle.py``):
  * e4m3 encode: exhaustive over all 65,536 bf16 bit patterns against torch's
    ``.to(torch.float8_e4m3fn)`` (an independent library routine).
  * UE8M0 scale: exhaustive over every finite non-negative bf16 absmax against
    torch's ``pow(2, ceil(log2(x/448)))`` form used by the reference.
  * silu: all 65,536 bf16 gate values against a 40-digit ``decimal`` evaluation.
  * quant / silu-quant: the reference's own torch formula
    (``tasks/reference/L1/fp8_linear.py:41-64``) on seeded tensors, plus the
    committed golden fixtures.
  * GEMM: float64 brute force on tiny shapes, torch fp32 dequant-matmul on
    small shapes, and closed-form special cases (single non-zero K block,
    identity-like weights, all-equal scales).
  * weight block requant: the reference's torch formula (DeepGEMM's
    ``per_block_cast_to_fp8`` on the dequantized weight) executed by torch on
    the CPU, ``quant_block128``'s division form under UE8M0 (equal there,
    since 1/sf is exact), and the identity on power-of-two-scaled blocks
    whose largest code is 448.
  * moe_align_block_size: each expert's slots hold exactly its pairs in
    (token, slot) order (checked against a stable argsort), the reference's
    buffer-size bound, sentinel and searchsorted block owners; moe_sum:
    inputs whose fp32 sums are exact, where per-add bf16 rounding, a single
    final rounding and the accumulator order give different answers, and on
    the GPU torch.sum itself (the reference's at::sum_out).
  * MoE layout: brute-force placement on small routings (each expert's rows
    counted by a direct loop), the structural invariants of the layout
    (segments start on alignment boundaries, (token, slot) order inside a
    segment, injective destinations), and the reference's torch formula for
    the unpermute-and-reduce (fp32 and bf16 weights) within one bf16 ulp.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkbn_oracle.so")
_SRC_PATH = os.path.join(_HERE, "kbn_oracle.c")
_LOCK = threading.Lock()
_LIB = None

GROUP = 128
FP8_MAX = 448.0
EPS = 1e-10

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (via its Makefile) if missing or stale."""
    stale = (not os.path.exists(_LIB_PATH)
             or os.path.getmtime(_LIB_PATH) < os.path.getmtime(_SRC_PATH))
    if force or stale:
        cmd = ["make", "-s", "-C", _HERE]
        if force:
            cmd.append("-B")
        subprocess.run(cmd, check=True)
    return _LIB_PATH


def lib():
    global _LIB
    with _LOCK:
        if _LIB is None:
            build()
            L = ctypes.CDLL(_LIB_PATH)
            L.orc_e4m3_encode.restype = ctypes.c_uint8
            L.orc_e4m3_encode.argtypes = [ctypes.c_float]
            L.orc_e4m3_decode.restype = ctypes.c_float
            L.orc_e4m3_decode.argtypes = [ctypes.c_uint8]
            L.orc_ue8m0_from_ratio.restype = ctypes.c_float
            L.orc_ue8m0_from_ratio.argtypes = [ctypes.c_float]
            L.orc_silu_bf16.restype = ctypes.c_uint16
            L.orc_silu_bf16.argtypes = [ctypes.c_uint16]
            L.orc_double_to_bf16.restype = ctypes.c_uint16
            L.orc_double_to_bf16.argtypes = [ctypes.c_double]
            L.orc_float_to_bf16.restype = ctypes.c_uint16
            L.orc_float_to_bf16.argtypes = [ctypes.c_float]
            qargs = [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, ctypes.c_float, ctypes.c_int]
            L.orc_quant_group128.restype = ctypes.c_int
            L.orc_quant_group128.argtypes = qargs
            L.orc_quant_group128_f32.restype = ctypes.c_int
            L.orc_quant_group128_f32.argtypes = qargs
            L.orc_silu_mul_quant.restype = ctypes.c_int
            L.orc_silu_mul_quant.argtypes = qargs
            L.orc_gemm_nt_sample.restype = ctypes.c_int
            L.orc_gemm_nt_sample.argtypes = [_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64,
                                             _I64, _I64, _I64, _P, _I64, _P, _I64, _P, ctypes.c_int]
            L.orc_grouped_gemm_nt_sample.restype = ctypes.c_int
            L.orc_grouped_gemm_nt_sample.argtypes = [_P, _P, _I64, _I64, _P, _P, _P,
                                                     _I64, _I64, _I64, _I64,
                                                     _P, _I64, _P, _I64, _P, ctypes.c_int]
            L.orc_rmsnorm_quant_f32.restype = ctypes.c_int
            L.orc_rmsnorm_quant_f32.argtypes = [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64,
                                                ctypes.c_float, ctypes.c_int]
            L.orc_float_to_f16.restype = ctypes.c_uint16
            L.orc_float_to_f16.argtypes = [ctypes.c_float]
            L.orc_f16_to_float.restype = ctypes.c_float
            L.orc_f16_to_float.argtypes = [ctypes.c_uint16]
            L.orc_rmsnorm_quant.restype = ctypes.c_int
            L.orc_rmsnorm_quant.argtypes = [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64,
                                            ctypes.c_float]
            _LIB = L
    return _LIB


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------------------
# bf16 helpers (numpy has no bf16: bf16 tensors travel as uint16 bit patterns)
# ---------------------------------------------------------------------------

def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (RNE) and return the bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------------------
# Scalar-table views of the C encoders (vectorised through lookup tables)
# ---------------------------------------------------------------------------

_E4M3_DECODE = None


def e4m3_decode_table() -> np.ndarray:
    global _E4M3_DECODE
    if _E4M3_DECODE is None:
        L = lib()
        _E4M3_DECODE = np.array([L.orc_e4m3_decode(i) for i in range(256)], dtype=np.float32)
    return _E4M3_DECODE


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return e4m3_decode_table()[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([L.orc_e4m3_encode(float(v)) for v in flat], dtype=np.uint8).reshape(np.shape(x))


def ue8m0_from_ratio(r: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.asarray(r, dtype=np.float32).ravel()
    return np.array([L.orc_ue8m0_from_ratio(float(v)) for v in flat], dtype=np.float32).reshape(np.shape(r))


_SILU_TABLE = None


def silu_bf16_table() -> np.ndarray:
    """bf16 silu(g) for every one of the 65,536 bf16 bit patterns g."""
    global _SILU_TABLE
    if _SILU_TABLE is None:
        L = lib()
        _SILU_TABLE = np.array([L.orc_silu_bf16(i) for i in range(65536)], dtype=np.uint16)
    return _SILU_TABLE


# ---------------------------------------------------------------------------
# Quantizers
# ---------------------------------------------------------------------------

def quant_group128(x_bits: np.ndarray, eps: float = EPS, use_ue8m0: bool = True):
    """Per-token-group 1x128 quant (tasks/baseline/L1/fp8_linear.py:181-215).

    ``x_bits``: uint16 bf16 bit patterns [M, K].  Returns (q uint8 [M,K],
    s float32 [M, K/128] row-major)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // GROUP), dtype=np.float32)
    rc = lib().orc_quant_group128(_ptr(x), M, K, K, _ptr(q), K, _ptr(s), K // GROUP, 1,
                                  float(eps), int(use_ue8m0))
    if rc:
        raise ValueError(f"orc_quant_group128 failed ({rc}); K must be a multiple of 128")
    return q, s


def quant_group128_f32(x: np.ndarray, eps: float = EPS, use_ue8m0: bool = True):
    """Per-token-group 1x128 quant of fp16 or fp32 values
    (tasks/baseline/L1/fp8_linear.py:181-215; :197 widens the input to fp32,
    exactly for these types).  ``x``: float16 or float32 [M, K].  Returns
    (q uint8 [M,K], s float32 [M, K/128] row-major)."""
    v = np.ascontiguousarray(np.asarray(x).astype(np.float32))
    M, K = v.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // GROUP), dtype=np.float32)
    rc = lib().orc_quant_group128_f32(_ptr(v), M, K, K, _ptr(q), K, _ptr(s), K // GROUP, 1,
                                      float(eps), int(use_ue8m0))
    if rc:
        raise ValueError(f"orc_quant_group128_f32 failed ({rc}); K must be a multiple of 128")
    return q, s


def silu_mul_quant(in_bits: np.ndarray, eps: float = EPS, use_ue8m0: bool = True):
    """Fused SiLU*Mul + 1x128 quant (tasks/baseline/L1/silu_mul_quant_fp8.py:48-76).

    ``in_bits``: uint16 bf16 [M, 2*Nh].  Returns (q uint8 [M, Nh], s float32
    [M, Nh/128] row-major values; the device op stores them column-major)."""
    x = np.ascontiguousarray(in_bits, dtype=np.uint16)
    M, N2 = x.shape
    Nh = N2 // 2
    q = np.empty((M, Nh), dtype=np.uint8)
    s = np.empty((M, Nh // GROUP), dtype=np.float32)
    rc = lib().orc_silu_mul_quant(_ptr(x), M, Nh, N2, _ptr(q), Nh, _ptr(s), Nh // GROUP, 1,
                                  float(eps), int(use_ue8m0))
    if rc:
        raise ValueError(f"orc_silu_mul_quant failed ({rc}); N/2 must be a multiple of 128")
    return q, s


def quant_block128(w_f32: np.ndarray, eps: float = EPS, use_ue8m0: bool = True):
    """128x128 block quant of a float32 [R, C] matrix
    (bench/kernels/scenario_registry.py:185-221): one scale per block, codes
    via the C encoder.  Returns (q uint8 [R, C], s float32 [ceil(R/128), ceil(C/128)])."""
    w = np.asarray(w_f32, dtype=np.float32)
    R, C = w.shape
    RB, CB = -(-R // GROUP), -(-C // GROUP)
    pad = np.zeros((RB * GROUP, CB * GROUP), dtype=np.float32)
    pad[:R, :C] = w
    amax = np.abs(pad.reshape(RB, GROUP, CB, GROUP)).max(axis=(1, 3))
    ratio = (np.maximum(amax, np.float32(eps)) / np.float32(FP8_MAX)).astype(np.float32)
    s = ue8m0_from_ratio(ratio) if use_ue8m0 else ratio
    sx = np.repeat(np.repeat(s, GROUP, 0), GROUP, 1)[:R, :C]
    v = np.clip(w / sx, -FP8_MAX, FP8_MAX).astype(np.float32)
    q = _encode_fast(v)
    return q, s.astype(np.float32)


def block_requant(w: np.ndarray, s_in=None, use_ue8m0: bool = True, eps: float = 1e-4):
    """Load-time 128x128 block requantization of a weight [N, K] or [E, N, K]
    (tasks/baseline/L1/fp8_linear.py:453-554).

    ``w`` is either uint8 e4m3 codes, dequantized as fp32(code) * s_in[block]
    (:486, :533-535), or float32 values (s_in None).  Each block then goes
    through DeepGEMM v2.1.1.post3's ``per_block_cast_to_fp8`` (called at
    :497-499 and :543-545; DeepGEMM is not vendored in the reference):
    zero-padded to whole blocks, amax = max|x| clamped below at eps (1e-4
    there), sf = amax / 448, rounded up to a power of two under UE8M0, codes =
    e4m3(x * (1 / sf)) with the reciprocal taken in float32.  Every |x * (1/sf)|
    is at most 448 (1 + 2^-23)^2, which the cast rounds to 448, so clipping to
    +-448 before the nearest-code encoder changes nothing.  Returns (uint8
    codes of w's shape, float32 scales [(E,) ceil(N/128), ceil(K/128)])."""
    w = np.asarray(w)
    squeeze = w.ndim == 2
    if squeeze:
        w = w[None]
        if s_in is not None:
            s_in = np.asarray(s_in)[None]
    E, N, K = w.shape
    NB, KB = -(-N // GROUP), -(-K // GROUP)
    if w.dtype == np.uint8:
        s = np.asarray(s_in, dtype=np.float32)[:, :NB, :KB]
        sx = np.repeat(np.repeat(s, GROUP, 1), GROUP, 2)[:, :N, :K]
        x = (e4m3_decode(w) * sx).astype(np.float32)
    else:
        x = np.asarray(w, dtype=np.float32)
    pad = np.zeros((E, NB * GROUP, KB * GROUP), dtype=np.float32)
    pad[:, :N, :K] = x
    amax = np.abs(pad.reshape(E, NB, GROUP, KB, GROUP)).max(axis=(2, 4))
    sf = (np.maximum(amax, np.float32(eps)) / np.float32(FP8_MAX)).astype(np.float32)
    if use_ue8m0:
        sf = ue8m0_from_ratio(sf)
    inv = (np.float32(1.0) / sf).astype(np.float32)
    ix = np.repeat(np.repeat(inv, GROUP, 1), GROUP, 2)[:, :N, :K]
    v = np.clip(x * ix, -FP8_MAX, FP8_MAX).astype(np.float32)
    q = _encode_fast(v)
    return (q[0], sf[0]) if squeeze else (q, sf)


def _encode_fast(v: np.ndarray) -> np.ndarray:
    """Vectorised e4m3 encoding of already-clamped float32 values: nearest
    code by value with ties to the even code, matching ``orc_e4m3_encode``
    (checked against it in tests)."""
    table = e4m3_decode_table()
    pos = np.arange(0, 127, dtype=np.uint8)      # 0x00..0x7E, non-negative finite codes
    vals = table[pos].astype(np.float64)
    a = np.abs(v.astype(np.float64)).ravel()
    idx = np.searchsorted(vals, a, side="left")
    idx = np.clip(idx, 1, len(vals) - 1)
    lo, hi = vals[idx - 1], vals[idx]
    dlo, dhi = a - lo, hi - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((pos[idx] & 1) == 0))
    code = np.where(pick_hi, pos[idx], pos[idx - 1]).astype(np.uint8)
    exact0 = a == 0.0
    code[exact0] = 0
    sign = (np.signbit(v.ravel()) & (code != 0x7F)).astype(np.uint8) << 7
    return (code | sign).reshape(v.shape)


# ---------------------------------------------------------------------------
# GEMM oracles (float64 accumulation at sampled output positions)
# ---------------------------------------------------------------------------

def gemm_nt_sample(A, sA, W, sW, rows=None, cols=None, ue8m0: bool = False) -> np.ndarray:
    """D[rows][:, cols] of the block-scaled NT GEMM in float64.

    A uint8 [M,K]; sA float32 [M,K/128] (any strides: a numpy view is made
    contiguous here); W uint8 [N,K]; sW float32 [ceil(N/128), K/128].
    ``ue8m0`` rounds every scale up to a power of two first (the UE8M0 cast
    contract)."""
    A = np.ascontiguousarray(A, dtype=np.uint8)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    sA = np.ascontiguousarray(sA, dtype=np.float32)
    sW = np.ascontiguousarray(sW, dtype=np.float32)
    M, K = A.shape
    N = W.shape[0]
    rows = np.arange(M, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.arange(N, dtype=np.int64) if cols is None else np.ascontiguousarray(cols, dtype=np.int64)
    out = np.empty((len(rows), len(cols)), dtype=np.float64)
    rc = lib().orc_gemm_nt_sample(_ptr(A), K, _ptr(sA), sA.shape[1], 1, _ptr(W), K, _ptr(sW), sW.shape[1],
                                  M, N, K, _ptr(rows), len(rows), _ptr(cols), len(cols), _ptr(out), int(ue8m0))
    if rc:
        raise ValueError(f"orc_gemm_nt_sample failed ({rc})")
    return out


def grouped_gemm_nt_sample(A, sA, B, sB, expert_ids, rows=None, cols=None, ue8m0: bool = False) -> np.ndarray:
    """Contiguous grouped GEMM at sampled rows/cols (NaN for rows with id -1).

    A uint8 [M_sum,K]; sA float32 [M_sum,K/128]; B uint8 [E,N,K];
    sB float32 [E,ceil(N/128),K/128]; expert_ids int32 [M_sum]."""
    A = np.ascontiguousarray(A, dtype=np.uint8)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    sA = np.ascontiguousarray(sA, dtype=np.float32)
    sB = np.ascontiguousarray(sB, dtype=np.float32)
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    M_sum, K = A.shape
    E, N, _ = B.shape
    rows = np.arange(M_sum, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.arange(N, dtype=np.int64) if cols is None else np.ascontiguousarray(cols, dtype=np.int64)
    out = np.empty((len(rows), len(cols)), dtype=np.float64)
    rc = lib().orc_grouped_gemm_nt_sample(_ptr(A), _ptr(sA), sA.shape[1], 1, _ptr(B), _ptr(sB), _ptr(ids),
                                          M_sum, N, K, E, _ptr(rows), len(rows), _ptr(cols), len(cols),
                                          _ptr(out), int(ue8m0))
    if rc:
        raise ValueError(f"orc_grouped_gemm_nt_sample failed ({rc})")
    return out


# ---------------------------------------------------------------------------
# Contiguous MoE layout (tasks/baseline/L2/fused_experts.py:32-136)
# ---------------------------------------------------------------------------

def compute_aligned_M(M: int, num_topk: int, num_experts: int, alignment: int) -> int:
    """fused_experts.py:32-39: M_sum = roundup(M*k + E*(align-1), align)."""
    m_sum = M * num_topk + num_experts * (alignment - 1)
    rem = m_sum % alignment
    return m_sum + (alignment - rem if rem else 0)


def permute_contiguous(topk_ids: np.ndarray, num_experts: int, alignment: int):
    """fused_experts.py:42-116 restated: returns (expert_ids int32 [M_sum],
    dest int64 [M*k] destination row of each (token, slot), M_sum).

    Expert e owns rows [off[e], off[e] + roundup(count[e], align)); the first
    count[e] of them hold its tokens in (token, slot) order (stable sort) and
    carry id e, the rest are padding with id -1.  A pair whose id lies outside
    [0, num_experts) is dropped (dest -1); the reference's scatter_add fails
    on such ids instead."""
    ids = np.asarray(topk_ids, dtype=np.int64)
    M, k = ids.shape
    flat = ids.reshape(-1)
    M_sum = compute_aligned_M(M, k, num_experts, alignment)
    valid = (flat >= 0) & (flat < num_experts)
    counts = np.bincount(flat[valid], minlength=num_experts).astype(np.int64)
    aligned = (counts + alignment - 1) // alignment * alignment
    off = np.zeros(num_experts + 1, dtype=np.int64)
    off[1:] = np.cumsum(aligned)
    expert_ids = np.full(M_sum, -1, dtype=np.int32)
    for e in range(num_experts):
        expert_ids[off[e]:off[e] + counts[e]] = e
    order = np.argsort(flat, kind="stable")
    within = np.zeros_like(flat)
    seen = np.zeros(num_experts, dtype=np.int64)
    for pos in order:
        e = flat[pos]
        if 0 <= e < num_experts:
            within[pos] = seen[e]
            seen[e] += 1
    dest = np.where(valid, off[np.where(valid, flat, 0)] + within, -1)
    return expert_ids, dest, M_sum


# ---------------------------------------------------------------------------
# Sorted-token MoE (tasks/baseline/L1/csrc/moe_align.cu, moe_sum.cu,
# tasks/baseline/L1/moe_grouped_gemm.py:86-189)
# ---------------------------------------------------------------------------

def moe_align_block_size(topk_ids: np.ndarray, num_experts: int, block_size: int, sorted_len: int | None = None):
    """moe_align.cu:56-205 restated (the counting, padded prefix sum, sentinel
    fill and per-block expert search), with pairs placed in flattened
    (token, slot) order inside each expert.  The reference places them with
    atomics (:28-40), so any order inside an expert is one it can produce.

    Returns (sorted_ids int32 [sorted_len], expert_ids int32 [total /
    block_size], total, cumsum int32 [E + 1]).  ``sorted_len`` defaults to
    the reference's buffer size (vllm_fused_experts.py:74-78).  Pairs with
    ids outside [0, E) are not placed."""
    flat = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    numel = flat.size
    if sorted_len is None:
        sorted_len = numel * block_size if numel < num_experts else numel + num_experts * (block_size - 1)
    valid = (flat >= 0) & (flat < num_experts)
    counts = np.bincount(flat[valid], minlength=num_experts).astype(np.int64)
    padded = (counts + block_size - 1) // block_size * block_size
    cumsum = np.zeros(num_experts + 1, dtype=np.int64)
    cumsum[1:] = np.cumsum(padded)
    total = int(cumsum[-1])
    sorted_ids = np.full(sorted_len, numel, dtype=np.int32)
    fill = cumsum[:-1].copy()
    for i in range(numel):                      # (token, slot) order
        e = flat[i]
        if 0 <= e < num_experts:
            sorted_ids[fill[e]] = i
            fill[e] += 1
    # expert of block b: last e with cumsum[e] <= b * block_size (:185-199)
    starts = np.arange(total // block_size, dtype=np.int64) * block_size
    expert_ids = (np.searchsorted(cumsum, starts, side="right") - 1).astype(np.int32)
    return sorted_ids, expert_ids, total, cumsum.astype(np.int32)


def moe_sum(x_bits: np.ndarray) -> np.ndarray:
    """moe_sum.cu:8-63 on bf16 bit patterns x [M, top_k, H] -> [M, H].

    top_k in 2..4: the kernel's bf16 accumulator, 0 + x_0 + x_1 ..., each sum
    rounded to bf16 (:14-19).  Otherwise at::sum_out (:58-60): fp32 sums in
    four accumulators taking slots j % 4, combined ((a0 + a1) + a2) + a3 and
    rounded once (torch's reduction order for this shape on the MI355X,
    measured against torch.sum)."""
    x = bf16_bits_to_f32(np.asarray(x_bits, dtype=np.uint16))
    M, k, H = x.shape
    if 2 <= k <= 4:
        acc = np.zeros((M, H), dtype=np.float32)
        for j in range(k):
            acc = bf16_bits_to_f32(f32_to_bf16_bits(acc + x[:, j]))
        return f32_to_bf16_bits(acc)
    parts = []
    for q in range(min(4, k)):
        a = x[:, q].copy()
        for j in range(q + 4, k, 4):
            a = (a + x[:, j]).astype(np.float32)
        parts.append(a)
    tot = parts[0]
    for a in parts[1:]:
        tot = (tot + a).astype(np.float32)
    return f32_to_bf16_bits(tot)


def fused_moe_gemm_sample(A, sA, B, sB, sorted_ids, expert_ids, total: int, block_m: int, num_valid: int,
                          top_k: int, topk_weights=None, cols=None, naive: bool = False) -> dict:
    """moe_grouped_gemm.py:86-189 on its FP8 block-scaled path, in float64:
    for every pair t placed in a block below ``total``,
    C[t, n] = w[t] * sum_kb sA[t // top_k, kb] sB[e, n // 128, kb] (A[t // top_k] . B[e, n]) over block kb.
    With ``naive`` (no sorted list) block b holds pair b alone.  Returns
    {pair t: float64 [len(cols)]}."""
    B = np.asarray(B)
    E, N, K = B.shape
    cols = np.arange(N, dtype=np.int64) if cols is None else np.asarray(cols, dtype=np.int64)
    rows_of = {}                                  # expert -> pairs
    nblocks = total // block_m
    for b in range(nblocks):
        e = int(expert_ids[b])
        if naive:
            pairs = [b] if b < num_valid else []
        else:
            pairs = [int(t) for t in sorted_ids[b * block_m:(b + 1) * block_m] if 0 <= t < num_valid]
        rows_of.setdefault(e, []).extend(pairs)
    out = {}
    for e, pairs in rows_of.items():
        if not pairs:
            continue
        arows = np.array([t // top_k for t in pairs], dtype=np.int64)
        vals = gemm_nt_sample(np.asarray(A)[arows], np.asarray(sA)[arows], B[e], np.asarray(sB)[e], cols=cols)
        for r, t in enumerate(pairs):
            w = 1.0 if topk_weights is None else float(np.asarray(topk_weights, dtype=np.float32).reshape(-1)[t])
            out[t] = vals[r] * w
    return out


def unpermute_and_reduce(mm2_out_f32: np.ndarray, inv_perm: np.ndarray, topk_weights: np.ndarray,
                         bf16_products: bool = False) -> np.ndarray:
    """fused_experts.py:119-136: out[m] = sum_j w[m,j] * mm2_out[inv_perm[m,j]]
    (float32 result; the reference then rounds it into the bf16 output).

    The reference multiplies the bf16 rows by the weights in torch, so each
    product is rounded to float32 (float32 weights) or to bf16 (bf16 weights,
    ``bf16_products``), and sums the top_k products in float32.  The sum is
    taken here in slot order j = 0, 1, ..., one rounding per addition,
    starting from +0.  Slots whose inv_perm is outside [0, rows) contribute
    nothing."""
    y = np.asarray(mm2_out_f32, dtype=np.float32)
    inv = np.asarray(inv_perm, dtype=np.int64)
    w = np.asarray(topk_weights, dtype=np.float32)
    M, k = inv.shape
    out = np.zeros((M, y.shape[1]), dtype=np.float32)
    for j in range(k):
        r = inv[:, j]
        ok = (r >= 0) & (r < y.shape[0])
        p = (y[np.where(ok, r, 0)] * w[:, j:j + 1]).astype(np.float32)
        if bf16_products:
            p = bf16_bits_to_f32(f32_to_bf16_bits(p))
        out = np.where(ok[:, None], (out + p).astype(np.float32), out)
    return out


# ---------------------------------------------------------------------------
# Fused RMSNorm + 1x128 quant (tasks/baseline/L1/csrc/rmsnorm_quant.cu:21-201)
# ---------------------------------------------------------------------------

def rmsnorm_quant(x_bits: np.ndarray, w_bits: np.ndarray, eps: float = 1e-6, residual_bits=None):
    """RMSNorm of bf16 ``x [M, H]`` (of ``residual + x`` when ``residual_bits``
    is given) with bf16 weight ``w [H]``, quantized 1x128 to e4m3 with UE8M0
    scales.  Returns ``(codes uint8 [M, H], scales fp32 [M, ceil(H/128)])``,
    plus, for the residual variant, ``(residual_out, x_out)`` bf16 bits: the
    bf16 sum and the bf16 normalized row (the reference overwrites its inputs
    with them).  Sum of squares in the fixed fp32 order of ``orc_rmsnorm_quant``."""
    x = np.array(x_bits, dtype=np.uint16, copy=True, order="C")
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    M, H = x.shape
    if w.shape != (H,):
        raise ValueError("weight must be [H]")
    G = -(-H // 128)
    q = np.empty((M, H), dtype=np.uint8)
    s = np.empty((M, G), dtype=np.float32)
    r = None if residual_bits is None else np.array(residual_bits, dtype=np.uint16, copy=True, order="C")
    rc = lib().orc_rmsnorm_quant(_ptr(x), M, H, H, _ptr(w), None if r is None else _ptr(r), H, _ptr(q), H,
                                 _ptr(s), G, 1, float(eps))
    if rc:
        raise ValueError(f"orc_rmsnorm_quant failed ({rc})")
    return (q, s) if r is None else (q, s, r, x)


_RND = {"bf16": 0, "fp16": 1, "fp32": 2}


def rmsnorm_quant_values(x: np.ndarray, w: np.ndarray, dtype: str, eps: float = 1e-6, residual=None):
    """``rmsnorm_quant`` for bf16, fp16 or fp32 rows (``dtype``): ``x [M, H]``,
    ``w [H]`` and ``residual`` are float arrays holding numbers of that type;
    the residual sum and the normalized row written back are rounded to it
    (tasks/baseline/L1/csrc/rmsnorm_quant.cu:111 dispatches over the float
    types).  Returns ``(codes, scales)``, plus ``(residual_out, x_out)`` as
    float32 values for the residual variant.  Same summation order as
    ``rmsnorm_quant``."""
    v = np.array(x, dtype=np.float32, copy=True, order="C")
    wf = np.ascontiguousarray(w, dtype=np.float32)
    M, H = v.shape
    if wf.shape != (H,):
        raise ValueError("weight must be [H]")
    G = -(-H // 128)
    q = np.empty((M, H), dtype=np.uint8)
    s = np.empty((M, G), dtype=np.float32)
    r = None if residual is None else np.array(residual, dtype=np.float32, copy=True, order="C")
    rc = lib().orc_rmsnorm_quant_f32(_ptr(v), M, H, H, _ptr(wf), None if r is None else _ptr(r), H, _ptr(q), H,
                                     _ptr(s), G, 1, float(eps), _RND[dtype])
    if rc:
        raise ValueError(f"orc_rmsnorm_quant_f32 failed ({rc})")
    return (q, s) if r is None else (q, s, r, v)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits of float32 values, nearest even (the oracle's C
    rounding, used by rmsnorm_quant_values)."""
    f = np.ascontiguousarray(x, dtype=np.float32).ravel()
    L = lib()
    return np.array([L.orc_float_to_f16(float(t)) for t in f], dtype=np.uint16).reshape(np.shape(x))


# ---------------------------------------------------------------------------
# The reference's own CPU path, restated in torch (timed as the CPU baseline)
# ---------------------------------------------------------------------------
# tasks/reference/L1/fp8_linear.py is the reference's torch-only semantic
# version of the path: the weight is dequantized per 128x128 block
# (_expand_weight_scale, :24-38) and multiplied in fp32 by F.linear (:96-104);
# the activation quant is :41-64.  These restatements run on the host cores
# for the bench's CPU baseline; they are not checkers (the C routines above
# are), but the test suite checks them against those.

def torch_expand_weight_scale(scale, rows: int, cols: int):
    """Per-element fp32 weight scale of a [rows, cols] block-scaled weight
    (fp8_linear.py:24-38, the [ceil(r/128), ceil(c/128)] case)."""
    s = scale.float()
    return s.repeat_interleave(GROUP, dim=-2).repeat_interleave(GROUP, dim=-1)[..., :rows, :cols]


def torch_dense_linear(a_bf16, w_codes, w_scale):
    """Fp8Linear.forward of the reference CPU path (fp8_linear.py:96-104):
    fp32 dequantized weight, F.linear of the fp32 input, bf16 result.  Pass
    the bf16 input (the literal form) or its 1x128-quantized-dequantized copy
    (the form the GPU path computes)."""
    import torch
    import torch.nn.functional as F
    n, k = w_codes.shape
    w = w_codes.float() * torch_expand_weight_scale(w_scale, n, k)
    return F.linear(a_bf16.reshape(-1, k).float(), w).to(torch.bfloat16)


def torch_quant_group128(x_bf16, use_ue8m0: bool = True, eps: float = EPS):
    """Per-token-group 1x128 quant of the reference CPU path (fp8_linear.py:
    41-64): fp32 group absmax clamped below at eps, divided by 448, rounded
    up to a power of two by 2^ceil(log2(.)), then codes = fp8(clamp(x / s))."""
    import torch
    flat = x_bf16.reshape(-1, x_bf16.shape[-1]).float()
    groups = flat.shape[-1] // GROUP
    g = flat.view(flat.shape[0], groups, GROUP)
    scale = g.abs().amax(dim=-1).clamp_min(eps) / FP8_MAX
    if use_ue8m0:
        scale = torch.pow(2.0, torch.ceil(torch.log2(scale)))
    q = torch.clamp(flat / scale.repeat_interleave(GROUP, dim=-1), -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale


def torch_dequant_group128(q, scale):
    """fp32 values of 1x128-quantized activations (codes x group scale)."""
    return q.float() * scale.repeat_interleave(GROUP, dim=-1)


def torch_grouped_linear(a_codes, a_scale, w_codes, w_scale, expert_ids):
    """The contiguous-layout grouped GEMM as a per-expert-segment loop of the
    reference's dense CPU path (fused_experts.py:32-136 layout; dequantized
    operands, fp32 matmul, bf16 rows): returns {row: output} for the rows of
    every expert that expert_ids names."""
    import torch
    out = {}
    ids = expert_ids.tolist()
    rows = [r for r, e in enumerate(ids) if e >= 0]
    by_e: dict = {}
    for r in rows:
        by_e.setdefault(ids[r], []).append(r)
    a = torch_dequant_group128(a_codes, a_scale)
    n, k = w_codes.shape[-2:]
    for e, rs in by_e.items():
        w = w_codes[e].float() * torch_expand_weight_scale(w_scale[e], n, k)
        y = (a[rs] @ w.t()).to(torch.bfloat16)
        for i, r in enumerate(rs):
            out[r] = y[i]
    return out
