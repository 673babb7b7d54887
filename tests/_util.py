"""Shared helpers for the parity tests: seeded inputs and comparisons."""
from __future__ import annotations

import numpy as np
import torch

import oracle


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16 tensor (any device)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().astype(np.uint16)


def from_bits(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.int16)).view(torch.bfloat16).to(device)


def fp8_codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def to_fp8(codes: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).to(device)


def seeded_bf16(shape, seed: int, std: float = 1.0, outlier_frac: float = 0.0, outlier_mul: float = 50.0):
    """CPU torch.Generator(seed) draws in fp32, cast to bf16 (the BASELINE
    input recipe: identical bytes for the oracle and the kernel)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    if outlier_frac:
        x = torch.where(torch.rand(*shape, generator=g) < outlier_frac, x * outlier_mul, x)
    return x.bfloat16()


def quantized_gemm_inputs(M: int, N: int, K: int, seed: int, w_std: float = 0.02):
    """A ~ N(0,1) quantized 1x128 and W ~ N(0, w_std) quantized 128x128 by
    the oracle; returns numpy (qa, sa, qw, sw)."""
    a = seeded_bf16((M, K), seed)
    g = torch.Generator().manual_seed(seed + 1000)
    w = (torch.randn(N, K, generator=g) * w_std).numpy()
    qa, sa = oracle.quant_group128(bf16_bits(a))
    qw, sw = oracle.quant_block128(w)
    return qa, sa, qw, sw


def assert_gemm_close(got_bf16: torch.Tensor, ref: np.ndarray, what: str = "") -> dict:
    """bf16 tolerance of the north star: max relative error <= 1e-2 (max |d| /
    max |ref|), cosine >= 0.9999, and elementwise |d| <= 1e-2 + 1e-2*|ref|
    (the kb_nano runner's bf16 atol/rtol)."""
    got = got_bf16.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    d = np.abs(got - ref)
    rel = d.max() / max(np.abs(ref).max(), 1e-30)
    cos = float((got * ref).sum() / max(np.sqrt((got * got).sum() * (ref * ref).sum()), 1e-300))
    bad = d > 1e-2 + 1e-2 * np.abs(ref)
    assert rel <= 1e-2, f"{what}: max relative error {rel:.3e}"
    assert cos >= 0.9999, f"{what}: cosine {cos:.6f}"
    assert not bad.any(), f"{what}: {bad.sum()} elements outside atol=rtol=1e-2"
    return {"rel": rel, "cos": cos}


def tile_cover(M: int, N: int, rng, bm: int = 64, bn: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """Rows and columns whose cross product puts at least one point inside
    every bm x bn block of an M x N output: one random row of each bm-row
    block and one random column of each bn-column block.  Every output tile
    the GEMM planner uses (64x64, 64x128, 128x128, 128x256, 256x192,
    256x256, and the tiles of a split tail) is a union of such blocks, so
    each of them is sampled.  Added to those: the first and last row and
    column of the matrix, and of the first and the last tile at each tile
    size (64, 128 and 256 rows; 64, 128 and 256 columns), i.e. the edges of
    every edge tile."""
    def pick(n, b, sizes):
        nb = -(-n // b)
        out = [i * b + int(rng.integers(0, min(b, n - i * b))) for i in range(nb)]
        for t in sizes:
            last = ((n - 1) // t) * t
            out += [0, min(t, n) - 1, last, n - 1, max(last - 1, 0)]
        return np.unique(np.clip(np.array(out, dtype=np.int64), 0, n - 1))
    return pick(M, bm, (64, 128, 256)), pick(N, bn, (64, 128, 256))


def assert_all_written(D: torch.Tensor, what: str = "") -> None:
    """A GEMM output prefilled with NaN must hold no NaN (or infinity)
    afterwards: an output tile the launch skipped, or wrote only in part,
    fails this wherever it lies."""
    bad = ~torch.isfinite(D)
    if bool(bad.any()):
        idx = bad.nonzero()
        r, c = (int(v) for v in idx[0])
        raise AssertionError(f"{what}: {int(bad.sum())} outputs unwritten or non-finite, first at ({r}, {c})")
