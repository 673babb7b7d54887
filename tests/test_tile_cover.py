"""CPU checks of the full-size GEMM tests' coverage helpers (tests/_util.py):
the sampled rows x columns hit every output tile of every tile shape the
planner uses, and an output tile that a launch skipped (left NaN) or filled
with stale finite values fails the checks the GPU tests apply.  The dropped
tiles are planted in CPU arrays; no kernel runs."""
import itertools

import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_all_written, assert_gemm_close, quantized_gemm_inputs, tile_cover

TILES = [(64, 64), (64, 128), (128, 128), (128, 256), (256, 256)]
SHAPES = [(1, 10240), (8, 57344), (64, 8192), (128, 24576), (4096, 7168), (4096, 36864), (77, 203), (300, 1000)]


@pytest.mark.parametrize("M,N", SHAPES)
def test_every_tile_holds_a_sample(M, N):
    rows, cols = tile_cover(M, N, np.random.default_rng(M * N))
    assert rows.min() >= 0 and rows.max() < M and cols.min() >= 0 and cols.max() < N
    for bm, bn in TILES:
        rt = np.unique(rows // bm)
        ct = np.unique(cols // bn)
        assert np.array_equal(rt, np.arange(-(-M // bm))), (bm, bn)
        assert np.array_equal(ct, np.arange(-(-N // bn))), (bm, bn)
        # edge tiles: their first and last row / column are sampled
        last_r, last_c = ((M - 1) // bm) * bm, ((N - 1) // bn) * bn
        for r in {0, min(bm, M) - 1, last_r, M - 1}:
            assert r in rows, (bm, r)
        for c in {0, min(bn, N) - 1, last_c, N - 1}:
            assert c in cols, (bn, c)


def _full_gemm(M, N, K, seed):
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=seed)
    return oracle.gemm_nt_sample(qa, sa, qw, sw)


@pytest.mark.parametrize("bm,bn", TILES)
def test_a_dropped_tile_fails(bm, bn):
    """Every tile of a 300 x 640 output, one at a time: left NaN it fails
    the all-written check; filled with a neighbour's values (stale finite
    memory) it fails the oracle comparison at the sampled points."""
    M, N, K = 300, 640, 256
    ref = _full_gemm(M, N, K, seed=5)
    rows, cols = tile_cover(M, N, np.random.default_rng(1))
    assert_gemm_close(torch.from_numpy(ref[rows][:, cols]).bfloat16(), ref[rows][:, cols], "clean")
    for tm, tn in itertools.product(range(-(-M // bm)), range(-(-N // bn))):
        r0, c0 = tm * bm, tn * bn
        r1, c1 = min(r0 + bm, M), min(c0 + bn, N)
        skipped = torch.from_numpy(ref.copy()).bfloat16()
        skipped[r0:r1, c0:c1] = float("nan")
        with pytest.raises(AssertionError, match="unwritten"):
            assert_all_written(skipped, "planted")
        stale = ref.copy()
        stale[r0:r1, c0:c1] = np.roll(ref, 7, axis=1)[r0:r1, c0:c1] * 0.5
        got = torch.from_numpy(stale[rows][:, cols]).bfloat16()
        with pytest.raises(AssertionError):
            assert_gemm_close(got, ref[rows][:, cols], f"tile ({tm}, {tn})")
