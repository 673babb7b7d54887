"""Writes the committed golden fixtures of this directory from the CPU oracle.

The reference ships no golden vectors for the FP8 linear path, so these
fixtures are this build's own regression anchors, produced by the oracle
(itself pinned exhaustively and by closed forms in tests/test_oracle.py):

* quant_edge.npz        -- 1x128 quant of an edge-case bf16 tensor [8, 1024]:
                           zero groups, groups whose absmax is 448 * 2^k, e4m3
                           round-half-even ties, subnormal-range values,
                           near-bf16-max values, mixed signs; UE8M0 and plain
                           fp32 scales.
* silu_mul_quant.npz    -- fused SiLU*Mul + quant of a seeded [128, 512] bf16
                           input (gate | up, 0.1% x50 outliers, tiny values).
* gemm_cfg1.npz         -- BASELINE config 1 (M=64, N=K=2048, seed 0): hashes
                           of the quantized inputs, the sha256 of the oracle's
                           bf16 output and its first 16 rows x 64 columns.

Run from the repository root:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests._util import bf16_bits, quantized_gemm_inputs, seeded_bf16  # noqa: E402


def quant_edge_input() -> np.ndarray:
    g = torch.Generator().manual_seed(11)
    x = torch.randn(8, 1024, generator=g)
    x[0, :256] = 0.0                                        # two all-zero groups
    x[1, :128] = 448.0 * torch.linspace(-1, 1, 128)         # absmax exactly 448 (scale 1)
    x[1, 128:256] = 448.0 * 2.0 ** 5 * torch.linspace(-1, 1, 128)   # absmax 448 * 2^5
    # e4m3 ties under scale 1: 1.0625 -> 1.0, 1.1875 -> 1.25, 3.125 -> 3.0, 0.0087890625 -> 4 * 2^-9 (subnormal)
    ties = torch.tensor([1.0625, 1.1875, -1.0625, -1.1875, 3.125, -3.125, 0.0087890625, -0.0087890625, 448.0])
    x[2, 256:384] = 0.5
    x[2, 256:256 + len(ties)] = ties
    x[3, :] = torch.randn(1024, generator=g) * 1e-30        # subnormal-range inputs
    x[4, :] = 3.0e38 * torch.sign(torch.randn(1024, generator=g))  # near bf16 max
    x[5, ::7] *= 50.0                                       # outliers
    x[6, :] = -x[6, :].abs()                                # all negative
    x[7, 512:640] = 2.0 ** -126                             # bf16 min normal
    return bf16_bits(x.bfloat16())


def silu_input() -> np.ndarray:
    x = seeded_bf16((128, 512), seed=17, outlier_frac=1e-3)
    x[1] = (x[1].float() * 1e-19).bfloat16()               # tiny gate and up values
    x[2, 256:] = (x[2, 256:].float() * 3e-38).bfloat16()   # fp32-subnormal products
    x[3, :256] = 0.0                                        # zero gate
    return bf16_bits(x)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gemm_cfg1():
    M = 64
    N = K = 2048
    qa, sa, qw, sw = quantized_gemm_inputs(M, N, K, seed=0)
    ref = oracle.gemm_nt_sample(qa, sa, qw, sw, ue8m0=True)       # float64, all rows/cols
    ref_bf16 = oracle.f32_to_bf16_bits(ref.astype(np.float32))
    return dict(M=M, N=N, K=K, seed=0,
                inputs_sha256=np.array(sha(qa) + sha(sa) + sha(qw) + sha(sw)),
                out_bf16_sha256=np.array(sha(ref_bf16)),
                out_slice=ref[:16, :64].astype(np.float64))


def main():
    x = quant_edge_input()
    q1, s1 = oracle.quant_group128(x, use_ue8m0=True)
    q0, s0 = oracle.quant_group128(x, use_ue8m0=False)
    np.savez_compressed(os.path.join(HERE, "quant_edge.npz"), x_bits=x, q_ue8m0=q1, s_ue8m0=s1, q_fp32=q0, s_fp32=s0)
    x = silu_input()
    q1, s1 = oracle.silu_mul_quant(x, use_ue8m0=True)
    q0, s0 = oracle.silu_mul_quant(x, use_ue8m0=False)
    np.savez_compressed(os.path.join(HERE, "silu_mul_quant.npz"), x_bits=x, q_ue8m0=q1, s_ue8m0=s1, q_fp32=q0,
                        s_fp32=s0)
    np.savez_compressed(os.path.join(HERE, "gemm_cfg1.npz"), **gemm_cfg1())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
