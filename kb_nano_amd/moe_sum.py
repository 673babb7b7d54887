"""Top-k reduction of the experts' outputs.

Drop-in for ``tasks/baseline/L1/moe_sum.py`` (kb_nano): ``MoeSum.forward(input
[M*topk, D], topk) -> [M, D]`` into a reused output buffer, with
``kbn_moe_sum`` in place of ``_C.moe_sum`` (csrc/moe_sum.cu).  Same
arithmetic: for topk 2..4 a bf16 accumulator rounded after every add, for
other topk the fp32 order of the reference's ``at::sum_out``.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _ops


class MoeSum(nn.Module):
    def __init__(self):
        super().__init__()
        self._output = None

    def forward(self, input: torch.Tensor, topk: int) -> torch.Tensor:
        total = input.size(0)
        M = total // topk
        D = input.size(1)
        if self._output is None or self._output.size(0) < M or self._output.size(1) < D \
                or self._output.device != input.device:
            self._output = torch.empty(M, D, device=input.device, dtype=input.dtype)
        output = self._output[:M, :D]
        _ops.moe_sum(input.view(M, topk, D), output)
        return output
