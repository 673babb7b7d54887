"""Binding this package into a kb_nano tree on MI355X.

kb_nano's baseline modules for this path cannot be imported on ROCm:
``tasks/baseline/L1/fp8_linear.py:31`` and ``fp8_grouped_gemm_contiguous.py:26``
import ``deep_gemm``, ``moe_align.py`` / ``moe_sum.py`` / ``rmsnorm_quant.py``
load CUDA extensions (``from .csrc import _C``) and
``tasks/baseline/L2/vllm_fused_experts.py:51`` imports ``vllm._C``.  The
kernel_swapper imports every baseline module a model uses while it discovers
its targets (``infra/kernel_swapper.py:204``), the L2 models import the L1
modules by relative import, and the weight loader imports
``postprocess_fp8_weights[_batched]`` from the baseline ``fp8_linear``
(``infra/weight_loader.py:1015-1017``).  A candidate file alone therefore
never gets the chance to be swapped in: the tree fails at the first of those
imports.

``install(pkg_root)`` makes those module names resolve to this package's
modules (entries in ``sys.modules``), so every import of them -- discovery,
the model files' relative imports, the weight loader -- gets the gfx950
implementation.  It must run before anything imports the tree's
``tasks.baseline`` modules: from a ``sitecustomize.py`` or ``.pth`` hook, or
at the top of the tree's entry point.  Each aliased module defines the same
target class last (the rule of ``_find_module_class``,
``infra/kernel_swapper.py:131-144``), with the reference's name, so
discovery finds the same targets, and ``patch_class``
(``infra/kernel_swapper.py:294-305``) still swaps candidates in and out.
"""
from __future__ import annotations

import importlib
import sys

# kb_nano module (relative to its package root) -> this package's module
ALIASES = {
    "tasks.baseline.L1.fp8_linear": "kb_nano_amd.fp8_linear",
    "tasks.baseline.L1.fp8_grouped_gemm_contiguous": "kb_nano_amd.fp8_grouped_gemm_contiguous",
    "tasks.baseline.L1.silu_mul_quant_fp8": "kb_nano_amd.silu_mul_quant_fp8",
    "tasks.baseline.L1.moe_grouped_gemm": "kb_nano_amd.moe_grouped_gemm",
    "tasks.baseline.L1.moe_align": "kb_nano_amd.moe_align",
    "tasks.baseline.L1.moe_sum": "kb_nano_amd.moe_sum",
    "tasks.baseline.L1.rmsnorm_quant": "kb_nano_amd.rmsnorm_quant",
    "tasks.baseline.L2.fused_experts": "kb_nano_amd.fused_experts",
    "tasks.baseline.L2.vllm_fused_experts": "kb_nano_amd.vllm_fused_experts",
}


def install(pkg_root: str = "kb_nano", only: list[str] | None = None) -> dict[str, str]:
    """Alias the kb_nano baseline modules of this path, under the package
    ``pkg_root`` (the name the tree is imported as), to this package's
    modules.  ``only`` limits it to some of the ``ALIASES`` keys.  Raises if
    one of those names was already imported from the tree (too late: its
    importers hold the old module).  Returns the names installed."""
    done = {}
    for rel, ours in ALIASES.items():
        if only is not None and rel not in only:
            continue
        name = f"{pkg_root}.{rel}"
        mod = importlib.import_module(ours)
        prev = sys.modules.get(name)
        if prev is not None and prev is not mod:
            raise RuntimeError(f"{name} was imported before kb_nano_amd.integration.install(); "
                               "install the aliases before anything imports the tree's baseline modules")
        sys.modules[name] = mod
        done[name] = ours
    return done
