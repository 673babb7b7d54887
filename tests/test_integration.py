"""CPU test of the kb_nano binding (kb_nano_amd.integration): a minimal fake
tree laid out like kb_nano's (package root, tasks/baseline/L1 + L2, infra),
written here from scratch, whose baseline modules fail to import the way the
reference's do on ROCm (``import deep_gemm``).  With the aliases installed,
target discovery in the style of infra/kernel_swapper.py:183-214 (import the
baseline module, take the last nn.Module class defined in it, :131-144), the
model file's relative import, a class swap in the style of :294-305 and the
weight loader's import of postprocess_fp8_weights (infra/weight_loader.py:
1015-1017) all resolve to kb_nano_amd."""
import importlib
import os
import sys
import textwrap

import pytest
import torch.nn as nn

FILES = {
    "__init__.py": "",
    "tasks/__init__.py": "",
    "tasks/baseline/__init__.py": "",
    "tasks/baseline/L1/__init__.py": "",
    "tasks/baseline/L2/__init__.py": "",
    "infra/__init__.py": "",
    # the baseline modules of the path, as unimportable on ROCm as the real ones
    "tasks/baseline/L1/fp8_linear.py": "import deep_gemm\n",
    "tasks/baseline/L1/fp8_grouped_gemm_contiguous.py": "import deep_gemm\n",
    "tasks/baseline/L1/silu_mul_quant_fp8.py": "import triton_for_cuda_only\n",
    "tasks/baseline/L1/moe_grouped_gemm.py": "from .fp8_grouped_gemm_contiguous import *\n",
    "tasks/baseline/L1/moe_align.py": "from .csrc import _C\n",
    "tasks/baseline/L1/moe_sum.py": "from .csrc import _C\n",
    "tasks/baseline/L1/rmsnorm_quant.py": "from .csrc import _C\n",
    "tasks/baseline/L2/fused_experts.py": "from ..L1.fp8_linear import PerTokenGroupQuantFp8\n",
    "tasks/baseline/L2/vllm_fused_experts.py": "import vllm._C\n",
    # a model file: relative imports of the L1 / L2 modules
    "tasks/baseline/L2/toy_mla.py": textwrap.dedent("""
        import torch.nn as nn
        from ..L1.fp8_linear import Fp8Linear
        from .fused_experts import FusedExperts

        class ToyBlock(nn.Module):
            def __init__(self):
                super().__init__()
                self.q_b = Fp8Linear()
                self.experts = FusedExperts()
    """),
    # the engine side: discovery, swap and the weight loader's import
    "infra/swap.py": textwrap.dedent("""
        import importlib, sys
        import torch.nn as nn
        PKG = __package__.rsplit(".", 1)[0]

        def last_module_class(mod):
            found = None
            for v in vars(mod).values():
                if isinstance(v, type) and issubclass(v, nn.Module) and v is not nn.Module \\
                        and v.__module__ == mod.__name__:
                    found = v
            return found

        def discover(names):
            return {n: last_module_class(importlib.import_module(f"{PKG}.tasks.baseline.{n}")) for n in names}

        def patch(original, replacement):
            undo = []
            for name, mod in list(sys.modules.items()):
                if mod is None or not name.startswith(PKG):
                    continue
                for attr in list(vars(mod)):
                    if getattr(mod, attr, None) is original:
                        undo.append((mod, attr))
                        setattr(mod, attr, replacement)
            return undo

        def restore(undo, original):
            for mod, attr in undo:
                setattr(mod, attr, original)
    """),
    "infra/weight_loader.py": textwrap.dedent("""
        def postprocess_names():
            from ..tasks.baseline.L1.fp8_linear import Fp8Linear, postprocess_fp8_weights, \\
                postprocess_fp8_weights_batched
            return Fp8Linear, postprocess_fp8_weights, postprocess_fp8_weights_batched
    """),
}

# target class of each baseline module: the last nn.Module class the
# reference defines in it (tasks/baseline/L1/fp8_linear.py:335,
# silu_mul_quant_fp8.py:79, fp8_grouped_gemm_contiguous.py:136,
# moe_grouped_gemm.py:282, moe_align.py:17, moe_sum.py:14,
# rmsnorm_quant.py:102, L2/fused_experts.py:156, L2/vllm_fused_experts.py:100)
TARGETS = {
    "L1.fp8_linear": "Fp8Linear",
    "L1.silu_mul_quant_fp8": "SiluMulQuantFp8",
    "L1.fp8_grouped_gemm_contiguous": "Fp8GroupedGemmContiguous",
    "L1.moe_grouped_gemm": "MoeGroupedGemm",
    "L1.moe_align": "MoeAlign",
    "L1.moe_sum": "MoeSum",
    "L1.rmsnorm_quant": "FusedAddRMSNormFP8Quant",
    "L2.fused_experts": "FusedExperts",
    "L2.vllm_fused_experts": "VllmFusedExperts",
}


@pytest.fixture
def fake_tree(tmp_path):
    pkg = "fake_kbnano_tree"
    for rel, text in FILES.items():
        p = tmp_path / pkg / rel
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(text)
    sys.path.insert(0, str(tmp_path))
    try:
        yield pkg
    finally:
        sys.path.remove(str(tmp_path))
        for name in [n for n in sys.modules if n == pkg or n.startswith(pkg + ".")]:
            del sys.modules[name]


def test_baseline_modules_fail_without_the_aliases(fake_tree):
    with pytest.raises(ImportError):
        importlib.import_module(f"{fake_tree}.tasks.baseline.L1.fp8_linear")


def test_tree_resolves_to_kb_nano_amd(fake_tree):
    import kb_nano_amd
    from kb_nano_amd import integration
    from kb_nano_amd import fp8_linear as ours
    installed = integration.install(fake_tree)
    assert len(installed) == len(integration.ALIASES)

    swap = importlib.import_module(f"{fake_tree}.infra.swap")
    found = swap.discover(list(TARGETS))
    for name, cls_name in TARGETS.items():
        cls = found[name]
        assert cls is not None and cls.__name__ == cls_name, (name, cls)
        assert cls.__module__.startswith("kb_nano_amd."), (name, cls.__module__)

    toy = importlib.import_module(f"{fake_tree}.tasks.baseline.L2.toy_mla")
    assert toy.Fp8Linear is kb_nano_amd.Fp8Linear
    assert toy.FusedExperts is kb_nano_amd.FusedExperts

    wl = importlib.import_module(f"{fake_tree}.infra.weight_loader")
    lin, pp, ppb = wl.postprocess_names()
    assert lin is ours.Fp8Linear and pp is ours.postprocess_fp8_weights
    assert ppb is ours.postprocess_fp8_weights_batched

    # a candidate class swapped in (and out) everywhere the tree refers to the target
    class Candidate(nn.Module):
        pass
    original = found["L1.fp8_linear"]
    undo = swap.patch(original, Candidate)
    try:
        assert undo and toy.Fp8Linear is Candidate
        assert isinstance(toy.ToyBlock().q_b, Candidate)
    finally:
        swap.restore(undo, original)
    assert toy.Fp8Linear is original and ours.Fp8Linear is original


def test_install_refuses_after_the_tree_was_imported(fake_tree):
    from kb_nano_amd import integration
    sys.modules[f"{fake_tree}.tasks.baseline.L1.moe_sum"] = type(os)("stale")
    with pytest.raises(RuntimeError, match="before anything imports"):
        integration.install(fake_tree, only=["tasks.baseline.L1.moe_sum"])
