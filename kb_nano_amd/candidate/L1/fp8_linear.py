"""kernel_swapper candidate for target ``fp8_linear``.

Copy (or symlink) to ``tasks/candidate/L1/fp8_linear.py`` in a kb_nano tree.
The loader (infra/kernel_swapper.py:328-355) imports this file standalone
and picks the class named like the baseline's target class, ``Fp8Linear``,
so only absolute imports are used."""
from kb_nano_amd.fp8_linear import (  # noqa: F401
    Fp8Linear,
    PerTokenGroupQuantFp8,
    _alloc_colmajor_scale,
    _Fp8PrefillBufs,
    postprocess_fp8_weights,
    postprocess_fp8_weights_batched,
)
