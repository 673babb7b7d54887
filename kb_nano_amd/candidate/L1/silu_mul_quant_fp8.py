"""kernel_swapper candidate for target ``silu_mul_quant_fp8`` (class
``SiluMulQuantFp8``); copy to ``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.silu_mul_quant_fp8 import SiluMulQuantFp8  # noqa: F401
