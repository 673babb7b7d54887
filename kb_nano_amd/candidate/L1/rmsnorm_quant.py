"""kernel_swapper candidate for target ``rmsnorm_quant`` (classes
``RMSNormFP8Quant``, ``FusedAddRMSNormFP8Quant``); copy to
``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.rmsnorm_quant import FusedAddRMSNormFP8Quant, RMSNormFP8Quant  # noqa: F401
