"""kernel_swapper candidate for target ``moe_sum`` (class ``MoeSum``); copy
to ``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.moe_sum import MoeSum  # noqa: F401
