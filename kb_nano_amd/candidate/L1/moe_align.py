"""kernel_swapper candidate for target ``moe_align`` (class ``MoeAlign``);
copy to ``tasks/candidate/L1/`` in a kb_nano tree."""
from kb_nano_amd.moe_align import MoeAlign  # noqa: F401
