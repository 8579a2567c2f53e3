"""Ring-attention compute path: block provider, merge, zigzag schedule and ring."""

from ringmaster_amd.ring.kernels import PROVIDERS, flash_ops, mi355x_hip_block  # noqa: F401
from ringmaster_amd.ring.merge import update_out_and_lse  # noqa: F401
from ringmaster_amd.ring.zigzag import zigzag_ring_attention  # noqa: F401
