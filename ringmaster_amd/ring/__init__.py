"""Ring-attention compute path: block provider, merge, ring schedules and emulated rings."""

from ringmaster_amd.ring.distflash import distflash_attention  # noqa: F401
from ringmaster_amd.ring.kernels import PROVIDERS, flash_ops, mi355x_hip_block  # noqa: F401
from ringmaster_amd.ring.loop import ring_attention, varlen_ring_attention  # noqa: F401
from ringmaster_amd.ring.merge import update_out_and_lse  # noqa: F401
from ringmaster_amd.ring.p2p_attn import ring_p2p_attention  # noqa: F401
from ringmaster_amd.ring.zigzag import zigzag_ring_attention  # noqa: F401
