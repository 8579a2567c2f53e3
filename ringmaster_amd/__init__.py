"""ringmaster_amd — MI355X-native ring-attention compute path for ringmaster.

A new block provider (``mi355x_hip``) plus the zigzag ring, LSE merge, zigzag
shard and context-parallel linear scan of axolotl-ai-cloud/ringmaster, computed by
hand-written gfx950 HIP kernels behind the C ABI in ``include/ringmaster_amd.h``.
"""

__version__ = "0.1.0"

from ringmaster_amd.balancers import contiguous_indices, head_tail_indices  # noqa: F401
from ringmaster_amd.ring import (  # noqa: F401
    PROVIDERS,
    flash_ops,
    mi355x_hip_block,
    update_out_and_lse,
    zigzag_ring_attention,
)
from ringmaster_amd.shard import zigzag_shard, zigzag_shard_batch, zigzag_unshard  # noqa: F401
from ringmaster_amd.strategies.state_passing import cp_linear_scan, local_linear_scan  # noqa: F401
