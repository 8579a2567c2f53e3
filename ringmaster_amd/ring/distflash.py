"""DistFlashAttn-style load-balanced causal ring, P ranks emulated on one MI355X.

Counterpart of ``DistFlashAttention`` / ``distflash_attention``
(ring/distflash.py:87-291). The reference keeps each rank's tokens contiguous and
balances the causal triangle by routing work: at distance ``d`` the block
``(q_i, kv_{i-d})`` is computed by the helper rank ``i - d`` (``d <= P // 2``, its
partial (out, lse) routed back to the owner) or by the owner ``i`` itself
(``d > P // 2``). Every causal block is computed exactly once, with the global merged
out/lse in the backward.

The emulation runs ``schedule.distflash_schedule``: the reference's steps in its merge
order (diagonal, owner-local phase 2, routed phase 1), each block tagged with the rank
that computes it. One launch per step covers every rank's block of that step; a routed
partial is merged straight into its owner's fp32 accumulator (the route is an address).
``only_ranks`` in ``ring_forward`` / ``ring_backward`` runs one worker's blocks at that
GPU's own grid, which is how ``bench.py --per-rank`` times the balance
(``schedule.distflash_work``: 5,5,5,5,4,4,4,4 blocks at P = 8).
"""

from __future__ import annotations

import math

from ringmaster_amd.ring.zigzag import EmulatedRing, check_ring_inputs, doc_for


def distflash_attention(q, k, v, *, group=None, scaling, cu_seqlens=None,
                        attn_implementation="flash_attention_2", timer=None):
    """Balanced contiguous causal ring. q/k/v: [P, b, H, L, d] (rank r's contiguous
    interface tensors stacked on dim 0); returns [P, b, L, H, d]. ``cu_seqlens`` set =>
    packed (document-masked) blocks, global offsets ``r * L`` (ring/distflash.py:73-85)."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    check_ring_inputs(q, k, v)
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q.shape[-1])
    return EmulatedRing.apply(q, k, v, float(scale), doc_for(cu_seqlens, q), timer, "distflash",
                              True)
