"""DistFlashAttn-style load-balanced causal ring, P ranks emulated on one MI355X.

Counterpart of ``DistFlashAttention`` / ``distflash_attention``
(ring/distflash.py:87-291). The reference keeps each rank's tokens contiguous and
balances the causal triangle by routing work: at distance ``d`` the block
``(q_i, kv_{i-d})`` is computed by the helper rank ``i - d`` (``d <= P // 2``, its
partial (out, lse) routed back to the owner) or by the owner ``i`` itself
(``d > P // 2``). Every causal block is computed exactly once, with the Dao op pair
(or its explicit fallback) using the global merged out/lse in the backward.

On one GPU the helper / owner placement has no counterpart: step ``d`` of the
emulation launches exactly the blocks ``(i, i - d)``, ``i >= d``, for every rank at
once, which is the contiguous ring's step ``d`` (``schedule.contiguous_schedule``);
the per-rank balance the schedule buys on P GPUs is ``schedule.distflash_work``.
The merge order differs from the reference's (diagonal, then owner-local blocks,
then routed partials) only by fp32 rounding.
"""

from __future__ import annotations

from ringmaster_amd.ring.p2p_attn import contiguous_ring
from ringmaster_amd.ring.zigzag import doc_for


def distflash_attention(q, k, v, *, group=None, scaling, cu_seqlens=None,
                        attn_implementation="flash_attention_2", timer=None):
    """Balanced contiguous causal ring. q/k/v: [P, b, H, L, d] (rank r's contiguous
    interface tensors stacked on dim 0); returns [P, b, L, H, d]. ``cu_seqlens`` set =>
    packed (document-masked) blocks, global offsets ``r * L`` (ring/distflash.py:73-85)."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    return contiguous_ring(q, k, v, causal=True, scaling=scaling, doc=doc_for(cu_seqlens, q),
                           timer=timer)
