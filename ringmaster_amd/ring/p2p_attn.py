"""Contiguous p2p ring attention, P ranks emulated on one MI355X.

Counterpart of ``RingP2PAttention`` / ``ring_p2p_attention`` (ring/p2p_attn.py:121-291):
rank ``r`` holds the contiguous chunk ``r`` of the sequence; at step ``s`` it attends
the KV block of rank ``(r - s) mod P`` (hop direction ring/p2p_attn.py:65-69), causal
rings skipping ``s > r`` and masking only the step-0 diagonal; the online-softmax merge
runs in the forward epilogue and the backward uses the global out/lse, the dK/dV
accumulators of a block updated in place at its owner (what the reference's dk/dv
rotation achieves after P hops, :243-281). One batched launch per ring step covers
every rank, as for the zigzag ring.
"""

from __future__ import annotations

import math

from ringmaster_amd.ring.zigzag import EmulatedRing, check_ring_inputs


def contiguous_ring(q, k, v, *, causal: bool, scaling=None, doc=None, timer=None, window=None,
                    dropout=None, right=None):
    """q/k/v: [P, b, H, L, d] bf16, rank r's contiguous interface tensors stacked on
    dim 0. Returns out [P, b, L, H, d]. ``doc``: per-token document ids of the packed
    sequence, [S] or [b, S] per batch row (document-masked blocks; without ``causal`` every
    key of the query's document). ``window``: one bound per rank on the global
    ``pos_q - pos_k`` of its queries (sliding windows), or None; ``right`` (non-causal rings
    without documents): one bound per rank on the global ``pos_k - pos_q``, or None.
    ``dropout``: None or (p, seed), one mask over (global query, global key) for every
    block."""
    check_ring_inputs(q, k, v)
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q.shape[-1])
    return EmulatedRing.apply(q, k, v, float(scale), doc, timer, "contiguous", bool(causal),
                              None if window is None else tuple(int(w) for w in window), dropout,
                              None if right is None else tuple(int(w) for w in right))


def ring_p2p_attention(q, k, v, *, group=None, causal, scaling, timer=None):
    """q/k/v: [P, b, H, L, d]; returns [P, b, L, H, d] (each rank's interface output
    layout, ring/p2p_attn.py:284-291). ``group`` must be None: the ranks are the
    leading axis. GQA is native (no KV repetition)."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    return contiguous_ring(q, k, v, causal=causal, scaling=scaling, timer=timer)
