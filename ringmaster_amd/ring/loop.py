"""The ring attention entry points of ring/loop.py, P ranks emulated on one MI355X.

``ring_attention`` dispatches like the reference (ring/loop.py:20-61): one rank is a
single block call, ``rotate_method="allgather"`` is the gather-then-attend ring
(:201-228), anything else (the reference's ``alltoall``) is the p2p ring with its
preconditions (FA2-class implementation, zero dropout, no window: :52-57).
``varlen_ring_attention`` attends within each packed document over the gathered K/V
(:102-198), each batch row with its own documents. Inputs are the per-rank interface tensors ``[b, H, L, d]`` stacked on a
leading rank axis; outputs are ``[P, b, L, H, d]``.

Gathering K/V and attending once per rank computes the same blocks as the p2p ring
(a bottom-right causal mask over ``K[0 : (r + 1) L]`` is the ring's diagonal-causal
plus full earlier blocks), so both methods run the emulated contiguous ring: on one
GPU every rank already reads every KV block in place from HBM.

Sliding windows (the gather ring and the packed ring: ring/loop.py:185-186,201-228)
keep the reference's positions: the gather ring's single block call aligns rank r's
queries bottom-right against the gathered keys, which for a causal ring is the global
position ``r L + i`` and for a non-causal ring (all P blocks gathered) ``(P - 1) L + i``;
there the window is the block provider's, flash attention's ``(left, right)`` (a
non-causal ring bounded on the right too); the packed ring compares global indices and
reads ``left`` only, as its math path does (:185-186). Dropout in the gather ring draws one mask over
(global query, gathered key) pairs per call; its blocks take their coordinates from it.
"""

from __future__ import annotations

import torch

from ringmaster_amd.ring.kernels import PROVIDERS, new_dropout_seed, window_bounds, window_left
from ringmaster_amd.ring.p2p_attn import contiguous_ring
from ringmaster_amd.ring.zigzag import doc_for


def _method(rotate_method) -> str:
    return str(getattr(rotate_method, "value", rotate_method)).lower()


def ring_attention(q, k, v, *, group=None, causal: bool, scaling=None, dropout: float = 0.0,
                   provider: str = "mi355x_hip", rotate_method="alltoall",
                   attn_implementation: str = "flash_attention_2", window=None, timer=None):
    """q/k/v: [P, b, H, L, d]; returns [P, b, L, H, d]."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    if provider not in PROVIDERS:
        raise KeyError(provider)
    if provider != "mi355x_hip":
        raise NotImplementedError(f"provider {provider!r} has no MI355X ring in this build")
    if q.dim() != 5:
        raise ValueError("q/k/v must be [world, b, H, L, d]")
    if q.shape[0] == 1:
        block = PROVIDERS[provider]
        out, _ = block(q[0].transpose(1, 2), k[0].transpose(1, 2), v[0].transpose(1, 2),
                       causal=causal, scaling=scaling, dropout=dropout,
                       attn_implementation=attn_implementation, window=window)
        return out.unsqueeze(0)
    if _method(rotate_method) == "allgather":
        if not 0.0 <= float(dropout) < 1.0:
            raise ValueError(f"dropout must lie in [0, 1) (got {dropout})")
        drop = (float(dropout), new_dropout_seed(q.device)) if dropout else None
        # the block provider's window (flash semantics); rank r's L queries sit bottom-right
        # against at least L gathered keys, so bounds of sk keys or more change nothing
        left, right = window_bounds(window, bool(causal))
        P, L = q.shape[0], q.shape[3]
        bounds = rights = None
        if left is not None:  # bottom-right aligned against the gathered keys
            bounds = [left if causal else left - (P - 1 - r) * L for r in range(P)]
        if right is not None:  # non-causal: query i of rank r at (P - 1) L + i
            rights = [right + (P - 1 - r) * L for r in range(P)]
        return contiguous_ring(q, k, v, causal=causal, scaling=scaling, timer=timer,
                               window=bounds, dropout=drop, right=rights)
    if dropout or window is not None or attn_implementation not in ("flash_attention_2", "math"):
        raise ValueError("P2P Ring requires FA2, zero dropout, and no sliding window")
    return contiguous_ring(q, k, v, causal=causal, scaling=scaling, timer=timer)


def varlen_ring_attention(q, k, v, *, group=None, scaling, cu_seqlens, causal=True,
                          dropout=0.0, window=None, attn_implementation="math", timer=None):
    """Packed documents over contiguous shards (ring/loop.py:103-198): ``cu_seqlens`` covers
    the ``b S`` tokens of the flattened batch (``S = P L``), and batch row ``i`` packs the
    documents of tokens ``[i S, (i + 1) S)`` (:178). A query at global position ``r L + i``
    of its row attends the keys of its own document in that row: the earlier ones
    (``causal``, :183-184), or all of them (``causal=False``, keys up to the document end as
    in :149), within ``window[0]`` positions behind it when a window is given (:185-186).
    ``dropout`` drops probabilities with the kernels' hash mask over (row, head, global query,
    gathered key). q/k/v: [P, b, H, L, d]; returns [P, b, L, H, d]."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    if not 0.0 <= float(dropout) < 1.0:
        raise ValueError(f"dropout must lie in [0, 1) (got {dropout})")
    if not isinstance(cu_seqlens, torch.Tensor):
        cu_seqlens = torch.as_tensor(cu_seqlens)
    left = window_left(window)
    if left is not None and not causal:
        raise NotImplementedError("sliding windows on a non-causal packed ring are not supported")
    drop = (float(dropout), new_dropout_seed(q.device)) if dropout else None
    return contiguous_ring(q, k, v, causal=bool(causal), scaling=scaling,
                           doc=doc_for(cu_seqlens, q, rows=q.shape[1]), timer=timer,
                           window=None if left is None else [left] * q.shape[0], dropout=drop)
