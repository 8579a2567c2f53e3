"""CPU restatement of the Mamba2 CP causal convolution (test infrastructure only).

The reference wraps ``causal_conv1d_fn`` (from the third-party causal-conv1d
package, not installed here; unpinned: resolved from the transformers module's
globals, mamba.py:29-31) with a halo exchange: every rank all-gathers the last
``width - 1`` tokens of its shard and prepends its predecessor's (zeros on rank 0),
and with packed documents convolves each document segment of its shard separately,
masking the halo by document (mamba.py:46-101). ``causal_conv1d_fn``'s published
semantics are a depthwise conv1d with ``width - 1`` zeros of left padding, then the
activation (None or silu); :func:`causal_conv1d_fn` states that with torch's conv1d.
Only ``tests/`` may import this module.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def causal_conv1d_fn(x, weight, bias=None, activation=None):
    """x [B, C, T], weight [C, W], bias [C] or None -> [B, C, T]."""
    W = weight.shape[-1]
    y = F.conv1d(x, weight.unsqueeze(1), bias, padding=W - 1, groups=x.shape[1])[..., : x.shape[-1]]
    if activation in ("silu", "swish"):
        y = F.silu(y)
    elif activation is not None:
        raise ValueError(activation)
    return y


def doc_ids_from_cu(cu_seqlens):
    """Per-token document id (ring/varlen_blocks.py:45-48)."""
    seg = torch.as_tensor(cu_seqlens, dtype=torch.int64).diff()
    return torch.repeat_interleave(torch.arange(seg.numel()), seg)


def cp_conv(xs, weight, bias=None, activation=None, cu_seqlens=None):
    """The conv hook of mamba.py:46-101 on every rank. xs: per-rank [B, C, L] shards of
    one contiguous sequence; returns the per-rank outputs. The halo is the all-gather of
    every shard's last width - 1 tokens (mamba.py:56); rank r prepends rank r-1's
    (zeros on rank 0, :57). Packed inputs: the shard is cut at document boundaries
    (:72-79); the first segment of a rank > 0 keeps the halo tokens of its own document
    (:83-89); every segment is convolved separately (:90-98)."""
    world = len(xs)
    width = weight.shape[-1] - 1
    if width == 0:
        return [causal_conv1d_fn(x, weight, bias, activation) for x in xs]
    halos = [x[..., -width:] for x in xs]
    L = xs[0].shape[-1]
    documents = None
    if cu_seqlens is not None:
        documents = doc_ids_from_cu(cu_seqlens).reshape(xs[0].shape[0], L * world)
    outs = []
    for rank, x in enumerate(xs):
        prefix = halos[rank - 1] if rank else torch.zeros_like(halos[0])
        if documents is None:
            outs.append(causal_conv1d_fn(torch.cat((prefix, x), dim=-1), weight, bias,
                                         activation)[..., width:])
            continue
        rows = []
        for row in range(x.shape[0]):
            local = documents[row, rank * L:(rank + 1) * L]
            starts = torch.cat((local.new_zeros(1),
                                (local[1:] != local[:-1]).nonzero().flatten() + 1,
                                local.new_tensor([L]))).tolist()
            parts = []
            for start, end in zip(starts[:-1], starts[1:]):
                values = x[row:row + 1, :, start:end]
                if start == 0 and rank:
                    prefix_docs = documents[row, rank * L - width:rank * L]
                    history = prefix[row:row + 1] * (prefix_docs == local[0]).to(x.dtype)
                    values = torch.cat((history, values), dim=-1)
                result = causal_conv1d_fn(values, weight, bias, activation)
                parts.append(result[..., -(end - start):])
            rows.append(torch.cat(parts, dim=-1))
        outs.append(torch.cat(rows, dim=0))
    return outs
