"""CPU restatement of the zigzag shard (test infrastructure only).

Follows balancers.py:11-29 (index generators), shard.py:34-36 (pad multiple),
shard.py:120-147 (global shift labels, padding: ids 0, labels -100, position ids
continuing) and shard.py:150-176 (``_zigzag_shard``); the unshard is the
position-id scatter of tests/test_zigzag_shard.py:39-43.
"""

from __future__ import annotations

import torch


def contiguous_indices(seq_len, world):
    if seq_len % world != 0:
        raise ValueError(f"seq_len {seq_len} not divisible by world {world}")
    c = seq_len // world
    return [list(range(r * c, (r + 1) * c)) for r in range(world)]


def head_tail_indices(seq_len, world):
    if seq_len % (2 * world) != 0:
        raise ValueError(f"seq_len {seq_len} not divisible by 2*world ({2 * world}) for head_tail")
    c = seq_len // (2 * world)
    return [list(range(r * c, (r + 1) * c)) + list(range((2 * world - 1 - r) * c, (2 * world - r) * c))
            for r in range(world)]


def pad_multiple(seq_len, cp_size):
    rem = seq_len % cp_size
    return 0 if rem == 0 else cp_size - rem


def zigzag_index(total, rank, world):
    half = total // (2 * world)
    lo, hi = rank, 2 * world - 1 - rank
    return torch.cat([torch.arange(lo * half, (lo + 1) * half),
                      torch.arange(hi * half, (hi + 1) * half)])


def zigzag_shard_tensor(x, world, rank, pad_value=0):
    """[b, S, ...] -> rank's [b, L, ...] with padding rows of ``pad_value``."""
    seq = x.shape[1]
    pad = pad_multiple(seq, 2 * world)
    if pad:
        x = torch.cat([x, torch.full((x.shape[0], pad, *x.shape[2:]), pad_value, dtype=x.dtype)], 1)
    return x.index_select(1, zigzag_index(seq + pad, rank, world)).contiguous()


def zigzag_unshard_tensor(shards, seq):
    """list of per-rank [b, L, ...] -> [b, seq, ...] by global position scatter."""
    world = len(shards)
    local = shards[0].shape[1]
    total = world * local
    full = torch.empty((shards[0].shape[0], total, *shards[0].shape[2:]), dtype=shards[0].dtype)
    for r, sh in enumerate(shards):
        full[:, zigzag_index(total, r, world)] = sh
    return full[:, :seq]


def zigzag_shard_batch(batch, cp_rank, cp_size):
    """``_zigzag_shard`` (shard.py:150-176) on a dict of CPU tensors."""
    bsz, seq_len = batch["input_ids"].shape[:2]
    pad_len = pad_multiple(seq_len, 2 * cp_size)
    if "shift_labels" not in batch and batch.get("labels") is not None:
        labels = batch["labels"]
        shift = torch.full_like(labels, -100)
        shift[:, :-1] = labels[:, 1:]
        batch["shift_labels"] = shift
    if batch.get("position_ids") is None:
        batch["position_ids"] = torch.arange(seq_len, dtype=torch.long).unsqueeze(0).expand(bsz, -1)
    total = seq_len + pad_len
    if pad_len:
        for key, val in list(batch.items()):
            if isinstance(val, torch.Tensor) and val.dim() > 1 and val.size(1) == seq_len:
                fill = -100 if key in ("labels", "shift_labels") else 0
                pad = torch.full((val.size(0), pad_len, *val.shape[2:]), fill, dtype=val.dtype)
                if key == "position_ids" and val.ndim == 2:
                    pad = val[:, -1:] + torch.arange(1, pad_len + 1, dtype=val.dtype)
                batch[key] = torch.cat([val, pad], dim=1)
    idx = zigzag_index(total, cp_rank, cp_size)
    for key, val in list(batch.items()):
        if isinstance(val, torch.Tensor) and val.dim() > 1 and val.size(1) == total:
            batch[key] = val.index_select(1, idx).contiguous()
    return batch, (seq_len, pad_len)
