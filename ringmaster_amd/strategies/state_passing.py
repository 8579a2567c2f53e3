"""Context-parallel linear scan on the MI355X (strategies/state_passing.py:19-59).

``cp_linear_scan`` computes ``h_t = a_t h_{t-1} + b_t`` over ``world`` contiguous
shards exactly as the reference's state passing does (zero-init local scan per
shard, prefix-combine of the shards' (decay, carry) pairs in rank order, then
``h += cumA * H_in``), with the P shards emulated in one kernel on one GPU. It is
differentiable: the backward is the exact gradient of the same map.

``a`` is ``[batch, L, d]`` (elementwise decay, as in the reference) or
``[batch, L, G]`` with ``G`` dividing ``d`` (one decay per channel group, e.g. a
Mamba2 head decay broadcast over headdim x d_state); ``b`` is ``[batch, L, d]``.
"""

from __future__ import annotations

import torch

from ringmaster_amd import abi


def _prep(a, b, world):
    abi.require_device(a, b)
    if a.dim() != 3 or b.dim() != 3 or a.shape[:2] != b.shape[:2]:
        raise ValueError("a must be [batch, L, d or G] and b [batch, L, d]")
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise NotImplementedError("the MI355X scan carries fp32 states")
    groups = a.shape[2]
    if b.shape[2] % groups:
        raise ValueError(f"decay groups {groups} must divide d {b.shape[2]}")
    if b.shape[1] % world:
        raise ValueError(f"L {b.shape[1]} not divisible by world {world}")
    return a.contiguous(), b.contiguous(), groups


def linear_scan_forward(a, b, world: int = 1, return_chunk_state: bool = False):
    a, b, groups = _prep(a, b, world)
    batch, L, d = b.shape
    h = torch.empty_like(b)
    cs = torch.empty((world, batch, 2, d), dtype=torch.float32, device=b.device) \
        if return_chunk_state else None
    abi.check(abi.lib().rmx_linear_scan_fwd(a.data_ptr(), b.data_ptr(), h.data_ptr(),
                                            abi.ptr(cs), batch, L, d, groups, world,
                                            abi.stream_of(b)))
    return (h, cs) if return_chunk_state else h


def linear_scan_backward(a, h, dh, world: int = 1):
    a, h, groups = _prep(a, h, world)
    abi.require_device(dh)
    if dh.shape != h.shape:
        raise ValueError("dh must be shaped like h")
    dh = dh.contiguous().float()
    batch, L, d = h.shape
    da = torch.zeros_like(a)
    db = torch.empty_like(h)
    abi.check(abi.lib().rmx_linear_scan_bwd(a.data_ptr(), h.data_ptr(), dh.data_ptr(),
                                            da.data_ptr(), db.data_ptr(), batch, L, d, groups,
                                            world, abi.stream_of(h)))
    return da, db


class _CPLinearScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, world):
        h = linear_scan_forward(a, b, world)
        ctx.save_for_backward(a, h)
        ctx.world = world
        return h

    @staticmethod
    def backward(ctx, dh):
        a, h = ctx.saved_tensors
        da, db = linear_scan_backward(a, h, dh, ctx.world)
        return da, db, None


def local_linear_scan(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """h_t = a_t h_{t-1} + b_t from zero (strategies/state_passing.py:19-26)."""
    return _CPLinearScan.apply(a, b, 1)


def cp_linear_scan(a: torch.Tensor, b: torch.Tensor, world: int) -> torch.Tensor:
    """Exact CP linear scan of the full ``[batch, L, d]`` sequence split into ``world``
    contiguous shards; returns every shard's corrected hidden states (rank order)."""
    return _CPLinearScan.apply(a, b, int(world))
