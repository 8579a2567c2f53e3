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

import ctypes
import os

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


def _h_in(h_in, b):
    if h_in is None:
        return None
    abi.require_device(h_in)
    if h_in.shape != (b.shape[0], b.shape[2]):
        raise ValueError(f"h_in must be [batch, d] = {(b.shape[0], b.shape[2])} "
                         f"(got {tuple(h_in.shape)})")
    if h_in.dtype != torch.float32:
        raise NotImplementedError("the MI355X scan carries fp32 states")
    return h_in.contiguous()


# Below this many channels (batch * d) a thread per channel along L leaves part of the
# MI355X idle, and sequences of CHUNKED_MIN_L tokens or more take the chained scan that is
# parallel over L (measured on MI355X: at 131072 channels x L=2048 the chained scan is
# 12% faster over fwd+bwd, at 524288 x 256 the per-channel scan 1.6x).
CHUNKED_MAX_CHANNELS = (1 << 18) - 1
CHUNKED_MIN_L = 256
_ALGOS = ("auto", "per_channel", "chunked")


def _workspace(algo, batch, L, d, groups, world, chunk_state, device):
    """The L-parallel path's workspace (uint8 tensor), or None for the per-channel path."""
    if algo not in _ALGOS:
        raise ValueError(f"algo must be one of {_ALGOS} (got {algo!r})")
    if algo == "per_channel" or batch * L * d == 0:
        return None
    tc = ctypes.c_int32(0)
    nbytes = abi.lib().rmx_linear_scan_workspace(batch, L, d, groups, ctypes.byref(tc))
    aligned_cs = not chunk_state or (L // world) % tc.value == 0
    if algo == "auto" and not (batch * d <= CHUNKED_MAX_CHANNELS and L >= CHUNKED_MIN_L
                               and aligned_cs):
        return None
    if not aligned_cs:
        raise ValueError(f"the chunked scan returns chunk states only when L / world "
                         f"({L // world}) is a multiple of its {tc.value}-token chunks")
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _debug_status(ws, like):
    """With ``RINGMASTER_AMD_DEBUG=1``, wait for an L-parallel scan and raise RuntimeError if
    one of its chunks gave up waiting for its predecessor (its outputs then hold NaN)."""
    if ws is not None and os.environ.get("RINGMASTER_AMD_DEBUG") == "1":
        abi.check(abi.lib().rmx_linear_scan_status(ws.data_ptr(), ws.numel(), abi.stream_of(like)))


def linear_scan_forward(a, b, world: int = 1, return_chunk_state: bool = False, h_in=None,
                        algo: str = "auto"):
    """h for the whole ``[batch, L, d]`` input split into ``world`` shards, from ``h_in``
    (``[batch, d]``, zero when None); with ``return_chunk_state`` also every shard's
    ``(A_r, B_r)`` as ``[world, batch, 2, d]``. ``algo``: ``"per_channel"`` (a thread per
    channel walks L), ``"chunked"`` (the chained scan parallel over L) or ``"auto"``
    (chunked for long sequences with few channels)."""
    a, b, groups = _prep(a, b, world)
    h_in = _h_in(h_in, b)
    batch, L, d = b.shape
    ws = _workspace(algo, batch, L, d, groups, world, return_chunk_state, b.device)
    h = torch.empty_like(b)
    cs = torch.empty((world, batch, 2, d), dtype=torch.float32, device=b.device) \
        if return_chunk_state else None
    abi.check(abi.lib().rmx_linear_scan_fwd(a.data_ptr(), b.data_ptr(), abi.ptr(h_in),
                                            h.data_ptr(), abi.ptr(cs), batch, L, d, groups,
                                            world, abi.ptr(ws), 0 if ws is None else ws.numel(),
                                            abi.stream_of(b)))
    _debug_status(ws, b)
    return (h, cs) if return_chunk_state else h


def linear_scan_backward(a, h, dh, world: int = 1, h_in=None, algo: str = "auto"):
    """(da, db) of :func:`linear_scan_forward`, plus dh_in when ``h_in`` is given."""
    a, h, groups = _prep(a, h, world)
    h_in = _h_in(h_in, h)
    abi.require_device(dh)
    if dh.shape != h.shape:
        raise ValueError("dh must be shaped like h")
    dh = dh.contiguous().float()
    batch, L, d = h.shape
    ws = _workspace(algo, batch, L, d, groups, world, False, h.device)
    da = torch.zeros_like(a)
    db = torch.empty_like(h)
    dh_in = torch.empty_like(h_in) if h_in is not None else None
    abi.check(abi.lib().rmx_linear_scan_bwd(a.data_ptr(), h.data_ptr(), abi.ptr(h_in),
                                            dh.data_ptr(), da.data_ptr(), db.data_ptr(),
                                            abi.ptr(dh_in), batch, L, d, groups, world,
                                            abi.ptr(ws), 0 if ws is None else ws.numel(),
                                            abi.stream_of(h)))
    _debug_status(ws, h)
    return (da, db) if h_in is None else (da, db, dh_in)


class _CPLinearScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, world, h_in):
        h = linear_scan_forward(a, b, world, h_in=h_in)
        ctx.save_for_backward(a, h, h_in)
        ctx.world = world
        return h

    @staticmethod
    def backward(ctx, dh):
        a, h, h_in = ctx.saved_tensors
        grads = linear_scan_backward(a, h, dh, ctx.world, h_in=h_in)
        dh_in = grads[2] if h_in is not None else None
        return grads[0], grads[1], None, dh_in


def local_linear_scan(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """h_t = a_t h_{t-1} + b_t from zero (strategies/state_passing.py:19-26)."""
    return _CPLinearScan.apply(a, b, 1, None)


def _group_size(group, call="cp_linear_scan(a, b, group)",
                where="strategies/state_passing.py:29", emulate="world=P") -> int:
    if group is None:
        return 1
    if isinstance(group, int):
        raise TypeError(f"{call}: the third argument is the process group ({where}); "
                        f"emulate P ranks with {emulate}")
    import torch.distributed as dist

    return dist.get_world_size(group)


def cp_linear_scan(a: torch.Tensor, b: torch.Tensor, group=None, *, world: int | None = None,
                   h_in: torch.Tensor | None = None) -> torch.Tensor:
    """Exact context-parallel linear scan ``h_t = a_t h_{t-1} + b_t``
    (``cp_linear_scan(a, b, group)``, strategies/state_passing.py:29-59), differentiable.

    * ``group`` as in the reference: ``None`` (or a group of one rank) scans the given
      chunk from zero, the reference's ``world == 1`` path. This one-GPU build runs no
      collectives, so a group of several ranks raises ``NotImplementedError``.
    * ``h_in`` (fp32 ``[batch, d]``): one rank's call on its local chunk ``a, b [batch,
      L_local, d]`` given the state entering it, i.e. the rank-ordered prefix of the
      earlier ranks' ``(A_j, B_j)`` (``:55-57``, see :func:`cp_scan_prefix`): returns
      ``local_h + cum_a * h_in`` (``:59``); ``h_in`` receives its gradient
      (``a_0 * g_0``), which a multi-process caller returns to the earlier ranks.
    * ``world=P``: the full ``[batch, L, d]`` sequence split into P contiguous shards,
      every rank emulated in one launch (rank order, corrected states of every shard).
    """
    if _group_size(group) != 1:
        raise NotImplementedError(
            "the MI355X build emulates the ranks on one GPU: pass the full sequence with "
            "world=P, or one rank's chunk with its carried-in h_in")
    if world is not None and h_in is not None and int(world) != 1:
        raise ValueError("h_in is the state entering one rank's chunk: use world=1 with it")
    return _CPLinearScan.apply(a, b, int(world or 1), h_in)


def cp_scan_prefix(chunk_states: torch.Tensor) -> torch.Tensor:
    """The state entering every rank's chunk from the gathered ``(A_r, B_r)`` pairs
    (``[world, batch, 2, d]``, what :func:`linear_scan_forward` returns as its chunk
    state): ``H_in_r = A_{r-1} H_in_{r-1} + B_{r-1}``, ``H_in_0 = 0``
    (strategies/state_passing.py:55-57), as ``[world, batch, d]``, by the scan kernel
    over the rank axis."""
    abi.require_device(chunk_states)
    if chunk_states.dim() != 4 or chunk_states.shape[2] != 2:
        raise ValueError("chunk_states must be [world, batch, 2, d]")
    world, batch, _, d = chunk_states.shape
    out = torch.zeros((world, batch, d), dtype=torch.float32, device=chunk_states.device)
    if world > 1:
        a = chunk_states[:-1, :, 0].transpose(0, 1).contiguous().float()   # [batch, world-1, d]
        b = chunk_states[:-1, :, 1].transpose(0, 1).contiguous().float()
        out[1:] = linear_scan_forward(a, b, 1).transpose(0, 1)
    return out
