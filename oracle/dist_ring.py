"""CPU restatement of the DISTRIBUTED zigzag ring (test infrastructure only).

Each process is one rank holding its zigzag shard; K/V blocks move to rank + 1
every step by point-to-point messages (the ``_ishift`` hop,
ring/p2p_attn.py:65-84) and, in the backward, the dK/dV accumulators travel with
their KV block (``_shift_sync``, ring/zigzag.py:199-200,244-252) so they are back
at their owner after ``world`` hops. The step cases and the merge follow
ring/zigzag.py:70-149 (forward) and :151-254 (backward) on top of the oracle's
block operations. Used by the gloo test of configs[0]; the product path (one GPU)
emulates the same ring inside one process.
"""

from __future__ import annotations

import math

import torch
import torch.distributed as dist

from oracle.ring_math import (causal_mask, masked_block_bwd, masked_block_fwd, merge_slice,
                              update_out_and_lse)


def ring_shift(t: torch.Tensor, group=None) -> torch.Tensor:
    """Send ``t`` to rank + 1 and receive rank - 1's (ring/p2p_attn.py:65-84)."""
    world = dist.get_world_size(group)
    rank = dist.get_rank(group)
    recv = torch.empty_like(t)
    ops = [dist.P2POp(dist.isend, t.contiguous(), (rank + 1) % world, group),
           dist.P2POp(dist.irecv, recv, (rank - 1) % world, group)]
    for req in dist.batch_isend_irecv(ops):
        req.wait()
    return recv


def zigzag_forward(q, k, v, group=None, scaling=None):
    """q/k/v: this rank's interface tensors [b, H, L, d] (two zigzag chunks). Returns
    (out [b, L, H, d] in q.dtype, lse [b, H, L] fp32) — ring/zigzag.py:70-149."""
    world, rank = dist.get_world_size(group), dist.get_rank(group)
    d = q.shape[-1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(d)
    qd, ck, cv = (t.transpose(1, 2).float().contiguous() for t in (q, k, v))
    L = qd.shape[1]
    half = L // 2
    out = lse = None
    for s in range(world):
        nk = nv = None
        if s + 1 < world:
            nk, nv = ring_shift(ck, group), ring_shift(cv, group)
        if s == 0:
            bo, bl = masked_block_fwd(qd, ck, cv, causal_mask(L, L), scale)
            out, lse = update_out_and_lse(out, lse, bo, bl)
        elif s <= rank:
            bo, bl = masked_block_fwd(qd, ck[:, :half], cv[:, :half], 0.0, scale)
            out, lse = update_out_and_lse(out, lse, bo, bl)
        else:
            bo, bl = masked_block_fwd(qd[:, half:], ck, cv, 0.0, scale)
            out, lse = merge_slice(out, lse, bo, bl, slice(half, None))
        if nk is not None:
            ck, cv = nk, nv
    return out.to(q.dtype), lse.squeeze(-1).transpose(1, 2).contiguous()


def zigzag_backward(dout, q, k, v, out, lse, group=None, scaling=None):
    """Reverse-ring backward with the global out/lse (ring/zigzag.py:151-254).
    dout/out [b, L, H, d]; returns (dq, dk, dv) in the interface layout [b, H, L, d], fp32."""
    world, rank = dist.get_world_size(group), dist.get_rank(group)
    d = q.shape[-1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(d)
    qd, ck, cv = (t.transpose(1, 2).float().contiguous() for t in (q, k, v))
    dod, od = dout.float(), out.float()
    L = qd.shape[1]
    half = L // 2
    dq = torch.zeros_like(qd)
    dk_acc = torch.zeros_like(ck)
    dv_acc = torch.zeros_like(cv)
    for s in range(world):
        nk = nv = None
        if s + 1 < world:
            nk, nv = ring_shift(ck, group), ring_shift(cv, group)
        if s == 0:
            dqb, dkb, dvb = masked_block_bwd(dod, qd, ck, cv, od, lse, causal_mask(L, L), scale)
            dq += dqb
            dk_acc += dkb
            dv_acc += dvb
        elif s <= rank:
            dqb, dk0, dv0 = masked_block_bwd(dod, qd, ck[:, :half], cv[:, :half], od, lse, 0.0,
                                             scale)
            dq += dqb
            dk_acc[:, :half] += dk0
            dv_acc[:, :half] += dv0
        else:
            dq1, dkb, dvb = masked_block_bwd(dod[:, half:], qd[:, half:], ck, cv, od[:, half:],
                                             lse[:, :, half:], 0.0, scale)
            dq[:, half:] += dq1
            dk_acc += dkb
            dv_acc += dvb
        # the accumulators follow their KV block; after `world` hops they are home
        dk_acc, dv_acc = ring_shift(dk_acc, group), ring_shift(dv_acc, group)
        if nk is not None:
            ck, cv = nk, nv
    return dq.transpose(1, 2), dk_acc.transpose(1, 2), dv_acc.transpose(1, 2)
