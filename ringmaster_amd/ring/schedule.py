"""Zigzag ring schedule as per-step lists of block problems (pure host logic).

Restates the step cases of ``ZigzagRingAttention`` (ring/zigzag.py:9-14,127-143 and
the backward :212-252). Rank ``r`` holds zigzag chunks ``r`` (early, rows
``[0, h)``) and ``2P-1-r`` (late, rows ``[h, 2h)``); at step ``s`` it sees the KV
block of rank ``(r - s) mod P`` (ring/zigzag.py:93, direction ring/p2p_attn.py:65-69):

* ``s == 0``       local block, causal on the concatenated ``2h x 2h`` block;
* ``1 <= s <= r``  all Q rows x the early half ``[0, h)`` of the remote KV;
* ``s > r``        the late Q rows ``[h, 2h)`` x the whole remote KV.

The forward additionally tags each block with whether it is the first / last
ring step that touches its Q rows, so the kernel epilogue can initialise the
running fp32 (out, lse) at the first touch and emit the final bf16 out + lse at
the last one. Early rows are last touched at step ``r``, late rows at ``P-1``;
when the two halves of one block disagree the block is split by rows (for the
causal step-0 block: early rows x keys ``[0, h)``, late rows x keys ``[0, 2h)``,
both bottom-right causal, which is exactly the global causal mask again).
"""

from __future__ import annotations

import dataclasses


@dataclasses.dataclass(frozen=True)
class Block:
    rank: int
    q_lo: int
    q_hi: int
    kv_rank: int
    k_lo: int
    k_hi: int
    causal: bool
    first: bool = True
    last: bool = True
    worker: int | None = None  # the rank whose GPU computes the block (None: ``rank``)

    @property
    def runs_on(self) -> int:
        return self.rank if self.worker is None else self.worker

    @property
    def pairs(self) -> int:
        """Attended (q, k) pairs of this block (bottom-right causal when ``causal``)."""
        sq, sk = self.q_hi - self.q_lo, self.k_hi - self.k_lo
        if not self.causal:
            return sq * sk
        off = sk - sq
        return sum(max(0, min(sk, i + off + 1)) for i in range(sq))


def zigzag_schedule(world: int, local_len: int, *, split_final: bool) -> list[list[Block]]:
    """Blocks of every ring step. ``split_final=False`` gives one block per rank per
    step (what the backward uses: each KV block is then visited once per step)."""
    if world < 1:
        raise ValueError("world must be positive")
    if local_len % 2:
        raise ValueError(f"local length {local_len} must hold two equal zigzag chunks")
    h = local_len // 2
    steps: list[list[Block]] = []
    for s in range(world):
        blocks: list[Block] = []
        for r in range(world):
            rem = (r - s) % world
            e_first = l_first = s == 0
            e_last = s == r
            l_last = s == world - 1
            if s == 0:
                if not split_final or e_last == l_last:
                    blocks.append(Block(r, 0, 2 * h, rem, 0, 2 * h, True, True, e_last and l_last))
                else:
                    blocks.append(Block(r, 0, h, rem, 0, h, True, e_first, e_last))
                    blocks.append(Block(r, h, 2 * h, rem, 0, 2 * h, True, l_first, l_last))
            elif s <= r:
                if not split_final or e_last == l_last:
                    blocks.append(Block(r, 0, 2 * h, rem, 0, h, False, False, e_last and l_last))
                else:
                    blocks.append(Block(r, 0, h, rem, 0, h, False, False, e_last))
                    blocks.append(Block(r, h, 2 * h, rem, 0, h, False, False, l_last))
            else:
                blocks.append(Block(r, h, 2 * h, rem, 0, 2 * h, False, False, l_last))
        steps.append(blocks)
    return steps


def zigzag_gidx(rank: int, half: int, world: int) -> list[int]:
    """Global token indices of ``rank``'s two chunks, early then late (ring/zigzag.py:40-46)."""
    return (list(range(rank * half, (rank + 1) * half))
            + list(range((2 * world - 1 - rank) * half, (2 * world - rank) * half)))


def ring_pairs_per_rank(world: int, local_len: int) -> int:
    """Pairs each rank attends: L(L+1)/2 + (P-1) * 2h^2, equal on every rank."""
    h = local_len // 2
    return local_len * (local_len + 1) // 2 + (world - 1) * 2 * h * h


# ---------------------------------------------------------------- contiguous layouts
def contiguous_schedule(world: int, local_len: int, *, causal: bool) -> list[list[Block]]:
    """Blocks of every step of the contiguous ring (rank ``r`` owns tokens
    ``[r L, (r + 1) L)``): at step ``s`` rank ``r`` attends the KV block of rank
    ``(r - s) mod P`` (ring/p2p_attn.py:161-185, hop direction :65-69), all of it;
    causal rings skip ``s > r`` (the KV lies in the future) and make only the
    step-0 diagonal block causal. A rank's rows are first touched at step 0 and last
    at step ``r`` (causal) or ``P - 1``.

    The same per-step block sets are DistFlash's (ring/distflash.py:1-20): its
    step ``d`` computes exactly the blocks ``(i, i - d)``, ``i >= d``, whether a
    helper (``d <= P // 2``, partial routed to the owner) or the owner itself
    (``d > P // 2``) runs them; only the rank doing the work differs."""
    if world < 1:
        raise ValueError("world must be positive")
    if local_len < 1:
        raise ValueError("local length must be positive")
    steps: list[list[Block]] = []
    for s in range(world):
        blocks = []
        for r in range(world):
            if causal and s > r:
                continue
            last = s == (r if causal else world - 1)
            blocks.append(Block(r, 0, local_len, (r - s) % world, 0, local_len,
                                causal and s == 0, s == 0, last))
        steps.append(blocks)
    return steps


def contiguous_gidx(rank: int, local_len: int) -> list[int]:
    """Global token indices of ``rank``'s contiguous chunk."""
    return list(range(rank * local_len, (rank + 1) * local_len))


def distflash_schedule(world: int, local_len: int) -> list[list[Block]]:
    """DistFlash's steps (ring/distflash.py:87-152) in the reference's merge order, every
    causal block ``(q_i, kv_j)``, ``i >= j``, exactly once:

    * step 0: each rank's diagonal block, causal (:113);
    * phase 2, ``d = P//2 + 1 .. P-1`` (:115-121): the query owner ``r`` computes
      ``(q_r, kv_{r-d})`` for ``r >= d`` with the KV block rotated to it;
    * phase 1, ``d = 1 .. P//2`` (:123-133): the helper ``r`` (the KV owner) computes
      ``(q_{r+d}, kv_r)`` for ``r + d < P`` and routes the partial (out, lse) to the
      owner ``r + d``, which merges it after its own blocks.

    ``rank`` is the query owner (whose rows the block merges into), ``kv_rank`` the KV
    owner, ``worker`` the rank that computes it; ``first`` / ``last`` mark the first
    and last block merged into the owner's rows in this order."""
    if world < 1:
        raise ValueError("world must be positive")
    if local_len < 1:
        raise ValueError("local length must be positive")
    half = world // 2
    order = [[(r, r, r) for r in range(world)]]  # (query owner, KV owner, worker)
    for d in range(half + 1, world):
        order.append([(r, r - d, r) for r in range(d, world)])
    for d in range(1, half + 1):
        order.append([(r + d, r, r) for r in range(world - d)])
    last = {}
    for s, step in enumerate(order):
        for qi, _, _ in step:
            last[qi] = s
    return [[Block(qi, 0, local_len, kj, 0, local_len, s == 0, s == 0, last[qi] == s, worker=w)
             for qi, kj, w in step] for s, step in enumerate(order)]


def distflash_work(world: int) -> list[int]:
    """Causal blocks each rank computes under the DistFlash schedule
    (ring/distflash.py:98-152): its diagonal, the owner-local blocks
    ``(r, r - d)`` with ``d > P // 2`` (phase 2) and the helper blocks
    ``(r + d, r)`` with ``1 <= d <= P // 2`` (phase 1). P=4 gives 3, 3, 2, 2
    against the plain ring's 1, 2, 3, 4 (ring/distflash.py:15)."""
    half = world // 2
    work = [1] * world
    for r in range(world):
        work[r] += sum(1 for d in range(half + 1, world) if r - d >= 0)
        work[r] += sum(1 for d in range(1, half + 1) if r + d < world)
    return work
