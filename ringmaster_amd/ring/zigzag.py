"""Zigzag (head_tail) ring attention, P ranks emulated in one process on one MI355X.

Mirrors ``ZigzagRingAttention`` (ring/zigzag.py:70-260): the same three step
cases, the online-softmax merge, and the reverse-ring backward that uses the
GLOBAL merged out/lse for every block and lets the dK/dV accumulators travel
with their KV block to the owner. Differences that come from running every rank
on one GPU (no collectives, one process):

* inputs are the per-rank interface tensors stacked on a leading rank axis,
  ``q/k/v [P, b, H, L, d]`` (each ``[b, H, L, d]`` exactly as the reference
  receives it); the output is ``[P, b, L, H, d]``, grads ``[P, b, H, L, d]``;
* a ring hop is index arithmetic: at step ``s`` rank ``r`` reads the KV block
  of rank ``(r - s) mod P`` in place from HBM (one remote block resident per
  rank per step, within the reference's 2-block prefetch budget), and the
  dK/dV accumulator of that block is updated in place at its owner's slot;
* each ring step is ONE batched kernel launch over all P ranks (their per-rank
  problems share the launch), forward and backward;
* the merge is fused into the forward epilogue, the first/last touch of each
  row group initialises/finalises in-kernel, and gradients accumulate in fp32
  (the reference accumulates in bf16, ring/zigzag.py:165-168).

Packed sequences (``cu_seqlens``) use document masks on global indices for every
block (ring/zigzag.py:86-120,170-209); dense inputs use the causal / full cases.
"""

from __future__ import annotations

import math
import os

import torch

from ringmaster_amd import abi
from ringmaster_amd.ring import ops
from ringmaster_amd.ring.schedule import contiguous_schedule, distflash_schedule, zigzag_schedule


def doc_ids_from_cu(cu_seqlens: torch.Tensor, device, total: int | None = None) -> torch.Tensor:
    """Per-token document id over the full sequence (ring/varlen_blocks.py:45-48).

    With ``total`` (the sequence length) the ids come from a search of the document
    starts over ``arange(total)`` on the device: the same ids for a consistent
    ``cu_seqlens`` (0 first, ``total`` last) and no device-to-host synchronization."""
    cu = cu_seqlens.to(device=device, dtype=torch.int64)
    if total is None:
        seg = cu.diff()
        return torch.repeat_interleave(
            torch.arange(seg.numel(), device=device, dtype=torch.int32), seg).contiguous()
    pos = torch.arange(total, device=device, dtype=torch.int64)
    return torch.searchsorted(cu[1:], pos, right=True).to(torch.int32).contiguous()


def _fwd_mode(first: bool, last: bool) -> int:
    if first and last:
        return abi.FWD_WRITE
    if first:
        return abi.FWD_ACC_INIT
    if last:
        return abi.FWD_ACC_FINAL
    return abi.FWD_ACC_MERGE


_ROWS_CACHE: dict = {}


def _global_rows(layout: str, P: int, L: int, device) -> torch.Tensor:
    """Global token index of every local row of every rank, int32 [P, L], built on the
    device (zigzag: chunks r and 2P-1-r of length L/2, early first; contiguous: chunk r)
    and cached per (layout, P, L, device)."""
    key = (layout, P, L, str(device))
    rows = _ROWS_CACHE.get(key)
    if rows is None:
        r = torch.arange(P, device=device, dtype=torch.int32)[:, None]
        if layout == "zigzag":
            h = L // 2
            i = torch.arange(h, device=device, dtype=torch.int32)[None, :]
            rows = torch.cat([r * h + i, (2 * P - 1 - r) * h + i], dim=1).contiguous()
        else:
            rows = (r * L + torch.arange(L, device=device, dtype=torch.int32)[None, :]).contiguous()
        _ROWS_CACHE[key] = rows
    return rows


class _Ctx:
    """Per-call tensors shared by the forward and backward passes. ``layout`` is
    "zigzag" (rank r holds chunks r and 2P-1-r), "contiguous" (rank r holds chunk r)
    or "distflash" (contiguous chunks, DistFlash's helper / owner work placement); the
    zigzag and DistFlash rings are causal only."""

    def __init__(self, q, k, scale, doc, layout="zigzag", causal=True, window=None,
                 dropout=None, right=None):
        self.P, self.b, self.hq, self.L, self.d = q.shape
        self.hkv = k.shape[2]
        self.half = self.L // 2
        self.scale = scale
        self.doc = doc
        self.layout, self.causal = layout, causal
        self.window = None if window is None else [int(w) for w in window]
        # right: one bound per rank on the global pos_k - pos_q of its queries (non-causal)
        self.right = None if right is None else [int(w) for w in right]
        if self.right is not None:
            if len(self.right) != self.P:
                raise ValueError("the right window takes one bound per rank")
            if causal or layout != "contiguous" or doc is not None:
                raise NotImplementedError("right-bounded windows run on non-causal contiguous "
                                          "rings without document masks")
        self.dropout = dropout  # None or (p, seed): one mask over (rank's query, gathered key)
        if dropout is not None and layout == "zigzag":
            raise NotImplementedError("dropout runs on contiguous shards")
        if self.window is not None:
            if len(self.window) != self.P:
                raise ValueError("the window takes one bound per rank")
            if layout == "zigzag" and doc is None:
                raise NotImplementedError("sliding windows run on contiguous shards")
        self.gidx = self.kgidx = self.rdoc = None
        if doc is not None:
            # doc: [S] (every batch row packs the same documents) or [b, S] (each row its
            # own, ring/loop.py:178). Per rank and row: the global index of every local row
            # and its document id, [P, 1 or b, L] (the kernels step by L per batch row)
            if not causal and layout != "contiguous":
                raise NotImplementedError("non-causal document masks run on contiguous shards")
            d2 = doc if doc.dim() == 2 else doc[None]
            if d2.shape[0] not in (1, self.b):
                raise ValueError(f"per-row documents must cover {self.b} rows (got {d2.shape[0]})")
            rows32 = _global_rows(layout, self.P, self.L, q.device)
            rows = rows32.long()
            bm = d2.shape[0]
            self.rdoc = d2[:, rows].permute(1, 0, 2).to(torch.int32).contiguous()
            self.gidx = rows32[:, None, :].expand(self.P, bm, self.L).contiguous()
            self.kgidx = self.gidx
            if not causal:
                # a key's bound is the first index of its document in its row: every query
                # of the document passes k_gidx <= q_gidx (ring/loop.py:149,183-184)
                start = torch.searchsorted(d2.contiguous(), d2.contiguous(), right=False)
                self.kgidx = start[:, rows].permute(1, 0, 2).to(torch.int32).contiguous()

    def schedule(self, split_final: bool):
        if self.layout == "zigzag":
            return zigzag_schedule(self.P, self.L, split_final=split_final)
        if self.layout == "distflash":
            return distflash_schedule(self.P, self.L)
        return contiguous_schedule(self.P, self.L, causal=self.causal)

    def mask(self, step: int) -> int:
        if self.doc is not None:
            return abi.MASK_DOC
        if self.right is not None:  # every block: the causal mask, its diagonal shifted
            return abi.MASK_CAUSAL
        return abi.MASK_CAUSAL if (self.causal and step == 0) else abi.MASK_FULL

    def block_window(self, bl):
        """The kernel's window bound for block ``bl`` (None: no window). ``window[r]``
        bounds ``pos_q - pos_k`` of rank r's queries in global positions: under document
        masks the kernel compares global indices directly; otherwise its positions are
        the block's bottom-right aligned ones, which differ from the global difference
        (contiguous chunks: rank r holds positions r L .. r L + L - 1) by a constant."""
        if self.window is None:
            return None
        w = self.window[bl.rank]
        if self.doc is not None:
            return w
        sq, sk = bl.q_hi - bl.q_lo, bl.k_hi - bl.k_lo
        shift = (bl.rank * self.L + bl.q_lo) - (bl.kv_rank * self.L + bl.k_lo) - (sk - sq)
        return w - shift

    def block_right(self, bl):
        """The kernel's right bound (the causal diagonal's shift) for block ``bl``: 0 when
        the ring has no right bound. ``right[r]`` bounds ``pos_k - pos_q`` of rank r's
        queries in global positions; the block's bottom-right aligned difference differs
        from it by the same constant as in :meth:`block_window`, with the opposite sign."""
        if self.right is None:
            return 0
        sq, sk = bl.q_hi - bl.q_lo, bl.k_hi - bl.k_lo
        shift = (bl.rank * self.L + bl.q_lo) - (bl.kv_rank * self.L + bl.k_lo) - (sk - sq)
        r = self.right[bl.rank] + shift
        if r < 0:
            raise NotImplementedError(f"block ({bl.rank}, {bl.kv_rank}): right bound {r} < 0")
        return min(r, 1 << 28)

    def block_drop(self, bl):
        """Dropout coordinates of block ``bl``: the global index of its first query row and of
        its first key (contiguous chunks), so every block of a ring draws from one mask."""
        return bl.rank * self.L + bl.q_lo, bl.kv_rank * self.L + bl.k_lo

    def idx(self, rank, lo, hi):
        return None if self.gidx is None else self.gidx[rank, :, lo:hi]

    def kidx(self, rank, lo, hi):
        return None if self.kgidx is None else self.kgidx[rank, :, lo:hi]

    def docs(self, rank, lo, hi):
        return None if self.rdoc is None else self.rdoc[rank, :, lo:hi]


class KernelTimer:
    """HIP-event timing of individual kernel launches on the launching stream.

    ``with timer("attn_fwd"):`` brackets one launch; ``mean_ms(name)`` averages the
    recorded launches after a synchronize."""

    def __init__(self):
        self.events: dict[str, list] = {}

    def __call__(self, name):
        timer = self

        class _Span:
            def __enter__(self):
                self.a = torch.cuda.Event(enable_timing=True)
                self.b = torch.cuda.Event(enable_timing=True)
                self.a.record()

            def __exit__(self, *exc):
                self.b.record()
                timer.events.setdefault(name, []).append((self.a, self.b))

        return _Span()

    def mean_ms(self, name):
        spans = self.events.get(name, [])
        if not spans:
            return None
        return sum(a.elapsed_time(b) for a, b in spans) / len(spans)

    def count(self, name):
        return len(self.events.get(name, []))

    def clear(self):
        self.events.clear()


class _NoTimer:
    def __call__(self, name):
        return self

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_TIMER = _NoTimer()


def _only(blocks, only_ranks):
    """The blocks the ranks in ``only_ranks`` compute (all blocks for None)."""
    return blocks if only_ranks is None else [bl for bl in blocks if bl.runs_on in only_ranks]


def ring_forward(q, k, v, scale: float, doc: torch.Tensor | None = None, timer=None,
                 layout: str = "zigzag", causal: bool = True, only_ranks=None, window=None,
                 dropout=None, right=None):
    """Emulated ring forward (zigzag or contiguous layout). q/k/v: [P, b, H, L, d] bf16
    (interface layout per rank).
    Returns (out [P, b, L, H, d] bf16, lse [P, b, H, L] fp32, out32 [P, b, L, H, d] fp32):
    ``out32`` is the running fp32 accumulator, which the last touch of every row leaves
    holding the final merged out (the backward's delta is computed from it).
    ``only_ranks`` (a set of ranks) launches only the blocks those ranks compute (for
    DistFlash the helper computes blocks of other ranks' queries), each step at the grid
    one GPU of a real P-GPU ring runs; outputs of the blocks left out are then not
    computed (per-rank timing). ``window`` (contiguous layouts or document masks): one
    bound per rank on the global ``pos_q - pos_k`` of its queries; ``right`` (non-causal
    contiguous rings): one bound per rank on the global ``pos_k - pos_q``."""
    timer = timer or _NO_TIMER
    c = _Ctx(q, k, scale, doc, layout, causal, window, dropout, right)
    qd, kd, vd = q.transpose(2, 3), k.transpose(2, 3), v.transpose(2, 3)  # [P, b, L, H, d] views
    dev = q.device
    out = torch.empty((c.P, c.b, c.L, c.hq, c.d), dtype=q.dtype, device=dev)
    lse = torch.empty((c.P, c.b, c.hq, c.L), dtype=torch.float32, device=dev)
    acc = torch.empty((c.P, c.b, c.L, c.hq, c.d), dtype=torch.float32, device=dev)
    acc_lse = None
    if c.P > 1:
        acc_lse = torch.empty((c.P, c.b, c.hq, c.L), dtype=torch.float32, device=dev)
    for s, blocks in enumerate(c.schedule(split_final=True)):
        jobs = []
        for bl in _only(blocks, only_ranks):
            r, kr = bl.rank, bl.kv_rank
            qs, ks = slice(bl.q_lo, bl.q_hi), slice(bl.k_lo, bl.k_hi)
            jobs.append(ops.FwdJob(
                q=qd[r][:, qs], k=kd[kr][:, ks], v=vd[kr][:, ks],
                mode=_fwd_mode(bl.first, bl.last),
                out=out[r][:, qs], lse=lse[r][:, :, qs],
                acc_out=acc[r][:, qs],
                acc_lse=None if acc_lse is None else acc_lse[r][:, :, qs],
                q_gidx=c.idx(r, bl.q_lo, bl.q_hi), k_gidx=c.kidx(kr, bl.k_lo, bl.k_hi),
                q_doc=c.docs(r, bl.q_lo, bl.q_hi), k_doc=c.docs(kr, bl.k_lo, bl.k_hi),
                window=c.block_window(bl), right=c.block_right(bl),
                **dict(zip(("drop_q0", "drop_k0"), c.block_drop(bl)))))
        with timer("attn_fwd"):
            ops.attn_fwd(jobs, scale=scale, mask=c.mask(s), dropout=c.dropout)
    return out, lse, acc


def ring_backward(dout, q, k, v, out, lse, scale: float, doc: torch.Tensor | None = None,
                  timer=None, layout: str = "zigzag", causal: bool = True, only_ranks=None,
                  window=None, dropout=None, right=None):
    """Reverse-ring backward with the global out/lse. dout: [P, b, L, H, d] bf16; out: the
    global out, fp32 (the forward's ``out32``) or bf16, [P, b, L, H, d].
    Returns fp32 (dq [P, b, L, Hq, d], dk, dv [P, b, L, Hkv, d]). Each step launches the
    KV-major dK/dV kernel and the Q-major dQ kernel over all ranks (``only_ranks``: over
    those ranks only, as in :func:`ring_forward`; the gradients are then partial)."""
    timer = timer or _NO_TIMER
    c = _Ctx(q, k, scale, doc, layout, causal, window, dropout, right)
    qd, kd, vd = q.transpose(2, 3), k.transpose(2, 3), v.transpose(2, 3)
    dev = q.device
    if not dout.is_contiguous():
        dout = dout.contiguous()
    if not out.is_contiguous():
        out = out.contiguous()
    delta = torch.empty((c.P, c.b, c.hq, c.L), dtype=torch.float32, device=dev)
    nlse = torch.empty_like(delta)
    if not lse.is_contiguous():
        lse = lse.contiguous()
    flat = (c.P * c.b, c.L, c.hq, c.d)
    lflat = (c.P * c.b, c.hq, c.L)
    with timer("attn_bwd_delta"):
        ops.attn_bwd_delta(out.reshape(flat), dout.reshape(flat), delta.reshape(lflat), c.hkv,
                           lse=lse.reshape(lflat), nlse=nlse.reshape(lflat))
    dq = torch.empty((c.P, c.b, c.L, c.hq, c.d), dtype=torch.float32, device=dev)
    dk = torch.empty((c.P, c.b, c.L, c.hkv, c.d), dtype=torch.float32, device=dev)
    dv = torch.empty_like(dk)
    for s, blocks in enumerate(c.schedule(split_final=False)):
        mode = abi.GRAD_WRITE_F32 if s == 0 else abi.GRAD_ACC_F32
        kv_jobs, q_jobs = [], []
        for bl in _only(blocks, only_ranks):
            r, kr = bl.rank, bl.kv_rank
            qs, ks = slice(bl.q_lo, bl.q_hi), slice(bl.k_lo, bl.k_hi)
            common = dict(
                q=qd[r][:, qs], k=kd[kr][:, ks], v=vd[kr][:, ks], dout=dout[r][:, qs],
                lse=lse[r][:, :, qs], delta=delta[r][:, :, qs], nlse=nlse[r][:, :, qs],
                q_gidx=c.idx(r, bl.q_lo, bl.q_hi), k_gidx=c.kidx(kr, bl.k_lo, bl.k_hi),
                q_doc=c.docs(r, bl.q_lo, bl.q_hi), k_doc=c.docs(kr, bl.k_lo, bl.k_hi),
                window=c.block_window(bl), right=c.block_right(bl),
                **dict(zip(("drop_q0", "drop_k0"), c.block_drop(bl))))
            kv_jobs.append(ops.BwdJob(dq_mode=abi.GRAD_NONE, dkv_mode=mode,
                                      dk_acc=dk[kr][:, ks], dv_acc=dv[kr][:, ks], **common))
            q_jobs.append(ops.BwdJob(dq_mode=mode, dkv_mode=abi.GRAD_NONE,
                                     dq_acc=dq[r][:, qs], **common))
        with timer("attn_bwd_dkdv"):
            ops.attn_bwd(kv_jobs, scale=scale, mask=c.mask(s), dropout=c.dropout)
        with timer("attn_bwd_dq"):
            ops.attn_bwd(q_jobs, scale=scale, mask=c.mask(s), dropout=c.dropout)
    return dq, dk, dv


class EmulatedRing(torch.autograd.Function):
    """The emulated ring (zigzag or contiguous layout) with its reverse-ring backward."""

    @staticmethod
    def forward(ctx, q, k, v, scale, doc, timer, layout, causal, window=None, dropout=None,
                right=None):
        out, lse, out32 = ring_forward(q, k, v, scale, doc, timer, layout, causal, window=window,
                                       dropout=dropout, right=right)
        ctx.save_for_backward(q, k, v, out32, lse)
        ctx.scale, ctx.doc, ctx.timer = scale, doc, timer
        ctx.layout, ctx.causal, ctx.window, ctx.dropout = layout, causal, window, dropout
        ctx.right = right
        return out

    @staticmethod
    def backward(ctx, d_out):
        q, k, v, out32, lse = ctx.saved_tensors
        dq, dk, dv = ring_backward(d_out, q, k, v, out32, lse, ctx.scale, ctx.doc, ctx.timer,
                                   ctx.layout, ctx.causal, window=ctx.window, dropout=ctx.dropout,
                                   right=ctx.right)
        # fp32 accumulators -> q.dtype, returned in the interface layout [P, b, H, L, d]
        return (dq.to(q.dtype).transpose(2, 3), dk.to(k.dtype).transpose(2, 3),
                dv.to(v.dtype).transpose(2, 3), None, None, None, None, None, None, None, None)


def check_ring_inputs(q, k, v):
    """Validation shared by the emulated rings (q/k/v: [world, b, H, L, d])."""
    abi.require_device(q, k, v)
    if q.dim() != 5 or k.dim() != 5 or v.dim() != 5:
        raise ValueError("q/k/v must be [world, b, H, L, d]")
    if q.shape[2] % k.shape[2]:
        raise ValueError("Query heads must be divisible by KV heads")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("the MI355X ring computes in bf16 or fp16")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share their dtype")


def check_cu_seqlens(cu_seqlens, total: int) -> None:
    """``cu_seqlens`` starts at 0, never decreases and ends at ``total`` (ValueError)."""
    cu = cu_seqlens.detach().to("cpu", torch.int64)
    if cu.dim() != 1 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be 1-D with at least two entries")
    if int(cu[0]) != 0 or int(cu[-1]) != total:
        raise ValueError(f"cu_seqlens must run from 0 to the full (padded) sequence {total} "
                         f"(got {int(cu[0])} .. {int(cu[-1])})")
    if bool((cu.diff() < 0).any()):
        raise ValueError("cu_seqlens must not decrease")


def doc_for(cu_seqlens, q, rows: int = 1):
    """Per-token document ids of the packed sequence (None when not packed): [S] over the
    sequence S = P L that every batch row shares (the zigzag and DistFlash rings,
    ring/zigzag.py:89-90), or with ``rows`` = b, [b, S] over ``cu_seqlens`` covering the
    b S tokens of the flattened batch, row ``i`` taking tokens ``[i S, (i + 1) S)`` (the
    packed contiguous ring, ring/loop.py:178). A host ``cu_seqlens`` is checked to cover
    the sequence; a device one is read without a synchronization and must end at that
    length, which the environment variable ``RINGMASTER_AMD_DEBUG=1`` checks too (at the
    cost of a device-to-host copy)."""
    if cu_seqlens is None:
        return None
    seq = q.shape[0] * q.shape[3]
    total = rows * seq
    if cu_seqlens.device.type == "cpu" or os.environ.get("RINGMASTER_AMD_DEBUG") == "1":
        check_cu_seqlens(cu_seqlens, total)
    doc = doc_ids_from_cu(cu_seqlens, q.device, total)
    return doc.reshape(rows, seq) if rows > 1 else doc


def zigzag_ring_attention(q, k, v, *, group=None, scaling=None, cu_seqlens=None, timer=None):
    """q/k/v: [P, b, H, L, d] — rank r's zigzag-sharded interface tensors stacked on dim 0
    (L = two chunks, early then late). Returns [P, b, L, H, d]; ``cu_seqlens`` set =>
    packed (document-masked) blocks. Counterpart of ``zigzag_ring_attention(q, k, v, *,
    group, scaling, cu_seqlens)`` (ring/zigzag.py:257-260): ``group`` must be None, the
    ranks being the leading axis of one process. ``timer`` (a :class:`KernelTimer`)
    records HIP events around every kernel launch."""
    if group is not None:
        raise ValueError("the emulated ring takes the ranks on the leading axis, not a group")
    check_ring_inputs(q, k, v)
    if q.shape[3] % 2:
        raise ValueError("local length must hold two equal zigzag chunks")
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q.shape[-1])
    return EmulatedRing.apply(q, k, v, float(scale), doc_for(cu_seqlens, q), timer, "zigzag", True)
