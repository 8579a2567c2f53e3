"""CPU restatement of the reference ring-attention math (test infrastructure only).

Follows ring/kernels.py:52-78 (math_block, with its sliding window; ``flash=True``: the
flash provider's window, ring/kernels.py:37-38), ring/loop.py:175-228
(the gather ring and the packed gather ring), ring/merge.py:13-31 (merge),
ring/zigzag.py:40-67,86-120,151-254 (zigzag schedule, forward and reverse-ring
backward), ring/p2p_attn.py:243-281 (explicit global-lse block backward) and
ring/varlen_blocks.py:45-80,176-200 (document masks). The P ranks of the ring are
emulated in one process: a ring hop is an index into per-rank lists, the dK/dV
accumulators travel with their KV block exactly as the reference's
``_shift_sync`` moves them.
"""

from __future__ import annotations

import math

import numpy as np
import torch

NEG_INF = float("-inf")


# ---------------------------------------------------------------- dropout mask
# The reference drops attention probabilities with torch's RNG (ring/kernels.py:74-75),
# which no other implementation reproduces. The MI355X kernels draw a counter-based mask
# instead: element (b, h, q, k) is kept when fmix32(bhmix ^ q C_Q ^ k C_K) >= floor(p 2^32)
# (fmix32: the MurmurHash3 finalizer), with the same 1 / (1 - p) scaling of the kept
# probabilities and the undropped lse. The functions below restate that mask, so the
# dropped math of a given seed is checked exactly; its agreement with torch's dropout is
# distributional only (keep rate, unbiasedness).
DROP_Q, DROP_K, DROP_BH = 0x85EBCA77, 0xC2B2AE3D, 0x9E3779B9


def fmix32(x):
    """MurmurHash3's 32-bit finalizer on a numpy uint32 array."""
    x = np.asarray(x, dtype=np.uint32)
    with np.errstate(over="ignore"):
        x = x ^ (x >> np.uint32(16))
        x = x * np.uint32(0x85EBCA6B)
        x = x ^ (x >> np.uint32(13))
        x = x * np.uint32(0xC2B2AE35)
        x = x ^ (x >> np.uint32(16))
    return x


def drop_p32(p):
    """The dropout probability as the C ABI carries it (the layout's fp32 ``dropout_p``):
    the mask's threshold and the keep scale are those of this value (0.3 -> 0.30000001...,
    whose threshold floor(p 2^32) is 52 counts above the float64 one's)."""
    return float(np.float32(p))


def dropout_keep(seed, bh, q_pos, k_pos, p):
    """Keep mask [len(q_pos), len(k_pos)] (bool) of the (batch, head) pair bh = b Hq + h:
    fmix32(bhmix ^ q DROP_Q ^ k DROP_K) >= floor(p32 2^32) with p32 = drop_p32(p),
    bhmix = fmix32(seed_lo ^ fmix32(seed_hi ^ bh DROP_BH)), arithmetic mod 2^32."""
    seed = int(seed) & ((1 << 64) - 1)
    lo, hi = np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32)
    with np.errstate(over="ignore"):
        bhmix = fmix32(lo ^ fmix32(hi ^ (np.uint32(bh) * np.uint32(DROP_BH))))
        qt = np.asarray(q_pos, dtype=np.int64).astype(np.uint32) * np.uint32(DROP_Q)
        kt = np.asarray(k_pos, dtype=np.int64).astype(np.uint32) * np.uint32(DROP_K)
    u = fmix32(bhmix ^ qt[:, None] ^ kt[None, :])
    thr = min(int(drop_p32(p) * 4294967296.0), 0xFFFFFFFF)
    return u >= np.uint32(thr)


def dropout_scale_mask(seed, b, hq, sq, sk, p, q0=0, k0=0):
    """fp32 [b, hq, sq, sk]: 1 / (1 - p32) where kept, 0 where dropped (p32 = drop_p32(p))."""
    keep = np.stack([np.stack([dropout_keep(seed, bi * hq + h, np.arange(sq) + q0,
                                            np.arange(sk) + k0, p) for h in range(hq)])
                     for bi in range(b)])
    return torch.from_numpy(keep.astype(np.float32)) / (1.0 - drop_p32(p))


# ---------------------------------------------------------------- blocks
def flash_window(window, causal, sk):
    """The (left, right) bounds that flash attention 2 applies for ``window_size`` (the
    flash provider hands the window to ``flash_attn_func``, ring/kernels.py:37-38; the
    library is not installed here, so its published argument rules are restated): a bound
    of at least sk keys counts as -1; causal sets right to 0; then a -1 bound facing a
    non-negative one becomes sk. Returns (left, right), None for a side left unbounded."""
    lo, hi = (int(x) for x in window)
    lo = -1 if lo >= sk else lo
    hi = -1 if hi >= sk else hi
    if causal:
        hi = 0
    if lo < 0 <= hi:
        lo = sk
    if hi < 0 <= lo:
        hi = sk
    return (lo if lo >= 0 else None), (hi if hi >= 0 else None)


def math_block(q, k, v, *, causal, scaling, dropout=0.0, window=None, drop_seed=None,
               drop_q0=0, drop_k0=0, flash=False):
    """Explicit-softmax block (ring/kernels.py:52-78). q/k/v [b, s, h, d] -> (out, lse).
    With ``dropout`` and ``drop_seed`` the probabilities are dropped by the hash mask of
    that seed (coordinates offset by drop_q0 / drop_k0) instead of torch's RNG. ``flash``:
    the window is the flash provider's (``flash_window``: pos_q - pos_k > left and
    pos_k - pos_q > right masked) instead of math_block's left bound."""
    qt, kt, vt = (t.transpose(1, 2).float() for t in (q, k, v))
    if qt.shape[1] != kt.shape[1]:
        if qt.shape[1] % kt.shape[1]:
            raise ValueError("Query heads must be divisible by KV heads")
        rep = qt.shape[1] // kt.shape[1]
        kt, vt = (t.repeat_interleave(rep, dim=1) for t in (kt, vt))
    scale = scaling if scaling is not None else 1.0 / math.sqrt(qt.shape[-1])
    scores = (qt @ kt.transpose(-1, -2)) * scale
    sq, sk = scores.shape[-2], scores.shape[-1]
    if causal:
        keep = torch.ones(sq, sk, dtype=torch.bool).tril(sk - sq)
        scores = scores.masked_fill(~keep, NEG_INF)
    if window is not None:
        iq = torch.arange(sq).unsqueeze(1) + (sk - sq)
        ik = torch.arange(sk).unsqueeze(0)
        if flash:
            left, right = flash_window(window, causal, sk)
            if left is not None:
                scores = scores.masked_fill(iq - ik > left, NEG_INF)
            if right is not None:
                scores = scores.masked_fill(ik - iq > right, NEG_INF)
        else:
            scores = scores.masked_fill(iq - ik > window[0], NEG_INF)
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.exp(scores - lse.unsqueeze(-1))
    if dropout and drop_seed is not None:
        b, hq = probs.shape[0], probs.shape[1]
        probs = probs * dropout_scale_mask(drop_seed, b, hq, sq, sk, dropout, drop_q0, drop_k0)
    elif dropout:
        probs = torch.nn.functional.dropout(probs, p=dropout)
    out = probs @ vt
    return out.transpose(1, 2).to(q.dtype), lse


def _repeat_kv(t, n_heads):
    """[b, s, Hkv, d] -> [b, s, Hq, d] (ring/varlen_blocks.py:61-66)."""
    if t.shape[2] == n_heads:
        return t
    return t.repeat_interleave(n_heads // t.shape[2], dim=2)


def doc_ids_from_cu(cu_seqlens):
    """Per-token document id (ring/varlen_blocks.py:45-48)."""
    seg = cu_seqlens.to(torch.int64).diff()
    return torch.repeat_interleave(torch.arange(seg.numel()), seg)


def additive_doc_mask(q_gidx, k_gidx, doc_ids, causal: bool):
    """0 where same document (and k <= q if causal), else -inf (ring/varlen_blocks.py:51-58)."""
    allow = doc_ids[q_gidx].unsqueeze(1) == doc_ids[k_gidx].unsqueeze(0)
    if causal:
        allow = allow & (k_gidx.unsqueeze(0) <= q_gidx.unsqueeze(1))
    return torch.where(allow, torch.zeros(()), torch.full((), NEG_INF))


def masked_block_fwd(q, k, v, add_mask, scale):
    """(out, lse) with an additive mask; lse -inf for rows with no key (ring/varlen_blocks.py:69-80)."""
    qf = q.transpose(1, 2).float()
    kf = _repeat_kv(k, q.shape[2]).transpose(1, 2).float()
    vf = _repeat_kv(v, q.shape[2]).transpose(1, 2).float()
    scores = (qf @ kf.transpose(-1, -2)) * scale + add_mask
    lse = torch.logsumexp(scores, dim=-1)
    safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
    p = torch.exp(scores - safe.unsqueeze(-1))
    out = p @ vf
    return out.transpose(1, 2).to(q.dtype), lse


def masked_block_bwd(d_out, q, k, v, out, lse, add_mask, scale):
    """dq, dk, dv of one block from the GLOBAL out/lse, GQA folded
    (ring/varlen_blocks.py:176-200, identity of ring/p2p_attn.py:243-281)."""
    nq = q.shape[2]
    qf = q.transpose(1, 2).float()
    kf = _repeat_kv(k, nq).transpose(1, 2).float()
    vf = _repeat_kv(v, nq).transpose(1, 2).float()
    dof = d_out.transpose(1, 2).float()
    of = out.transpose(1, 2).float()
    scores = (qf @ kf.transpose(-1, -2)) * scale + add_mask
    p = torch.exp(scores - lse.unsqueeze(-1))
    delta = (dof * of).sum(-1, keepdim=True)
    dv = p.transpose(-1, -2) @ dof
    dp = dof @ vf.transpose(-1, -2)
    ds = p * (dp - delta)
    dq = (ds @ kf) * scale
    dk = (ds.transpose(-1, -2) @ qf) * scale
    hkv = k.shape[2]
    if hkv != nq:
        dk = dk.unflatten(1, (hkv, nq // hkv)).sum(2)
        dv = dv.unflatten(1, (hkv, nq // hkv)).sum(2)
    return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2)


def causal_mask(sq, sk):
    """Additive bottom-right causal mask (ring/kernels.py:64-67)."""
    keep = torch.ones(sq, sk, dtype=torch.bool).tril(sk - sq)
    return torch.where(keep, torch.zeros(()), torch.full((), NEG_INF))


# ---------------------------------------------------------------- merge
def lse_to_bshd(block_lse, like):
    """[b, h, s] -> [b, s, h, 1] fp32 (ring/merge.py:13-17)."""
    if block_lse.dim() == 3 and block_lse.shape[1] == like.shape[2]:
        block_lse = block_lse.transpose(1, 2)
    return block_lse.unsqueeze(-1).contiguous().to(torch.float32)


def update_out_and_lse(out, lse, block_out, block_lse):
    """Online-softmax merge (ring/merge.py:20-31)."""
    block_lse = lse_to_bshd(block_lse, block_out)
    block_out = block_out.to(torch.float32)
    if out is None:
        return block_out, block_lse
    new_lse = torch.logaddexp(lse, block_lse)
    out = torch.exp(lse - new_lse) * out + torch.exp(block_lse - new_lse) * block_out
    return out, new_lse


def merge_slice(out, lse, block_out, block_lse, sl):
    """In-place merge of a partial block into rows ``sl`` (ring/zigzag.py:59-67)."""
    blk_lse = lse_to_bshd(block_lse, block_out)
    blk_out = block_out.to(torch.float32)
    o, lo = out[:, sl], lse[:, sl]
    new = torch.logaddexp(lo, blk_lse)
    out[:, sl] = torch.exp(lo - new) * o + torch.exp(blk_lse - new) * blk_out
    lse[:, sl] = new
    return out, lse


# ---------------------------------------------------------------- zigzag ring
def zigzag_gidx(rank, half, world):
    """Global token indices of rank's two chunks, early then late (ring/zigzag.py:40-46)."""
    return torch.cat([torch.arange(rank * half, (rank + 1) * half),
                      torch.arange((2 * world - 1 - rank) * half, (2 * world - rank) * half)])


def kv_source(rank, step, world):
    """Rank whose KV block ``rank`` holds at ring step ``step``: the KV moves to
    rank + 1 each hop, so step s sees rank - s (ring/zigzag.py:93,
    direction ring/p2p_attn.py:65-69)."""
    return (rank - step) % world


def _block_fwd(qd, k, v, scale, mask):
    return masked_block_fwd(qd, k, v, mask, scale)


def zigzag_ring_forward(qs, ks, vs, scaling=None, cu_seqlens=None, ranks=None):
    """Emulated zigzag ring forward (ring/zigzag.py:70-149).

    qs/ks/vs: per-rank lists of interface tensors [b, H, L, d]. Returns per-rank
    out [b, L, H, d] (in q.dtype) and lse [b, H, L] fp32. Dense inputs use the
    three step cases (causal local block, early KV half, late Q half); packed
    inputs use global-index document masks for every block (:86-120). ``ranks``
    restricts the computation to those ranks' queries (others are None)."""
    world = len(qs)
    d = qs[0].shape[-1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(d)
    qd = [q.transpose(1, 2).float() for q in qs]
    kd = [k.transpose(1, 2).float() for k in ks]
    vd = [v.transpose(1, 2).float() for v in vs]
    L = qd[0].shape[1]
    half = L // 2
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    outs, lses = [None] * world, [None] * world
    for rank in (range(world) if ranks is None else ranks):
        g = zigzag_gidx(rank, half, world)
        out = lse = None
        for s in range(world):
            rem = kv_source(rank, s, world)
            ck, cv = kd[rem], vd[rem]
            if s == 0:
                m = (additive_doc_mask(g, g, doc, True) if doc is not None
                     else causal_mask(L, L))
                bo, bl = _block_fwd(qd[rank], ck, cv, scale, m)
                out, lse = update_out_and_lse(out, lse, bo, bl)
            elif s <= rank:
                kg = torch.arange(rem * half, (rem + 1) * half)
                m = additive_doc_mask(g, kg, doc, True) if doc is not None else 0.0
                bo, bl = _block_fwd(qd[rank], ck[:, :half], cv[:, :half], scale, m)
                out, lse = update_out_and_lse(out, lse, bo, bl)
            else:
                m = (additive_doc_mask(g[half:], zigzag_gidx(rem, half, world), doc, True)
                     if doc is not None else 0.0)
                bo, bl = _block_fwd(qd[rank][:, half:], ck, cv, scale, m)
                out, lse = merge_slice(out, lse, bo, bl, slice(half, None))
        outs[rank] = out.to(qs[0].dtype)
        lses[rank] = lse.squeeze(-1).transpose(1, 2).contiguous()
    return outs, lses


def zigzag_ring_backward(d_outs, qs, ks, vs, outs, lses, scaling=None, cu_seqlens=None,
                         ranks=None):
    """Emulated reverse-ring backward with the global out/lse (ring/zigzag.py:151-254).

    d_outs/outs: per-rank [b, L, H, d]; lses [b, H, L]. The dK/dV accumulator that
    leaves rank r after each step is the one rank r+1 continues (the
    ``_shift_sync`` hop, ring/zigzag.py:199-200), so block ``rem`` gathers its
    gradient from every rank that visits it. Returns per-rank (dq, dk, dv) in the
    interface layout [b, H, L, d], fp32. ``ranks`` restricts the work to those
    ranks' queries (their dq, and only their share of every dK/dV)."""
    world = len(qs)
    d = qs[0].shape[-1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(d)
    qd = [q.transpose(1, 2).float() for q in qs]
    kd = [k.transpose(1, 2).float() for k in ks]
    vd = [v.transpose(1, 2).float() for v in vs]
    L = qd[0].shape[1]
    half = L // 2
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    dq = [torch.zeros_like(q) for q in qd]
    # cur_dk[r]: the accumulator rank r holds at the current step (travels with KV)
    cur_dk = [torch.zeros_like(k) for k in kd]
    cur_dv = [torch.zeros_like(v) for v in vd]
    active = range(world) if ranks is None else ranks
    for s in range(world):
        for rank in active:
            rem = kv_source(rank, s, world)
            g = zigzag_gidx(rank, half, world)
            dod, out, lse = d_outs[rank].float(), outs[rank].float(), lses[rank]
            ck, cv = kd[rem], vd[rem]
            if s == 0:
                m = additive_doc_mask(g, g, doc, True) if doc is not None else causal_mask(L, L)
                dqb, dkb, dvb = masked_block_bwd(dod, qd[rank], ck, cv, out, lse, m, scale)
                dq[rank] += dqb
                cur_dk[rank] += dkb
                cur_dv[rank] += dvb
            elif s <= rank:
                kg = torch.arange(rem * half, (rem + 1) * half)
                m = additive_doc_mask(g, kg, doc, True) if doc is not None else 0.0
                dqb, dk0, dv0 = masked_block_bwd(dod, qd[rank], ck[:, :half], cv[:, :half],
                                                 out, lse, m, scale)
                dq[rank] += dqb
                cur_dk[rank][:, :half] += dk0
                cur_dv[rank][:, :half] += dv0
            else:
                m = (additive_doc_mask(g[half:], zigzag_gidx(rem, half, world), doc, True)
                     if doc is not None else 0.0)
                dq1, dkb, dvb = masked_block_bwd(dod[:, half:], qd[rank][:, half:], ck, cv,
                                                 out[:, half:], lse[:, :, half:], m, scale)
                dq[rank][:, half:] += dq1
                cur_dk[rank] += dkb
                cur_dv[rank] += dvb
        # _shift_sync: rank r+1 receives what rank r held
        cur_dk = [cur_dk[(r - 1) % world] for r in range(world)]
        cur_dv = [cur_dv[(r - 1) % world] for r in range(world)]
    # after P hops every accumulator is back at its owner
    return ([t.transpose(1, 2) for t in dq], [t.transpose(1, 2) for t in cur_dk],
            [t.transpose(1, 2) for t in cur_dv])


# ---------------------------------------------------------------- contiguous rings
def contiguous_gidx(rank, local_len):
    """Global token indices of rank's contiguous chunk."""
    return torch.arange(rank * local_len, (rank + 1) * local_len)


def _contig_mask(rank, rem, L, step, causal, doc):
    """Mask of rank's block against rank rem's KV: document-masked on global indices for
    packed inputs (ring/varlen_blocks.py:51-58), else bottom-right causal on the step-0
    diagonal of a causal ring (ring/p2p_attn.py:168, :112-118) and nothing elsewhere."""
    if doc is not None:
        return additive_doc_mask(contiguous_gidx(rank, L), contiguous_gidx(rem, L), doc, causal)
    return causal_mask(L, L) if (causal and step == 0) else 0.0


def _prep(qs, ks, vs, scaling):
    d = qs[0].shape[-1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(d)
    return ([q.transpose(1, 2).float() for q in qs], [k.transpose(1, 2).float() for k in ks],
            [v.transpose(1, 2).float() for v in vs], scale)


def contiguous_ring_forward(qs, ks, vs, *, causal=True, scaling=None, cu_seqlens=None):
    """Contiguous p2p ring forward, the explicit path of RingP2PAttention.forward
    (ring/p2p_attn.py:161-185): rank r merges, in step order, its block against the KV
    rank (r - s) mod P holds at step s (kv_source), skipping s > r when causal; only
    the step-0 block is causal. qs/ks/vs: per-rank [b, H, L, d]; returns per-rank out
    [b, L, H, d] (q dtype) and lse [b, H, L] fp32."""
    world = len(qs)
    qd, kd, vd, scale = _prep(qs, ks, vs, scaling)
    L = qd[0].shape[1]
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    outs, lses = [], []
    for rank in range(world):
        out = lse = None
        for s in range(world):
            if causal and s > rank:
                continue
            rem = kv_source(rank, s, world)
            bo, bl = _block_fwd(qd[rank], kd[rem], vd[rem], scale,
                                _contig_mask(rank, rem, L, s, causal, doc))
            out, lse = update_out_and_lse(out, lse, bo, bl)
        outs.append(out.to(qs[0].dtype))
        lses.append(lse.squeeze(-1).transpose(1, 2).contiguous())
    return outs, lses


def contiguous_ring_backward(d_outs, qs, ks, vs, outs, lses, *, causal=True, scaling=None,
                             cu_seqlens=None):
    """Reverse contiguous ring with the global out/lse (ring/p2p_attn.py:243-281): after
    every step the dK/dV accumulator a rank holds moves on with its KV block (:266-275),
    so after P hops each block's gradient is back at its owner. d_outs/outs: per-rank
    [b, L, H, d]; returns per-rank (dq, dk, dv) [b, H, L, d] fp32."""
    world = len(qs)
    qd, kd, vd, scale = _prep(qs, ks, vs, scaling)
    L = qd[0].shape[1]
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    dq = [torch.zeros_like(q) for q in qd]
    cur_dk = [torch.zeros_like(k) for k in kd]
    cur_dv = [torch.zeros_like(v) for v in vd]
    for s in range(world):
        for rank in range(world):
            if causal and s > rank:
                continue
            rem = kv_source(rank, s, world)
            dqb, dkb, dvb = masked_block_bwd(d_outs[rank].float(), qd[rank], kd[rem], vd[rem],
                                             outs[rank].float(), lses[rank],
                                             _contig_mask(rank, rem, L, s, causal, doc), scale)
            dq[rank] += dqb
            cur_dk[rank] += dkb
            cur_dv[rank] += dvb
        cur_dk = [cur_dk[(r - 1) % world] for r in range(world)]
        cur_dv = [cur_dv[(r - 1) % world] for r in range(world)]
    return ([t.transpose(1, 2) for t in dq], [t.transpose(1, 2) for t in cur_dk],
            [t.transpose(1, 2) for t in cur_dv])


def distflash_forward(qs, ks, vs, *, scaling=None, cu_seqlens=None):
    """DistFlashAttention.forward (ring/distflash.py:98-152), in its merge order: the
    causal diagonal; the owner-local blocks (r, r - d) for d > P // 2 in increasing d
    (phase 2, :125-131); then the partials of the blocks (r, r - d), d = 1 .. P // 2,
    that helper r - d computed and routed back (phase 1, :133-142)."""
    world = len(qs)
    qd, kd, vd, scale = _prep(qs, ks, vs, scaling)
    L = qd[0].shape[1]
    half = world // 2
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    outs, lses = [], []
    for r in range(world):
        out, lse = update_out_and_lse(None, None, *_block_fwd(
            qd[r], kd[r], vd[r], scale, _contig_mask(r, r, L, 0, True, doc)))
        order = [d for d in range(half + 1, world)] + [d for d in range(1, half + 1)]
        for d in order:
            if r - d < 0:
                continue
            bo, bl = _block_fwd(qd[r], kd[r - d], vd[r - d], scale,
                                _contig_mask(r, r - d, L, d, True, doc))
            out, lse = update_out_and_lse(out, lse, bo, bl)
        outs.append(out.to(qs[0].dtype))
        lses.append(lse.squeeze(-1).transpose(1, 2).contiguous())
    return outs, lses


def distflash_backward(d_outs, qs, ks, vs, outs, lses, *, scaling=None, cu_seqlens=None):
    """DistFlashAttention.backward (ring/distflash.py:154-226): the diagonal seeds dq,
    dk, dv; phase 2 (d > P // 2): the owner r computes (r, r - d), keeps dq and sends the
    dK/dV with the KV back to owner r - d; phase 1 (d <= P // 2): helper r - d computes
    the block from the owner's (dout, q, out, lse), keeps dK/dV and returns dq."""
    world = len(qs)
    qd, kd, vd, scale = _prep(qs, ks, vs, scaling)
    L = qd[0].shape[1]
    half = world // 2
    doc = doc_ids_from_cu(cu_seqlens) if cu_seqlens is not None else None
    dq = [torch.zeros_like(q) for q in qd]
    dk = [torch.zeros_like(k) for k in kd]
    dv = [torch.zeros_like(v) for v in vd]

    def block(i, j, d):
        return masked_block_bwd(d_outs[i].float(), qd[i], kd[j], vd[j], outs[i].float(),
                                lses[i], _contig_mask(i, j, L, d, True, doc), scale)

    for r in range(world):
        a, b_, c = block(r, r, 0)
        dq[r] += a
        dk[r] += b_
        dv[r] += c
    for d in range(half + 1, world):  # phase 2: owner r, KV owner r - d
        for r in range(d, world):
            a, b_, c = block(r, r - d, d)
            dq[r] += a
            dk[r - d] += b_
            dv[r - d] += c
    for d in range(1, half + 1):  # phase 1: helper h computes for owner h + d
        for h in range(world - d):
            a, b_, c = block(h + d, h, d)
            dk[h] += b_
            dv[h] += c
            dq[h + d] += a
    return ([t.transpose(1, 2) for t in dq], [t.transpose(1, 2) for t in dk],
            [t.transpose(1, 2) for t in dv])


def allgather_ring_forward(qs, ks, vs, *, causal=True, scaling=None, window=None, dropout=0.0,
                           drop_seed=None, flash=False):
    """The gather ring (ring/loop.py:201-228): rank r attends the gathered K/V of ranks
    0..r (causal) or of every rank with ONE math_block call, whose bottom-right
    alignment places rank r's query i at position ``(end - 1) L + i`` against the
    gathered keys (``end`` = r + 1 causal, P otherwise); a window bounds that position
    minus the key's global index (``flash``: the flash provider's window, bounded on both
    sides). With dropout and ``drop_seed``: the hash mask over
    (global query r L + i, gathered key). qs/ks/vs per-rank [b, H, L, d] -> per-rank out
    [b, L, H, d] and lse [b, H, L]. Differentiable (torch autograd)."""
    world = len(qs)
    outs, lses = [], []
    for r in range(world):
        end = r + 1 if causal else world
        q = qs[r].transpose(1, 2)
        k = torch.cat([t.transpose(1, 2) for t in ks[:end]], dim=1)
        v = torch.cat([t.transpose(1, 2) for t in vs[:end]], dim=1)
        L = q.shape[1]
        o, lse = math_block(q, k, v, causal=causal, scaling=scaling, window=window,
                            dropout=dropout, drop_seed=drop_seed, drop_q0=r * L, flash=flash)
        outs.append(o)
        lses.append(lse)
    return outs, lses


def varlen_ring_forward(qs, ks, vs, cu_seqlens, *, scaling=None, causal=True, window=None,
                        dropout=0.0, drop_seed=None):
    """The packed gather ring's explicit path (ring/loop.py:103-198, the math branch
    :178-198). ``cu_seqlens`` covers the b S tokens of the flattened batch and is reshaped
    to one document list per batch row (:178). Rank r's query at global index ``r L + i``
    of row ``row`` attends gathered key j of the same row when both lie in one document
    (:182), ``j <= r L + i`` when ``causal`` (:183-184) and ``r L + i - j <= window[0]``
    when a window is given (:185-186). With ``dropout`` and ``drop_seed`` the kept
    probabilities follow the hash mask of that seed over (row, head, r L + i, j) instead of
    SDPA's RNG (:189-197). Per-rank [b, H, L, d] -> per-rank out [b, L, H, d] and lse
    [b, H, L]. Differentiable (torch autograd)."""
    world, b, L = len(qs), qs[0].shape[0], qs[0].shape[2]
    S = world * L
    doc = doc_ids_from_cu(cu_seqlens).reshape(b, S)
    k = torch.cat([t.transpose(1, 2) for t in ks], dim=1)
    v = torch.cat([t.transpose(1, 2) for t in vs], dim=1)
    kidx = torch.arange(S)
    scale = scaling if scaling is not None else 1.0 / math.sqrt(qs[0].shape[-1])
    outs, lses = [], []
    for r in range(world):
        qidx = torch.arange(r * L, r * L + L)
        allow = doc[:, qidx, None] == doc[:, None, :]  # [b, L, S]
        if causal:
            allow &= (kidx[None, :] <= qidx[:, None])[None]
        if window is not None:
            allow &= (qidx[:, None] - kidx[None, :] <= window[0])[None]
        m = torch.where(allow, torch.zeros(()), torch.full((), NEG_INF))[:, None]
        q = qs[r].transpose(1, 2)
        hq = q.shape[2]
        qf = q.transpose(1, 2).float()
        kf = _repeat_kv(k, hq).transpose(1, 2).float()
        vf = _repeat_kv(v, hq).transpose(1, 2).float()
        scores = (qf @ kf.transpose(-1, -2)) * scale + m
        lse = torch.logsumexp(scores, dim=-1)
        safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
        p = torch.exp(scores - safe.unsqueeze(-1))
        if dropout and drop_seed is not None:
            p = p * dropout_scale_mask(drop_seed, b, hq, L, S, dropout, q0=r * L, k0=0)
        elif dropout:
            p = torch.nn.functional.dropout(p, p=dropout)
        outs.append((p @ vf).transpose(1, 2).to(q.dtype))
        lses.append(lse)
    return outs, lses


def full_attention(q, k, v, *, causal=True, scaling=None, cu_seqlens=None):
    """Brute-force attention over the whole sequence in the caller's dtype (use
    fp64 to pin). q/k/v [b, S, H, d] -> out [b, S, H, d], lse [b, H, S]."""
    S = q.shape[1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q.shape[-1])
    g = torch.arange(S)
    if cu_seqlens is not None:
        m = additive_doc_mask(g, g, doc_ids_from_cu(cu_seqlens), causal).to(q.dtype)
    elif causal:
        m = causal_mask(S, S).to(q.dtype)
    else:
        m = torch.zeros(S, S, dtype=q.dtype)
    qf, kf, vf = q.transpose(1, 2), _repeat_kv(k, q.shape[2]).transpose(1, 2), \
        _repeat_kv(v, q.shape[2]).transpose(1, 2)
    scores = (qf @ kf.transpose(-1, -2)) * scale + m
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.softmax(scores, dim=-1) @ vf
    return out.transpose(1, 2), lse


def attention_rows(q_rows, k, v, q_pos, *, scaling=None, causal=True):
    """Exact attention for selected query rows against the full K/V (fp64-capable spot
    check at sizes where full attention is too large). q_rows [b, n, H, d], q_pos [n]
    global positions, k/v [b, S, Hkv, d]. Returns out [b, n, H, d], lse [b, H, n]."""
    S = k.shape[1]
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q_rows.shape[-1])
    kf = _repeat_kv(k, q_rows.shape[2]).transpose(1, 2)
    vf = _repeat_kv(v, q_rows.shape[2]).transpose(1, 2)
    qf = q_rows.transpose(1, 2)
    scores = (qf @ kf.transpose(-1, -2)) * scale
    if causal:
        allow = torch.arange(S).unsqueeze(0) <= q_pos.unsqueeze(1)
        scores = scores.masked_fill(~allow, NEG_INF)
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.softmax(scores, dim=-1) @ vf
    return out.transpose(1, 2), lse
