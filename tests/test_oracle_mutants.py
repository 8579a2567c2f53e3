"""Plant plausible mistakes in (copies of) the CPU oracle and check that the pinning
checks of test_oracle_pinning.py reject every one of them. A pinning check that a
mutant passes would pin nothing; these tests keep the checks honest. All on the CPU."""

import math

import pytest
import torch

from oracle import ring_math as rm
from oracle import state_passing as sp
from tests import test_oracle_pinning as pin


def _math_block_variant(q, k, v, *, causal, scaling, top_left=False, tile_gqa=False,
                        scale_mult=1.0):
    qt, kt, vt = (t.transpose(1, 2).double() for t in (q, k, v))
    rep = qt.shape[1] // kt.shape[1]
    if rep > 1:
        if tile_gqa:  # kv_head = q_head % hkv instead of q_head // (hq / hkv)
            kt, vt = kt.repeat(1, rep, 1, 1), vt.repeat(1, rep, 1, 1)
        else:
            kt, vt = (t.repeat_interleave(rep, dim=1) for t in (kt, vt))
    scale = (scaling if scaling is not None else 1.0 / math.sqrt(qt.shape[-1])) * scale_mult
    s = (qt @ kt.transpose(-1, -2)) * scale
    sq, sk = s.shape[-2:]
    if causal:
        keep = torch.ones(sq, sk, dtype=torch.bool).tril(0 if top_left else sk - sq)
        s = s.masked_fill(~keep, float("-inf"))
    lse = torch.logsumexp(s, -1)
    out = torch.softmax(s, -1) @ vt
    return out.transpose(1, 2), lse


@pytest.mark.parametrize("mutation", ["top_left_causal", "tiled_gqa", "scale"])
def test_block_mutants_are_caught(mutation):
    kw = {"top_left_causal": dict(top_left=True), "tiled_gqa": dict(tile_gqa=True),
          "scale": dict(scale_mult=1.01)}[mutation]
    fn = lambda q, k, v, causal, scaling: _math_block_variant(  # noqa: E731
        q, k, v, causal=causal, scaling=scaling, **kw)
    # the unmutated variant passes the same check
    pin.check_block(lambda q, k, v, causal, scaling: _math_block_variant(
        q, k, v, causal=causal, scaling=scaling), True, 4, 2, 3, 7)
    with pytest.raises(AssertionError):
        pin.check_block(fn, True, 4, 2, 3, 7)


def _window_block_variant(q, k, v, *, causal, scaling, window, inclusive=False,
                          top_left=False):
    qt, kt, vt = (t.transpose(1, 2).double() for t in (q, k, v))
    rep = qt.shape[1] // kt.shape[1]
    kt, vt = (t.repeat_interleave(rep, dim=1) for t in (kt, vt))
    s = (qt @ kt.transpose(-1, -2)) * (scaling if scaling is not None else 1 / math.sqrt(8))
    sq, sk = s.shape[-2:]
    if causal:
        s = s.masked_fill(~torch.ones(sq, sk, dtype=torch.bool).tril(sk - sq), float("-inf"))
    iq = torch.arange(sq)[:, None] + (0 if top_left else sk - sq)
    ik = torch.arange(sk)[None, :]
    far = iq - ik >= window[0] if inclusive else iq - ik > window[0]
    s = s.masked_fill(far, float("-inf"))
    return (torch.softmax(s, -1) @ vt).transpose(1, 2), torch.logsumexp(s, -1)


@pytest.mark.parametrize("mutation", ["inclusive_bound", "top_left_window"])
def test_window_mutants_are_caught(mutation):
    kw = {"inclusive_bound": dict(inclusive=True), "top_left_window": dict(top_left=True)}[mutation]
    pin.check_window_block(_window_block_variant, True, 4, 9, 1)
    with pytest.raises(AssertionError):
        pin.check_window_block(lambda *a, **k: _window_block_variant(*a, **k, **kw), True, 4, 9, 1)


def test_dropout_unscaled_mutant_is_caught():
    """Dropping without the 1 / (1 - p) rescale biases the output low."""
    def unscaled(q, k, v, *, causal, scaling, dropout, drop_seed):
        qt, kt, vt = (t.transpose(1, 2).double() for t in (q, k, v))
        s = (qt @ kt.transpose(-1, -2)) * (1 / math.sqrt(qt.shape[-1]))
        sq, sk = s.shape[-2:]
        if causal:
            s = s.masked_fill(~torch.ones(sq, sk, dtype=torch.bool).tril(sk - sq), float("-inf"))
        lse = torch.logsumexp(s, -1)
        pm = torch.exp(s - lse[..., None])
        pm = pm * rm.dropout_scale_mask(drop_seed, s.shape[0], s.shape[1], sq, sk, dropout).double() \
            * (1 - dropout)
        return (pm @ vt).transpose(1, 2), lse

    with pytest.raises(AssertionError):
        pin.check_dropout_unbiased(unscaled)


def test_merge_mutants_are_caught():
    def flipped(out, lse, block_out, block_lse):  # exp(new - blk) instead of exp(blk - new)
        block_lse = rm.lse_to_bshd(block_lse, block_out)
        if out is None:
            return block_out.float(), block_lse
        new = torch.logaddexp(lse, block_lse)
        return torch.exp(lse - new) * out + torch.exp(new - block_lse) * block_out, new

    def no_renorm(out, lse, block_out, block_lse):  # drops the running-out weight
        block_lse = rm.lse_to_bshd(block_lse, block_out)
        if out is None:
            return block_out.float(), block_lse
        new = torch.logaddexp(lse, block_lse)
        return out + torch.exp(block_lse - new) * block_out, new

    for mutant in (flipped, no_renorm):
        with pytest.raises(AssertionError):
            pin.check_merge(mutant)


def test_ring_direction_mutant_is_caught(monkeypatch):
    monkeypatch.setattr(rm, "kv_source", lambda rank, step, world: (rank + step) % world)
    with pytest.raises(AssertionError):
        pin.check_ring(4, half=2)


def test_ring_merge_slice_mutant_is_caught(monkeypatch):
    orig = rm.merge_slice

    def wrong_rows(out, lse, block_out, block_lse, sl):  # merges into the early rows
        return orig(out, lse, block_out, block_lse, slice(0, block_out.shape[1]))

    monkeypatch.setattr(rm, "merge_slice", wrong_rows)
    with pytest.raises(AssertionError):
        pin.check_ring(2, half=3)


def test_ring_backward_delta_mutant_is_caught(monkeypatch):
    def no_delta(d_out, q, k, v, out, lse, add_mask, scale):  # dS = P dP (delta dropped)
        nq = q.shape[2]
        qf, kf, vf = (rm._repeat_kv(t, nq).transpose(1, 2).double() for t in (q, k, v))
        dof = d_out.transpose(1, 2).double()
        p = torch.exp((qf @ kf.transpose(-1, -2)) * scale + add_mask - lse.unsqueeze(-1))
        dv = p.transpose(-1, -2) @ dof
        ds = p * (dof @ vf.transpose(-1, -2))
        dq, dk = (ds @ kf) * scale, (ds.transpose(-1, -2) @ qf) * scale
        hkv = k.shape[2]
        if hkv != nq:
            dk = dk.unflatten(1, (hkv, nq // hkv)).sum(2)
            dv = dv.unflatten(1, (hkv, nq // hkv)).sum(2)
        return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2)

    monkeypatch.setattr(rm, "masked_block_bwd", no_delta)
    with pytest.raises(AssertionError):
        pin.check_ring(2, half=3)


def test_zigzag_gidx_mutant_is_caught(monkeypatch):
    # late chunk first: the document masks then use the wrong global indices
    monkeypatch.setattr(rm, "zigzag_gidx", lambda r, h, w: torch.cat(
        [torch.arange((2 * w - 1 - r) * h, (2 * w - r) * h), torch.arange(r * h, (r + 1) * h)]))
    cu = torch.tensor([0, 6, 16], dtype=torch.int32)
    with pytest.raises(AssertionError):
        pin.check_ring(2, half=4, cu=cu)


def test_scan_mutants_are_caught():
    def no_correction(a, b, world):
        n = a.shape[1] // world
        return torch.cat([sp.local_linear_scan(a[:, r * n:(r + 1) * n], b[:, r * n:(r + 1) * n])
                          for r in range(world)], 1)

    def reversed_prefix(a, b, world):  # folds the ranks' pairs in the wrong order
        n = a.shape[1] // world
        outs, pairs = [], []
        for r in range(world):
            sa, sb = a[:, r * n:(r + 1) * n], b[:, r * n:(r + 1) * n]
            h = sp.local_linear_scan(sa, sb)
            pairs.append((torch.cumprod(sa, 1), h))
        for r in range(world):
            h_in = torch.zeros_like(b[:, 0])
            for j in reversed(range(r)):
                h_in = pairs[j][0][:, -1] * h_in + pairs[j][1][:, -1]
            outs.append(pairs[r][1] + pairs[r][0] * h_in.unsqueeze(1))
        return torch.cat(outs, 1)

    for mutant in (no_correction, reversed_prefix):
        with pytest.raises(AssertionError):
            pin.check_scan(mutant, world=4, T=16)


def test_correction_seq_idx_mutant_is_caught(monkeypatch):
    """A correction that ignores seq_idx (adds the carried state to a packed sequence
    that starts fresh on the rank) fails the packed-sequence pinning check."""
    real = sp.mamba2_cp_correction

    def ignore_seq_idx(out, h_final, C, cum_A, h_prev, num_heads, head_dim, seq_idx=None):
        return real(out, h_final, C, cum_A, h_prev, num_heads, head_dim, seq_idx=None)

    monkeypatch.setattr(sp, "mamba2_cp_correction", ignore_seq_idx)
    with pytest.raises(AssertionError):
        pin.test_mamba2_correction_packed_sequences(11)


@pytest.mark.parametrize("mutation", ["direction", "skip_past"])
def test_contiguous_ring_mutants_are_caught(monkeypatch, mutation):
    pin.check_contiguous(4, 3)  # the unmutated oracle passes
    if mutation == "direction":  # KV hops the other way round the ring
        monkeypatch.setattr(rm, "kv_source", lambda rank, step, world: (rank + step) % world)
    else:  # attends the block of step s > r instead of skipping it: future tokens leak in
        real = rm.contiguous_ring_forward

        def leaky(qs, ks, vs, *, causal=True, **kw):
            return real(qs, ks, vs, causal=False, **kw)
        monkeypatch.setattr(rm, "contiguous_ring_forward", leaky)
    with pytest.raises(AssertionError):
        pin.check_contiguous(4, 3)


@pytest.mark.parametrize("mutation", ["decay_sign", "no_dt", "ignore_t0", "decay_from_start"])
def test_chunk_state_mutants_are_caught(monkeypatch, mutation):
    """Plausible slips in the shard-state closed form (decay exponent reversed, the dt
    factor dropped, the document start ignored, decay measured from the shard start)
    fail its pinning against the SSD recurrence."""

    def mutant(x, B, e, cum_A, t0=None):
        bsz, T, H, _ = x.shape
        if mutation == "decay_sign":
            w = torch.exp(cum_A - cum_A[:, -1:, :]) * e
        elif mutation == "no_dt":
            w = torch.exp(cum_A[:, -1:, :] - cum_A)
        elif mutation == "decay_from_start":
            w = torch.exp(cum_A) * e
        else:
            w = torch.exp(cum_A[:, -1:, :] - cum_A) * e
        if t0 is not None and mutation != "ignore_t0":
            keep = torch.arange(T)[None, :] >= torch.as_tensor(t0).reshape(bsz, 1)
            w = w * keep[:, :, None].to(w.dtype)
        Bx = B.repeat_interleave(H // B.shape[2], dim=2)
        return torch.einsum("bth,bthd,bthn->bhdn", w, x, Bx)

    monkeypatch.setattr(sp, "chunk_state", mutant)
    with pytest.raises(AssertionError):
        pin.test_chunk_state_equals_ssd_final_state(2)


def _shard_batch_variant(batch, cp_rank, cp_size, *, zero_pad_pos=False, pad_label_zero=False,
                         per_shard_shift=False, swap_chunks=False):
    """oracle/shard.zigzag_shard_batch with one planted mistake."""
    from oracle import shard as osh

    bsz, seq_len = batch["input_ids"].shape[:2]
    pad_len = osh.pad_multiple(seq_len, 2 * cp_size)
    if not per_shard_shift and "labels" in batch:
        shift = torch.full_like(batch["labels"], -100)
        shift[:, :-1] = batch["labels"][:, 1:]
        batch["shift_labels"] = shift
    batch["position_ids"] = torch.arange(seq_len).unsqueeze(0).expand(bsz, -1)
    total = seq_len + pad_len
    for key, val in list(batch.items()):
        if pad_len and val.dim() > 1 and val.size(1) == seq_len:
            fill = -100 if key in ("labels", "shift_labels") and not pad_label_zero else 0
            pad = torch.full((val.size(0), pad_len, *val.shape[2:]), fill, dtype=val.dtype)
            if key == "position_ids" and not zero_pad_pos:
                pad = val[:, -1:] + torch.arange(1, pad_len + 1)
            batch[key] = torch.cat([val, pad], dim=1)
    half = total // (2 * cp_size)
    lo, hi = cp_rank, 2 * cp_size - 1 - cp_rank
    parts = [torch.arange(lo * half, (lo + 1) * half), torch.arange(hi * half, (hi + 1) * half)]
    idx = torch.cat(parts[::-1] if swap_chunks else parts)
    for key, val in list(batch.items()):
        if val.dim() > 1 and val.size(1) == total:
            batch[key] = val.index_select(1, idx)
    if per_shard_shift and "labels" in batch:  # shifted after sharding: boundary targets lost
        shift = torch.full_like(batch["labels"], -100)
        shift[:, :-1] = batch["labels"][:, 1:]
        batch["shift_labels"] = shift
    return batch, (seq_len, pad_len)


@pytest.mark.parametrize("mutation", ["zero_pad_pos", "pad_label_zero", "per_shard_shift",
                                      "swap_chunks"])
def test_shard_mutants_are_caught(mutation):
    from tests.test_shard_oracle import check_shard_batch

    check_shard_batch(_shard_batch_variant)  # the unmutated variant passes
    with pytest.raises(AssertionError):
        check_shard_batch(lambda b, r, w: _shard_batch_variant(b, r, w, **{mutation: True}))


def test_unshard_mutant_is_caught():
    from oracle import shard as osh
    from tests.test_shard_oracle import check_shard_batch

    def reversed_ranks(shards, seq):  # scatters rank r's rows to rank (P-1-r)'s positions
        return osh.zigzag_unshard_tensor(shards[::-1], seq)

    with pytest.raises(AssertionError):
        check_shard_batch(osh.zigzag_shard_batch, reversed_ranks)


def _varlen_shared_documents(qs, ks, vs, cu, *, causal):
    """Mutant: every batch row packed with row 0's documents (the mask of ring/loop.py:182
    built from the first S ids only)."""
    P, L = len(qs), qs[0].shape[2]
    S = P * L
    cu0 = torch.tensor([c for c in cu.tolist() if c <= S] + ([S] if S not in cu.tolist() else []))
    b = qs[0].shape[0]
    outs = [[] for _ in range(P)]
    lses = [[] for _ in range(P)]
    for row in range(b):
        o, l = rm.varlen_ring_forward([t[row:row + 1] for t in qs], [t[row:row + 1] for t in ks],
                                      [t[row:row + 1] for t in vs], cu0, causal=causal)
        for r in range(P):
            outs[r].append(o[r])
            lses[r].append(l[r])
    return [torch.cat(o) for o in outs], [torch.cat(x) for x in lses]


def _varlen_causal_ignored(qs, ks, vs, cu, *, causal):
    """Mutant: the causal flag dropped (every packed ring causal)."""
    return rm.varlen_ring_forward(qs, ks, vs, cu, causal=True)


@pytest.mark.parametrize("mutant,causal", [(_varlen_shared_documents, True),
                                            (_varlen_shared_documents, False),
                                            (_varlen_causal_ignored, False)])
def test_varlen_row_mutants_are_caught(mutant, causal):
    with pytest.raises(AssertionError):
        pin.check_varlen_rows(mutant, causal)
