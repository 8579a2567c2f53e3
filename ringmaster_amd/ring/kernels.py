"""Block-attention provider ``mi355x_hip`` and the Dao-signature op pair.

``mi355x_hip_block`` keeps the provider contract of the reference's ``PROVIDERS``
(ring/kernels.py:28-85): ``fn(q, k, v, *, causal, scaling, dropout,
attn_implementation, window) -> (out [b, sq, h, d] in q.dtype, lse [b, h, sq]
fp32)``, q/k/v ``[b, s, h, d]``, GQA by ``kv_head = q_head // (hq/hkv)``, causal
bottom-right aligned (ring/kernels.py:64-67), a sliding window ``(left, right)`` with
flash attention's semantics (the ``window_size`` that the flash provider passes on,
ring/kernels.py:37-38): ``pos_q - pos_k > left`` and ``pos_k - pos_q > right`` masked on
the same bottom-right aligned positions, a negative bound or one of at least ``sk`` keys
unbounded, and ``right`` 0 under ``causal`` (the math provider, ring/kernels.py:68-72,
reads ``left`` only: the two agree wherever ``right`` is unbounded or the call causal),
head dims that are
multiples of 8 up to 256, bf16 or fp16, and attention dropout (the Dao semantics: kept
probabilities scaled by 1 / (1 - p), lse undropped; the mask is the kernels' hash of
(seed, batch, head, query, key), so the backward replays it exactly). It is autograd-aware
like ``hf_kernels``/``math``; the lse output is not differentiable (as with flash).

``flash_ops()`` returns ``(fwd, bwd)`` with the positional signatures of the Dao
low-level ops that the ring schedules call (ring/p2p_attn.py:27-62,
ring/zigzag.py:131,219): ``fwd`` allocates ``(out, lse)``; ``bwd`` writes into the
caller's ``dq, dk, dv`` with the global out/lse.
"""

from __future__ import annotations

import math

import torch

from ringmaster_amd import abi
from ringmaster_amd.ring import ops


def _validate(q, k, v, dropout, softcap=0.0, alibi=None):
    """Checks of the provider contract."""
    abi.require_device(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q/k/v must be [batch, seq, heads, dim]")
    if q.shape[2] % k.shape[2]:
        raise ValueError("Query heads must be divisible by KV heads")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"mi355x_hip blocks compute in bf16 or fp16 (got {q.dtype})")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k and v must share their dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    d = q.shape[-1]
    if d % 8 or d > 256 or k.shape[-1] != d or v.shape[-1] != d:
        raise NotImplementedError(f"head_dim {d} is not supported (a multiple of 8, at most 256)")
    if not 0.0 <= float(dropout) < 1.0:
        raise ValueError(f"dropout must lie in [0, 1) (got {dropout})")
    if softcap:
        raise NotImplementedError("mi355x_hip blocks do not implement softcap")
    if alibi is not None:
        raise NotImplementedError("mi355x_hip blocks do not implement ALiBi")


_M64 = (1 << 64) - 1


def _splitmix64(x: int) -> int:
    """SplitMix64's output function (Steele, Lea and Flood, 2014) on a 64-bit integer."""
    x = (x + 0x9E3779B97F4A7C15) & _M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _M64
    return x ^ (x >> 31)


def dropout_rng_state(device=None) -> tuple[int, int]:
    """Draw dropout randomness the way flash attention does: the (seed, offset) of the
    device's default generator, whose offset the call advances by 4 (one philox step).
    ``torch.manual_seed`` resets both, so the draws are reproducible, and torch's CPU
    generator (the stream of samplers and other host randomness) is left untouched."""
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    gen = torch.cuda.default_generators[torch.cuda.current_device() if idx is None else idx]
    seed, offset = gen.initial_seed(), gen.get_offset()
    gen.set_offset(offset + 4)
    return int(seed) & _M64, int(offset)


def seed_of_rng_state(seed: int, offset: int) -> int:
    """The kernels' 64-bit mask seed of a generator (seed, offset) pair."""
    return _splitmix64(_splitmix64(seed) ^ offset)


def new_dropout_seed(device=None) -> int:
    """A 64-bit dropout mask seed from the device generator (see ``dropout_rng_state``)."""
    return seed_of_rng_state(*dropout_rng_state(device))


def window_bounds(window, causal: bool, sk: int | None = None):
    """Flash attention's ``window_size = (left, right)`` as the kernels' bounds ``(left,
    right)``: ``left`` on ``pos_q - pos_k``, ``right`` on ``pos_k - pos_q``, None where
    unbounded. The rules of flash attention 2's window arguments: a negative bound is
    unbounded, so is a bound of at least ``sk`` keys, a causal call is bounded at right = 0
    by its mask (``right`` is then None), and a window bounded on the left only is bounded
    on the right at ``sk`` (which masks keys only for rows of a block with sq > sk + 1).
    Without ``sk`` (blocks with sq <= sk) the last two rules change nothing."""
    if window is None:
        return None, None
    left, right = (int(x) for x in window)
    if sk is not None:
        left, right = (-1 if x >= sk else x for x in (left, right))
        if left >= 0 and right < 0:
            right = sk
    return (left if left >= 0 else None), (None if causal or right < 0 else right)


def window_left(window):
    """The packed ring's window (its math path reads ``window[0]`` only, ring/loop.py:
    185-186): the bound on ``pos_q - pos_k``, or None. ``(-1, -1)`` (and None) is no
    window; a negative ``left`` with a non-negative ``right`` is refused (the math path
    would mask every key at or before the diagonal)."""
    if window is None:
        return None
    left, right = (int(x) for x in window)
    if left < 0:
        if right >= 0:
            raise NotImplementedError(f"window {tuple(window)}: only left windows are supported")
        return None
    return left


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Keep views whose strides the kernels accept; copy anything else once."""
    if (t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1])
            and t.data_ptr() % 16 == 0):
        return t
    return t.contiguous()


def _mask_of(causal: bool, right):
    """The kernels' mask kind and right bound: a right-bounded window runs as the causal
    mask with its diagonal moved ``right`` keys to the right."""
    if causal:
        return abi.MASK_CAUSAL, 0
    if right is None:
        return abi.MASK_FULL, 0
    if right < 0:
        raise ValueError(f"right window bound {right} < 0")
    return abi.MASK_CAUSAL, min(int(right), 1 << 28)  # sk < 2^27: past that, unbounded


def block_forward(q, k, v, scale: float, causal: bool, keep_f32: bool = False, window=None,
                  dropout=None, right=None):
    """(out [b, sq, hq, d] in q's dtype, lse fp32 [b, hq, sq]) of one block; with ``keep_f32`` also
    the fp32 out (what the backward's delta is computed from). ``window``: bound on
    ``pos_q - pos_k`` (bottom-right aligned positions) or None; ``right``: bound on
    ``pos_k - pos_q`` of a non-causal block or None; ``dropout``: None or (p, seed)."""
    b, sq, hq, d = q.shape
    out = torch.empty((b, sq, hq, d), dtype=q.dtype, device=q.device)
    lse = torch.empty((b, hq, sq), dtype=torch.float32, device=q.device)
    out32 = torch.empty((b, sq, hq, d), dtype=torch.float32, device=q.device) if keep_f32 else None
    mask, shift = _mask_of(causal, right)
    ops.attn_fwd([ops.FwdJob(q=q, k=k, v=v, mode=abi.FWD_WRITE, out=out, lse=lse,
                             acc_out=out32, window=window, right=shift)],
                 scale=scale, mask=mask, dropout=dropout)
    return (out, lse, out32) if keep_f32 else (out, lse)


def block_backward(dout, q, k, v, out, lse, scale: float, causal: bool, dq=None, dk=None, dv=None,
                   out_f32=None, window=None, dropout=None, right=None):
    """dq, dk, dv (q's dtype) of one block using the given (global) out/lse; returns delta too.
    ``out_f32`` (the forward's fp32 out), when given, is what delta = rowsum(dout * out) reads;
    otherwise the 16-bit ``out`` is used, as a Dao-style backward does."""
    b, sq, hq, d = q.shape
    hkv = k.shape[2]
    if dout.stride() != out.stride():
        # the delta kernel reads a bf16 out and dout with one set of strides
        dout = torch.empty_like(out).copy_(dout)
    delta = torch.empty((b, hq, sq), dtype=torch.float32, device=q.device)
    nlse = torch.empty_like(delta)
    if not lse.is_contiguous():
        lse = lse.contiguous()
    ops.attn_bwd_delta(out if out_f32 is None else out_f32, dout, delta, hkv, lse=lse, nlse=nlse)
    dq_t = dq if (dq is not None and dq.stride() == dout.stride()) else torch.empty_like(dout)
    dk_t = dk if (dk is not None and dk.is_contiguous()) else torch.empty(
        k.shape, dtype=k.dtype, device=k.device)
    dv_t = dv if (dv is not None and dv.stride() == dk_t.stride()) else torch.empty_like(dk_t)
    mask, shift = _mask_of(causal, right)
    ops.attn_bwd([ops.BwdJob(q=q, k=k, v=v, dout=dout, lse=lse, delta=delta, nlse=nlse,
                             dq_mode=abi.GRAD_WRITE_BF16, dkv_mode=abi.GRAD_WRITE_BF16,
                             dq=dq_t, dk=dk_t, dv=dv_t, window=window, right=shift)],
                 scale=scale, mask=mask, dropout=dropout)
    for dst, src in ((dq, dq_t), (dk, dk_t), (dv, dv_t)):
        if dst is not None and dst is not src:
            dst.copy_(src)
    return (dq if dq is not None else dq_t, dk if dk is not None else dk_t,
            dv if dv is not None else dv_t, delta)


class _HipBlockAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal, scale, window, dropout):
        q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
        left, right = window
        out, lse, out32 = block_forward(q, k, v, scale, causal, keep_f32=True, window=left,
                                        dropout=dropout, right=right)
        ctx.save_for_backward(q, k, v, out, lse, out32)
        ctx.causal, ctx.scale, ctx.window, ctx.dropout = causal, scale, window, dropout
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse, out32 = ctx.saved_tensors
        dq, dk, dv, _ = block_backward(_kernel_ready(dout), q, k, v, out, lse, ctx.scale,
                                       ctx.causal, out_f32=out32, window=ctx.window[0],
                                       dropout=ctx.dropout, right=ctx.window[1])
        return dq, dk, dv, None, None, None, None


def mi355x_hip_block(q, k, v, *, causal, scaling, dropout=0.0, attn_implementation=None,
                     window=None, dropout_seed=None):
    """q/k/v: [b, s, h, d] bf16 or fp16 on the MI355X. Returns (out [b,s,h,d], lse [b,h,s]).
    ``dropout`` > 0 drops attention probabilities with the kernels' hash mask, seeded by
    ``dropout_seed`` (default: drawn from torch's CPU generator); the backward replays the
    same mask."""
    _validate(q, k, v, dropout)
    bounds = window_bounds(window, bool(causal), k.shape[1])
    scale = scaling if scaling is not None else 1.0 / math.sqrt(q.shape[-1])
    drop = None
    if dropout:
        drop = (float(dropout),
                new_dropout_seed(q.device) if dropout_seed is None else int(dropout_seed))
    return _HipBlockAttention.apply(q, k, v, bool(causal), float(scale), bounds, drop)


PROVIDERS = {
    "mi355x_hip": mi355x_hip_block,
}


# -- Dao-signature op pair (positional arguments as called at ring/zigzag.py:131,219) --
def _flash_attn_forward(q, k, v, dropout_p, softmax_scale, causal, window_size_left=-1,
                        window_size_right=-1, softcap=0.0, alibi_slopes=None,
                        return_softmax=False):
    _validate(q, k, v, dropout_p, softcap, alibi_slopes)
    left, right = window_bounds((window_size_left, window_size_right), bool(causal), k.shape[1])
    if return_softmax:
        raise NotImplementedError("return_softmax is not supported")
    rng_state, drop = None, None
    if dropout_p:
        gseed, goff = dropout_rng_state(q.device)
        drop = (float(dropout_p), seed_of_rng_state(gseed, goff))
        # the Dao ops' rng_state: the generator's (seed, offset) as int64 (the seed's 64 bits
        # read as signed), on the host, so the backward reads it without a device sync
        rng_state = torch.tensor([gseed - (1 << 64) if gseed >= (1 << 63) else gseed, goff],
                                 dtype=torch.int64)
    out, lse = block_forward(_kernel_ready(q), _kernel_ready(k), _kernel_ready(v),
                             float(softmax_scale), bool(causal), window=left, dropout=drop,
                             right=right)
    return out, lse, None, rng_state


def _flash_attn_backward(dout, q, k, v, out, lse, dq, dk, dv, dropout_p, softmax_scale, causal,
                         window_size_left=-1, window_size_right=-1, softcap=0.0,
                         alibi_slopes=None, deterministic=False, rng_state=None):
    _validate(q, k, v, dropout_p, softcap, alibi_slopes)
    left, right = window_bounds((window_size_left, window_size_right), bool(causal), k.shape[1])
    drop = None
    if dropout_p:
        if rng_state is None:
            raise ValueError("a backward with dropout needs the forward's rng_state")
        st = torch.as_tensor(rng_state).flatten().tolist()
        drop = (float(dropout_p), seed_of_rng_state(int(st[0]) & _M64, int(st[1])))
    _, _, _, delta = block_backward(_kernel_ready(dout), _kernel_ready(q), _kernel_ready(k),
                                    _kernel_ready(v), _kernel_ready(out), lse,
                                    float(softmax_scale), bool(causal), dq, dk, dv, window=left,
                                    dropout=drop, right=right)
    return dq, dk, dv, delta


def flash_ops():
    """(fwd, bwd) low-level ops, the drop-in for ``_flash_ops()`` (ring/p2p_attn.py:27-35)."""
    return _flash_attn_forward, _flash_attn_backward
