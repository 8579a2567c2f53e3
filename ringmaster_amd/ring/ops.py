"""Tensor-level wrappers of the batched block-attention kernels.

A *job* is one block problem of the C ABI: ``q[sq]`` attends ``k/v[sk]`` with
tensors given as ``[batch, seq, heads, dim]`` views (any strides on the first
three axes, contiguous ``dim``), lse-like tensors as ``[batch, heads, seq]``
views with a contiguous ``seq`` axis. All jobs of one call share the layout
(strides) of each tensor kind, as the per-rank views of one stacked tensor do,
and are launched together (up to 16 per kernel launch).
"""

from __future__ import annotations

import ctypes
import dataclasses

import torch

from ringmaster_amd import abi


@dataclasses.dataclass
class FwdJob:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    mode: int = abi.FWD_WRITE
    out: torch.Tensor | None = None
    lse: torch.Tensor | None = None
    acc_out: torch.Tensor | None = None
    acc_lse: torch.Tensor | None = None
    # document-mask metadata: [sq] / [sk], or [batch, sq] / [batch, sk] per batch row
    q_gidx: torch.Tensor | None = None
    k_gidx: torch.Tensor | None = None
    q_doc: torch.Tensor | None = None
    k_doc: torch.Tensor | None = None
    window: int | None = None  # bound on pos_q - pos_k (global indices with document masks)
    drop_q0: int = 0  # dropout coordinates of the first query / key
    drop_k0: int = 0
    right: int = 0  # causal masks: bound on pos_k - pos_q (0: causal attention)


@dataclasses.dataclass
class BwdJob:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    dout: torch.Tensor
    lse: torch.Tensor
    delta: torch.Tensor
    dq_mode: int
    dkv_mode: int
    nlse: torch.Tensor | None = None
    dq_acc: torch.Tensor | None = None
    dq: torch.Tensor | None = None
    dk_acc: torch.Tensor | None = None
    dv_acc: torch.Tensor | None = None
    dk: torch.Tensor | None = None
    dv: torch.Tensor | None = None
    q_gidx: torch.Tensor | None = None
    k_gidx: torch.Tensor | None = None
    q_doc: torch.Tensor | None = None
    k_doc: torch.Tensor | None = None
    window: int | None = None
    drop_q0: int = 0
    drop_k0: int = 0
    right: int = 0


def _i32_field(v, what):
    v = int(v)
    if not -(1 << 31) <= v < (1 << 31):
        raise ValueError(f"{what} {v} outside int32")
    return v


def _set_problem_extras(p, job):
    if job.window is not None:
        p.has_window, p.window_left = 1, _i32_field(job.window, "window bound")
    p.drop_q0 = _i32_field(job.drop_q0, "dropout query offset")
    p.drop_k0 = _i32_field(job.drop_k0, "dropout key offset")
    p.window_right = _i32_field(job.right, "right window bound")


def _set_dropout(lay, dropout):
    """``dropout``: None or (p, seed), seed a 64-bit integer."""
    if dropout is None or not dropout[0]:
        return
    p, seed = float(dropout[0]), int(dropout[1]) & ((1 << 64) - 1)
    lay.dropout_p = p
    lay.drop_seed_lo, lay.drop_seed_hi = seed & 0xFFFFFFFF, seed >> 32


_H = None  # the call's 16-bit element type (bf16 or fp16), the dtype of q

_ROLES = {
    # role -> (layout field prefix, number of strides, dtype)
    "q": ("q", 3, _H),
    "k": ("k", 3, _H),
    "v": ("v", 3, _H),
    "out": ("o", 3, _H),
    "dout": ("o", 3, _H),
    "dq": ("o", 3, _H),
    "acc_out": ("a", 3, torch.float32),
    "dq_acc": ("a", 3, torch.float32),
    "lse": ("l", 2, torch.float32),
    "acc_lse": ("l", 2, torch.float32),
    "delta": ("l", 2, torch.float32),
    "nlse": ("l", 2, torch.float32),
    "dk": ("dk", 3, _H),
    "dv": ("dk", 3, _H),
    "dk_acc": ("ka", 3, torch.float32),
    "dv_acc": ("ka", 3, torch.float32),
}

_DTYPES = {torch.bfloat16: abi.DTYPE_BF16, torch.float16: abi.DTYPE_F16}


def _fill_layout(jobs, batch, hq, hkv, head_dim, scale, mask, half=None) -> abi.AttnLayout:
    """The call's layout; ``half`` (default: the first job's q dtype) is the 16-bit type
    of q/k/v/out/dout and the 16-bit gradients."""
    half = half if half is not None else jobs[0].q.dtype
    if half not in _DTYPES:
        raise NotImplementedError(f"attention computes in bf16 or fp16 (got {half})")
    lay = abi.AttnLayout()
    lay.batch, lay.hq, lay.hkv, lay.head_dim = batch, hq, hkv, head_dim
    lay.scale = float(scale)
    lay.mask = mask
    lay.dtype = _DTYPES[half]
    seen: dict[str, tuple] = {}
    for job in jobs:
        for role, (prefix, n, dtype) in _ROLES.items():
            t = getattr(job, role, None)
            if t is None:
                continue
            dtype = half if dtype is _H else dtype
            if t.dtype != dtype:
                raise ValueError(f"{role} must be {dtype} (got {t.dtype})")
            abi.require_device(t)
            if n == 3:
                if t.dim() != 4 or t.stride(3) != 1:
                    raise ValueError(f"{role} must be [batch, seq, heads, dim] with contiguous dim")
                st = (t.stride(0), t.stride(1), t.stride(2))
            else:
                if t.dim() != 3 or (t.shape[2] > 1 and t.stride(2) != 1):
                    raise ValueError(f"{role} must be [batch, heads, seq] with contiguous seq")
                st = (t.stride(0), t.stride(1))
            if prefix in seen and seen[prefix] != st:
                raise ValueError(f"all {prefix}-kind tensors of one call must share strides "
                                 f"({seen[prefix]} vs {st} for {role})")
            seen[prefix] = st
    for prefix, st in seen.items():
        names = ("_sb", "_ss", "_sh") if len(st) == 3 else ("_sb", "_sh")
        for nm, s in zip(names, st):
            setattr(lay, prefix + nm, int(s))
    return lay


def _check_shapes(q, k, v, batch, hq, hkv, d):
    if q.shape[0] != batch or q.shape[2] != hq or q.shape[3] != d:
        raise ValueError(f"q shape {tuple(q.shape)} does not match the call layout")
    if k.shape[0] != batch or k.shape[2] != hkv or k.shape[3] != d or v.shape != k.shape:
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match")


def _int32(t):
    if t is None:
        return None
    if t.dtype != torch.int32 or t.stride(-1) != 1:
        raise ValueError("index tensors must be int32 with a contiguous last axis")
    abi.require_device(t)
    return t.data_ptr()


_META = ("q_gidx", "k_gidx", "q_doc", "k_doc")


def _set_meta_stride(lay, jobs, batch):
    """Document-mask metadata is [n] (every batch row shares it) or [batch, n] (per row,
    ring/loop.py:178): the layout's m_sb is the row stride, which all of a call's
    per-row arrays must share."""
    strides = set()
    for j in jobs:
        for name in _META:
            t = getattr(j, name)
            if t is None:
                continue
            if t.dim() == 1 or (t.dim() == 2 and t.shape[0] == 1):
                strides.add(0)
            elif t.dim() == 2 and t.shape[0] == batch:
                strides.add(t.stride(0))
            else:
                raise ValueError(f"{name} must be [n] or [batch, n] (got {tuple(t.shape)})")
    if len(strides) > 1:
        raise ValueError("the document metadata of one call must share its row stride")
    lay.m_sb = int(strides.pop()) if strides else 0


def attn_fwd(jobs: list[FwdJob], *, scale: float, mask: int, dropout=None) -> None:
    """Launch the batched block forward (rmx_attn_fwd) for ``jobs``; ``dropout`` is None or
    (p, seed)."""
    if not jobs:
        return
    q0, k0 = jobs[0].q, jobs[0].k
    batch, hq, d, hkv = q0.shape[0], q0.shape[2], q0.shape[3], k0.shape[2]
    for j in jobs:
        _check_shapes(j.q, j.k, j.v, batch, hq, hkv, d)
    lay = _fill_layout(jobs, batch, hq, hkv, d, scale, mask)
    _set_dropout(lay, dropout)
    _set_meta_stride(lay, jobs, batch)
    arr = (abi.FwdProblem * len(jobs))()
    for i, j in enumerate(jobs):
        p = arr[i]
        p.q, p.k, p.v = j.q.data_ptr(), j.k.data_ptr(), j.v.data_ptr()
        p.out, p.lse = abi.ptr(j.out), abi.ptr(j.lse)
        p.acc_out, p.acc_lse = abi.ptr(j.acc_out), abi.ptr(j.acc_lse)
        p.q_gidx, p.k_gidx = _int32(j.q_gidx), _int32(j.k_gidx)
        p.q_doc, p.k_doc = _int32(j.q_doc), _int32(j.k_doc)
        p.sq, p.sk, p.mode = j.q.shape[1], j.k.shape[1], j.mode
        _set_problem_extras(p, j)
    abi.check(abi.lib().rmx_attn_fwd(ctypes.byref(lay), arr, len(jobs), abi.stream_of(q0)))


def attn_bwd_delta(out: torch.Tensor, dout: torch.Tensor, delta: torch.Tensor, hkv: int,
                   lse: torch.Tensor | None = None, nlse: torch.Tensor | None = None) -> None:
    """delta[b, h, s] = sum_d dout * out (fp32). dout: [b, s, h, d] bf16 or fp16; out: the same
    type with the strides of dout, or the fp32 final out (any strides with a contiguous dim). With ``nlse``
    (and the global ``lse``), also nlse = -lse * log2(e), which the dK/dV kernel reads; lse,
    delta and nlse must share their strides."""
    batch, sq, hq, d = dout.shape
    if out.shape != dout.shape:
        raise ValueError("out and dout must share their shape")
    f32 = out.dtype == torch.float32
    if not f32 and (out.stride() != dout.stride() or out.dtype != dout.dtype):
        raise ValueError("a 16-bit out must share dout's type and strides")
    if (nlse is None) != (lse is None):
        raise ValueError("lse and nlse go together")
    job = FwdJob(q=dout, k=dout[:, :0, :hkv], v=dout[:, :0, :hkv], out=dout, lse=delta,
                 acc_out=out if f32 else None)
    jobs = [job]
    if nlse is not None:
        if lse.shape != delta.shape or nlse.shape != delta.shape:
            raise ValueError("lse, delta and nlse must share their shape")
        jobs += [FwdJob(q=dout, k=job.k, v=job.v, lse=lse), FwdJob(q=dout, k=job.k, v=job.v, lse=nlse)]
    lay = _fill_layout(jobs, batch, hq, hkv, d, 1.0, abi.MASK_FULL)
    abi.check(abi.lib().rmx_attn_bwd_delta(ctypes.byref(lay), out.data_ptr(), int(f32),
                                           dout.data_ptr(), delta.data_ptr(), abi.ptr(lse),
                                           abi.ptr(nlse), sq, abi.stream_of(dout)))


def attn_bwd(jobs: list[BwdJob], *, scale: float, mask: int, dropout=None) -> None:
    """Launch the batched block backward (rmx_attn_bwd) for ``jobs``; ``dropout`` must be the
    forward's (p, seed) and each job the forward's dropout offsets."""
    if not jobs:
        return
    q0, k0 = jobs[0].q, jobs[0].k
    batch, hq, d, hkv = q0.shape[0], q0.shape[2], q0.shape[3], k0.shape[2]
    for j in jobs:
        _check_shapes(j.q, j.k, j.v, batch, hq, hkv, d)
    lay = _fill_layout(jobs, batch, hq, hkv, d, scale, mask)
    _set_dropout(lay, dropout)
    _set_meta_stride(lay, jobs, batch)
    arr = (abi.BwdProblem * len(jobs))()
    for i, j in enumerate(jobs):
        p = arr[i]
        p.q, p.k, p.v, p.dout = j.q.data_ptr(), j.k.data_ptr(), j.v.data_ptr(), j.dout.data_ptr()
        p.lse, p.delta, p.nlse = j.lse.data_ptr(), j.delta.data_ptr(), abi.ptr(j.nlse)
        p.dq_acc, p.dq = abi.ptr(j.dq_acc), abi.ptr(j.dq)
        p.dk_acc, p.dv_acc = abi.ptr(j.dk_acc), abi.ptr(j.dv_acc)
        p.dk, p.dv = abi.ptr(j.dk), abi.ptr(j.dv)
        p.q_gidx, p.k_gidx = _int32(j.q_gidx), _int32(j.k_gidx)
        p.q_doc, p.k_doc = _int32(j.q_doc), _int32(j.k_doc)
        p.sq, p.sk = j.q.shape[1], j.k.shape[1]
        p.dq_mode, p.dkv_mode = j.dq_mode, j.dkv_mode
        _set_problem_extras(p, j)
    abi.check(abi.lib().rmx_attn_bwd(ctypes.byref(lay), arr, len(jobs), abi.stream_of(q0)))
