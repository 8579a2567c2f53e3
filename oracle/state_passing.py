"""CPU restatement of the recurrent state passing (test infrastructure only).

Follows strategies/state_passing.py:19-59 (local scan, ``cp_linear_scan`` with the
all-gather of (A_r, B_r) emulated as a list over ranks), the Mamba2 SSD reference
of tests/test_mamba_cp.py:16-32, and ``cp_state_prefix`` / ``mamba2_cp_correction``
(strategies/mamba.py:68-139), and the shard final state the CP scan wrapper gathers
(``final`` of mamba.py:113-141,160-172, computed there by mamba-ssm's
``mamba_chunk_scan_combined``, a dependency absent from the reference tree).
Autograd-capable (torch ops only); ``linear_scan_grads`` also gives the scan's gradients
from the explicit adjoint recurrence, for sequences too long for an autograd graph.
"""

from __future__ import annotations

import torch


def local_linear_scan(a, b):
    """h_t = a_t h_{t-1} + b_t from zero (strategies/state_passing.py:19-26). a, b: [batch, L, d]."""
    h = torch.zeros_like(b[:, 0])
    out = []
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        out.append(h)
    return torch.stack(out, dim=1)


def local_linear_scan_vec(a, b):
    """Same recurrence, vectorised over d with a Python loop over t (for larger L*d)."""
    h = torch.zeros_like(b[:, 0])
    out = torch.empty_like(b)
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        out[:, t] = h
    return out


def cp_linear_scan_emulated(a, b, world, scan=local_linear_scan):
    """cp_linear_scan for every rank of a ``world``-rank group, in one process
    (strategies/state_passing.py:29-59). a, b: full [batch, L, d]; returns full h."""
    L = a.shape[1]
    if L % world:
        raise ValueError("L not divisible by world")
    n = L // world
    locs, cums, pairs = [], [], []
    for r in range(world):
        sa, sb = a[:, r * n:(r + 1) * n], b[:, r * n:(r + 1) * n]
        local_h = scan(sa, sb)
        cum_a = torch.cumprod(sa, dim=1)
        locs.append(local_h)
        cums.append(cum_a)
        pairs.append((cum_a[:, -1], local_h[:, -1]))  # all-gathered (A_r, B_r)
    outs = []
    for r in range(world):
        h_in = torch.zeros_like(pairs[r][1])
        for j in range(r):
            h_in = pairs[j][0] * h_in + pairs[j][1]
        outs.append(locs[r] + cums[r] * h_in.unsqueeze(1))
    return torch.cat(outs, dim=1)


def rank_linear_scan(a, b, h_in):
    """One rank's ``cp_linear_scan`` on its local chunk given the state entering it
    (strategies/state_passing.py:38-39,59): the zero-init local scan corrected by
    ``cumprod(a) * h_in``. a, b: [batch, L_local, d]; h_in: [batch, d]."""
    return local_linear_scan(a, b) + torch.cumprod(a, dim=1) * h_in.unsqueeze(1)


def linear_scan_grads(a, b, dh, h_in=None):
    """h_t = a_t h_{t-1} + b_t from ``h_in`` (zero when None) and its gradients from the
    adjoint recurrence g_t = dh_t + a_{t+1} g_{t+1}: db_t = g_t, da_t = g_t h_{t-1},
    dh_in = a_0 g_0. Explicit (no autograd graph), vectorised over batch and channels with
    a loop over t, for long sequences. a, b, dh: [batch, L, d]; returns (h, da, db, dh_in)."""
    bsz, L, d = b.shape
    prev = torch.zeros_like(b[:, 0]) if h_in is None else h_in.clone()
    h_in0 = prev.clone()
    h = torch.empty_like(b)
    for t in range(L):
        prev = a[:, t] * prev + b[:, t]
        h[:, t] = prev
    db = torch.empty_like(b)
    g = torch.zeros_like(b[:, 0])
    for t in range(L - 1, -1, -1):
        g = dh[:, t] + (a[:, t + 1] * g if t + 1 < L else 0)
        db[:, t] = g
    h_before = torch.cat([h_in0[:, None], h[:, :-1]], dim=1)
    da = db * h_before
    return h, da, db, (a[:, 0] * db[:, 0] if L else torch.zeros_like(h_in0))


def scan_prefix(a, b, world):
    """The H_in of every rank (strategies/state_passing.py:49-57): the all-gathered
    (A_r, B_r) = (cumprod(a)[-1], local_h[-1]) of each chunk folded in rank order.
    a, b: full [batch, L, d]; returns [world, batch, d]."""
    n = a.shape[1] // world
    h_in = torch.zeros_like(b[:, 0])
    out = []
    for r in range(world):
        out.append(h_in)
        sa, sb = a[:, r * n:(r + 1) * n], b[:, r * n:(r + 1) * n]
        h_in = torch.cumprod(sa, dim=1)[:, -1] * h_in + local_linear_scan(sa, sb)[:, -1]
    return torch.stack(out)


def ssd_reference(x, dt, A, B, C):
    """Mamba2 SSD: h_t = exp(A dt_t) h_{t-1} + (dt_t B_t) (x) x_t; y_t = C_t . h_t
    (tests/test_mamba_cp.py:16-32). x [b,T,H,d], dt [b,T,H], A [H], B/C [b,T,G,n]."""
    bsz, T, H, d = x.shape
    G, n = B.shape[2], B.shape[3]
    hpg = H // G
    Bx = B.repeat_interleave(hpg, dim=2)
    Cx = C.repeat_interleave(hpg, dim=2)
    h = torch.zeros(bsz, H, d, n, dtype=x.dtype)
    outs = []
    for t in range(T):
        dA = torch.exp(A * dt[:, t])
        inp = dt[:, t][:, :, None, None] * x[:, t][:, :, :, None] * Bx[:, t][:, :, None, :]
        h = dA[:, :, None, None] * h + inp
        y = (Cx[:, t][:, :, None, :] * h).sum(-1)
        outs.append(y.reshape(bsz, H * d))
    return torch.stack(outs, 1), h


def cp_state_prefix_emulated(finals, decays):
    """H_in for every rank from per-rank (B_r = final state, A_r = chunk decay [b, H])
    (strategies/mamba.py:68-98): H_in_r = sum_{j<r} (prod_{j<k<r} A_k) B_j."""
    world = len(finals)
    prefixes = []
    for r in range(world):
        h_prev = torch.zeros_like(finals[r])
        for j in range(r):
            h_prev = decays[j][..., None, None] * h_prev + finals[j]
        prefixes.append(h_prev)
    return prefixes


def mamba2_cp_correction(out, h_final, C, cum_A, h_prev, num_heads, head_dim, seq_idx=None):
    """y_t += C_t . (exp(cumA_t) H_in); state += exp(cumA_last) H_in (strategies/mamba.py:101-139).
    seq_idx [b, T]: tokens with seq_idx != 0 start a fresh packed sequence on this rank and
    get no correction (:124-126); no state is updated when the last token of any batch
    row is such a token (seq_idx[:, -1].any(), :131-135)."""
    if not h_prev.any():
        return out, h_final
    B, T, _ = out.shape
    hpg = num_heads // C.shape[2]
    decay = torch.exp(cum_A).float()
    prop = decay[:, :, :, None, None] * h_prev[:, None].float()
    Cx = C.float().repeat_interleave(hpg, dim=2)
    dy = torch.einsum("bthn,bthdn->bthd", Cx, prop)
    if seq_idx is not None:
        dy = dy * (seq_idx == 0).to(dy.dtype)[:, :, None, None]
    corrected = out + dy.reshape(B, T, num_heads * head_dim).to(out.dtype)
    if seq_idx is not None and seq_idx[:, -1].any():
        return corrected, h_final
    h = h_final + (decay[:, -1, :, None, None] * h_prev.float()).to(h_final.dtype)
    return corrected, h


def chunk_state(x, B, e, cum_A, t0=None):
    """Final SSM state of a shard's scan from a zero state (``final`` of mamba.py:113-141;
    per document the state of the last segment, :120-141): the SSD recurrence of
    ``ssd_reference`` unrolled,
    ``S[b,h] = sum_{t >= t0[b]} exp(cum_A[b,T-1,h] - cum_A[b,t,h]) e[b,t,h] x[b,t,h] (x) B[b,t,g]``
    with ``cum_A = cumsum(A e)``. x [b,T,H,d], B [b,T,G,n], e / cum_A [b,T,H], t0 [b]
    (first token of each row's last document) or None. Returns [b,H,d,n]."""
    bsz, T, H, _ = x.shape
    G = B.shape[2]
    w = torch.exp(cum_A[:, -1:, :] - cum_A) * e
    if t0 is not None:
        keep = torch.arange(T)[None, :] >= torch.as_tensor(t0).reshape(bsz, 1)
        w = w * keep[:, :, None].to(w.dtype)
    Bx = B.repeat_interleave(H // G, dim=2)
    return torch.einsum("bth,bthd,bthn->bhdn", w, x, Bx)


def effective_dt(dt, dt_bias=None, dt_softplus=False, dt_limit=(0.0, float("inf"))):
    """The per-token step the shard's own scan uses (mamba.py:143-148, mamba-ssm's rule):
    dt + dt_bias whenever dt_bias is given, then softplus when dt_softplus, then clamped
    to dt_limit. (The CP wrapper's chunk decay, ``chunk_decay`` below, has its own rule.)"""
    e = dt if dt_bias is None else dt + dt_bias
    if dt_softplus:
        e = torch.nn.functional.softplus(e)
    return e.clamp(*dt_limit)


def chunk_decay(dt, A, dt_bias=None, dt_softplus=False):
    """cum_A and the chunk decay of the CP scan wrapper (strategies/mamba.py:276-283):
    dt_eff = softplus(dt + dt_bias) when dt_softplus (dt_bias is then optional), else dt;
    cum_A = cumsum(A dt_eff) over T; decay = exp(cum_A[:, -1]). dt [b, T, H], A [H]."""
    if dt_softplus:
        dt_eff = torch.nn.functional.softplus(dt + (dt_bias if dt_bias is not None else 0))
    else:
        dt_eff = dt
    cum_A = torch.cumsum(A[None, None, :] * dt_eff, dim=1)
    return cum_A, torch.exp(cum_A[:, -1])


def cp_scan_wrapper_emulated(outs, finals, dts, A, Cs, num_heads, head_dim, dt_bias=None,
                             dt_softplus=False, seq_idxs=None):
    """The correction of the reference's mamba_chunk_scan_combined wrapper
    (strategies/mamba.py:250-300) on every rank: chunk decay from dt, the cross-rank
    entering state (cp_state_prefix, :68-98; single hop for packed sequences, :94-95)
    and mamba2_cp_correction. outs [b, T, H*d], finals [b, H, d, n], dts [b, T, H],
    Cs [b, T, G, n] per rank. Returns per-rank (corrected out, corrected state)."""
    world = len(outs)
    cums, decays = zip(*[chunk_decay(dt, A, dt_bias, dt_softplus) for dt in dts])
    if seq_idxs is None:
        prefixes = cp_state_prefix_emulated(list(finals), list(decays))
    else:
        prefixes = [torch.zeros_like(finals[0])] + [finals[r - 1] for r in range(1, world)]
    return [mamba2_cp_correction(outs[r], finals[r], Cs[r], cums[r], prefixes[r], num_heads,
                                 head_dim, None if seq_idxs is None else seq_idxs[r])
            for r in range(world)]
