"""Mamba2 context-parallel state passing on the MI355X (strategies/mamba.py:68-139).

Every rank runs the intra-chunk SSD on its shard from a zero state, which leaves
two things to fix up: the state entering the shard (the exact prefix of the
earlier ranks' chunk states) and that state's contribution to the shard's
outputs and final state. With the P ranks emulated on one GPU the rank axis is
a leading tensor axis:

* :func:`cp_state_prefix_all` — ``H_in_r = sum_{j<r} (prod_{j<k<r} A_k) B_j`` for all
  ranks at once, computed by the fp32 linear-scan kernel over the rank axis
  (the all-gather + local loop of ``cp_state_prefix``, strategies/mamba.py:68-98);
* :func:`mamba2_cp_correction` — ``y += C . (e^{cumA} H_in)`` and
  ``h_final += e^{cumA_last} H_in`` (strategies/mamba.py:101-139), one MFMA kernel
  over every (batch, head) and token.
"""

from __future__ import annotations

import torch

from ringmaster_amd import abi
from ringmaster_amd.strategies.state_passing import (_group_size, linear_scan_backward,
                                                     linear_scan_forward)


def _prefix_forward(ssm_states, chunk_decays, single_hop):
    world, b, H = ssm_states.shape[:3]
    h_prev = torch.zeros_like(ssm_states)
    if world == 1:
        return h_prev, None, None
    if single_hop:
        h_prev[1:] = ssm_states[:-1]
        return h_prev, None, None
    # scan h_r = A_r h_{r-1} + B_r over the rank axis (one decay per head): then
    # H_in_r = h_{r-1}. Only ranks 0..world-2 feed a later rank.
    a = chunk_decays[:-1].permute(1, 0, 2).contiguous()                       # [b, world-1, H]
    bst = ssm_states[:-1].permute(1, 0, 2, 3, 4).reshape(b, world - 1, -1).contiguous()
    h = linear_scan_forward(a, bst, 1)                                         # [b, world-1, H*d*n]
    h_prev[1:] = h.reshape(b, world - 1, *ssm_states.shape[2:]).transpose(0, 1)
    return h_prev, a, h


class _StatePrefix(torch.autograd.Function):
    """Differentiable like the reference's all-gather + torch prefix: the gradient of
    the rank-axis scan comes from the fp32 linear-scan backward kernel."""

    @staticmethod
    def forward(ctx, ssm_states, chunk_decays, single_hop):
        h_prev, a, h = _prefix_forward(ssm_states, chunk_decays, single_hop)
        ctx.single_hop = single_hop
        ctx.shape = ssm_states.shape
        ctx.save_for_backward(a, h)
        return h_prev

    @staticmethod
    def backward(ctx, g):
        a, h = ctx.saved_tensors
        world, b = ctx.shape[:2]
        g_states = torch.zeros(ctx.shape, dtype=torch.float32, device=g.device)
        g_decays = torch.zeros(ctx.shape[:3], dtype=torch.float32, device=g.device)
        if world > 1 and ctx.single_hop:
            g_states[:-1] = g[1:]
        elif world > 1:
            dh = g[1:].transpose(0, 1).reshape(b, world - 1, -1)
            da, db = linear_scan_backward(a, h, dh, 1)
            g_states[:-1] = db.reshape(b, world - 1, *ctx.shape[2:]).transpose(0, 1)
            g_decays[:-1] = da.permute(1, 0, 2)
        return g_states, g_decays, None


def cp_state_prefix_all(ssm_states: torch.Tensor, chunk_decays: torch.Tensor, *,
                        single_hop: bool = False) -> torch.Tensor:
    """State entering every rank's shard, all ranks at once (the P ranks emulated on one GPU).

    ``ssm_states``: fp32 ``[world, b, nheads, head_dim, d_state]``, each rank's local
    final state (computed from h0 = 0); ``chunk_decays``: fp32 ``[world, b, nheads]``,
    each rank's chunk decay ``A_r = exp(sum_t A dt_t)``. Returns ``h_prev`` shaped like
    ``ssm_states`` (rank 0 receives zeros). ``single_hop`` keeps only the immediate
    predecessor (packed sequences), as the reference does. Differentiable in both
    inputs."""
    abi.require_device(ssm_states, chunk_decays)
    if ssm_states.dim() != 5 or chunk_decays.shape != ssm_states.shape[:3]:
        raise ValueError("ssm_states must be [world, b, H, d, n] and chunk_decays [world, b, H]")
    if ssm_states.dtype != torch.float32 or chunk_decays.dtype != torch.float32:
        raise NotImplementedError("the MI355X state passing carries fp32 states")
    return _StatePrefix.apply(ssm_states, chunk_decays, bool(single_hop))


def _zero_keep(*tensors):
    """0 * the sum of the gathered values: the reference's rank 0 adds it to its output so
    that the all-gather stays in its graph and the gather's backward fires on every rank
    (strategies/mamba.py:85-86)."""
    return 0.0 * sum(t.float().sum() for t in tensors)


def cp_state_prefix_gathered(gathered_states: torch.Tensor, gathered_decays: torch.Tensor,
                             rank: int, *, single_hop: bool = False):
    """One rank's ``(h_prev, zero_keep)`` from the all-gathered pairs, what the reference
    computes after its all-gather (strategies/mamba.py:82-98): ``gathered_states``
    ``[world, b, nheads, head_dim, d_state]`` and ``gathered_decays`` ``[world, b,
    nheads]`` fp32, rank order. ``zero_keep`` is a zero-valued scalar on rank 0 and None
    elsewhere. A multi-process caller all-gathers (chunk decay, final state) itself and
    calls this with its rank."""
    world = gathered_states.shape[0] if gathered_states.dim() == 5 else 0
    if not 0 <= rank < max(world, 1):
        raise ValueError(f"rank {rank} outside the {world} gathered ranks")
    h_prev = cp_state_prefix_all(gathered_states, gathered_decays, single_hop=single_hop)[rank]
    return h_prev, (_zero_keep(gathered_states, gathered_decays) if rank == 0 else None)


def cp_state_prefix(ssm_state: torch.Tensor, chunk_decay: torch.Tensor, group=None, *,
                    single_hop: bool = False):
    """Drop-in for the reference's per-rank ``cp_state_prefix(ssm_state, chunk_decay,
    group, *, single_hop)`` (strategies/mamba.py:68-98): this rank's ``(h_prev,
    zero_keep)`` for its local final state ``ssm_state`` fp32 ``[b, nheads, head_dim,
    d_state]`` and chunk decay ``[b, nheads]``. A group of one rank (or None) is the
    reference's single-rank case: ``h_prev`` is zeros and ``zero_keep`` the zero scalar of
    rank 0. This one-GPU build runs no collectives, so a group of several ranks raises
    ``NotImplementedError``: gather the pairs and call :func:`cp_state_prefix_gathered`, or
    emulate every rank with :func:`cp_state_prefix_all`."""
    if _group_size(group, "cp_state_prefix(ssm_state, chunk_decay, group)",
                   "strategies/mamba.py:68", "cp_state_prefix_all") != 1:
        raise NotImplementedError(
            "the MI355X build runs no collectives: all-gather (chunk decay, state) and call "
            "cp_state_prefix_gathered, or emulate the ranks with cp_state_prefix_all")
    abi.require_device(ssm_state, chunk_decay)
    if ssm_state.dim() != 4 or chunk_decay.shape != ssm_state.shape[:2]:
        raise ValueError("ssm_state must be [b, H, d, n] and chunk_decay [b, H]")
    return cp_state_prefix_gathered(ssm_state[None], chunk_decay[None], 0, single_hop=single_hop)


class _DtCumsum(torch.autograd.Function):
    """(cum_A, decay, e) from dt; e (the effective dt) only when ``want_e``."""

    @staticmethod
    def forward(ctx, dt, A, dt_bias, softplus, want_e):
        rows, T, H = dt.shape
        cum = torch.empty((rows, T, H), dtype=torch.float32, device=dt.device)
        decay = torch.empty((rows, H), dtype=torch.float32, device=dt.device)
        e = torch.empty((rows, T, H) if want_e else (0,), dtype=torch.float32, device=dt.device)
        abi.check(abi.lib().rmx_mamba2_dt_cumsum(
            dt.data_ptr(), int(dt.dtype == torch.float32), abi.ptr(dt_bias), A.data_ptr(),
            int(softplus), cum.data_ptr(), e.data_ptr() if want_e else None, decay.data_ptr(),
            rows, T, H, abi.stream_of(dt)))
        ctx.save_for_backward(dt, A, dt_bias, decay)
        ctx.softplus = softplus
        ctx.set_materialize_grads(False)
        return cum, decay, e

    @staticmethod
    def backward(ctx, g_cum, g_decay, g_e):
        dt, A, dt_bias, decay = ctx.saved_tensors
        rows, T, H = dt.shape
        if g_cum is None and g_decay is None and g_e is None:
            return None, None, None, None, None
        g_cum = None if g_cum is None else g_cum.contiguous().float()
        g_decay = None if g_decay is None else g_decay.contiguous().float()
        g_e = None if g_e is None or g_e.numel() == 0 else g_e.contiguous().float()
        g_dt = torch.empty((rows, T, H), dtype=torch.float32, device=dt.device)
        g_A = torch.zeros(H, dtype=torch.float32, device=dt.device)
        g_b = torch.zeros(H, dtype=torch.float32, device=dt.device) if dt_bias is not None else None
        abi.check(abi.lib().rmx_mamba2_dt_cumsum_bwd(
            dt.data_ptr(), int(dt.dtype == torch.float32), abi.ptr(dt_bias), A.data_ptr(),
            int(ctx.softplus), abi.ptr(g_cum), abi.ptr(g_e), abi.ptr(g_decay), decay.data_ptr(),
            g_dt.data_ptr(), g_A.data_ptr(), abi.ptr(g_b), rows, T, H, abi.stream_of(dt)))
        return g_dt.to(dt.dtype), g_A, g_b, None, None


def mamba2_chunk_decay(dt: torch.Tensor, A: torch.Tensor, dt_bias: torch.Tensor | None = None,
                       dt_softplus: bool = False):
    """``cum_A = cumsum(A * dt_eff, dim=T)`` and the chunk decay ``exp(cum_A[:, -1])`` of
    the reference's CP scan wrapper (strategies/mamba.py:276-283), with
    ``dt_eff = softplus(dt + dt_bias)`` when ``dt_softplus`` (else ``dt``). ``dt``:
    ``[..., T, nheads]`` bf16 or fp32; ``A``, ``dt_bias``: ``[nheads]``. Returns fp32
    ``cum_A`` shaped like ``dt`` and ``decay`` ``[..., nheads]``; differentiable in dt, A
    and dt_bias. Computed in fp32 (the reference's arithmetic when dt_bias or dt is fp32,
    as HF's fp32 dt_bias parameter makes it)."""
    abi.require_device(dt, A, dt_bias)
    if dt.dim() < 2 or A.dim() != 1 or A.shape[0] != dt.shape[-1]:
        raise ValueError("dt must be [..., T, nheads] and A [nheads]")
    if dt.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("dt must be bf16 or fp32")
    lead, (T, H) = dt.shape[:-2], dt.shape[-2:]
    d3 = dt.reshape(-1, T, H).contiguous()
    A32 = A.float().contiguous()
    b32 = None
    if dt_softplus and dt_bias is not None:
        b32 = dt_bias.float().contiguous()
    cum, decay, _ = _DtCumsum.apply(d3, A32, b32, bool(dt_softplus), False)
    return cum.reshape(*lead, T, H), decay.reshape(*lead, H)


class _ChunkState(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, B, e, cum_A, t0):
        rows, T, H, D = x.shape
        G, N = B.shape[2], B.shape[3]
        state = torch.empty((rows, H, D, N), dtype=torch.float32, device=x.device)
        abi.check(abi.lib().rmx_mamba2_chunk_state(
            x.data_ptr(), B.data_ptr(), e.data_ptr(), cum_A.data_ptr(), abi.ptr(t0),
            state.data_ptr(), rows, T, H, D, G, N, abi.stream_of(x)))
        ctx.save_for_backward(x, B, e, cum_A, t0)
        return state

    @staticmethod
    def backward(ctx, g):
        x, B, e, cum_A, t0 = ctx.saved_tensors
        rows, T, H, D = x.shape
        G, N = B.shape[2], B.shape[3]
        g = g.contiguous().float()
        g_x, g_B = torch.empty_like(x), torch.empty_like(B)
        g_e = torch.empty((rows, T, H), dtype=torch.float32, device=x.device)
        g_cum = torch.empty_like(g_e)
        lib = abi.lib()
        ws_bytes = lib.rmx_mamba2_chunk_state_bwd_workspace(rows, H, D, N)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        abi.check(lib.rmx_mamba2_chunk_state_bwd(
            x.data_ptr(), B.data_ptr(), e.data_ptr(), cum_A.data_ptr(), abi.ptr(t0),
            g.data_ptr(), g_x.data_ptr(), g_B.data_ptr(), g_e.data_ptr(), g_cum.data_ptr(),
            rows, T, H, D, G, N, abi.ptr(ws), ws_bytes, abi.stream_of(x)))
        if T:
            # every weight exp(cum_A[T-1] - cum_A[t]) also depends on cum_A[T-1]
            g_cum[:, T - 1] = -g_cum[:, :T - 1].sum(1)
        return g_x, g_B, g_e, g_cum, None


def last_document_start(seq_idx: torch.Tensor) -> torch.Tensor:
    """First token of each row's last document (int32 [rows]) from per-token document
    ids ``[rows, T]``, on the device and without a synchronization."""
    T = seq_idx.shape[-1]
    pos = torch.arange(1, T + 1, device=seq_idx.device, dtype=torch.int32)
    return ((seq_idx != seq_idx[:, -1:]).to(torch.int32) * pos).amax(1).to(torch.int32)


def mamba2_chunk_state(x: torch.Tensor, dt: torch.Tensor, A: torch.Tensor, B: torch.Tensor, *,
                       dt_bias: torch.Tensor | None = None, dt_softplus: bool = False,
                       dt_limit: tuple = (0.0, float("inf")),
                       seq_idx: torch.Tensor | None = None) -> torch.Tensor:
    """Final SSM state of each shard's scan from a zero state: the ``final_states`` of
    mamba-ssm's ``mamba_chunk_scan_combined(..., return_final_states=True)`` that the
    reference's CP wrapper gathers across ranks (mamba.py:113-141 and :160-172;
    strategies/mamba.py:250-300). ``state[h] = sum_t exp(cum_A[T-1] - cum_A[t]) e_t
    x_t (x) B_t`` over the last document's tokens (all tokens when ``seq_idx`` is None),
    with the step of the shard's own scan (mamba.py:143-148): ``e = dt + dt_bias`` whenever
    ``dt_bias`` is given, then softplus when ``dt_softplus``, then clamped to ``dt_limit``;
    and ``cum_A = cumsum(A e)``. ``x`` bf16 ``[..., T, H, D]``, ``dt`` ``[..., T, H]``,
    ``A`` ``[H]``, ``B`` bf16 ``[..., T, G, N]``, ``seq_idx`` int ``[..., T]``; returns
    fp32 ``[..., H, D, N]``, differentiable in x, B, dt, A and dt_bias. D, N in {64, 128}."""
    abi.require_device(x, dt, A, B, dt_bias, seq_idx)
    if x.dim() < 3 or B.dim() != x.dim() or dt.dim() != x.dim() - 1:
        raise ValueError("x must be [..., T, H, D], B [..., T, G, N] and dt [..., T, H]")
    lead, (T, H, D) = x.shape[:-3], x.shape[-3:]
    G, N = B.shape[-2:]
    if tuple(B.shape[:-2]) != (*lead, T) or tuple(dt.shape) != (*lead, T, H):
        raise ValueError("x, dt and B disagree on the batch or token axes")
    if A.dim() != 1 or A.shape[0] != H or H % G:
        raise ValueError("A must be [nheads] and nheads a multiple of ngroups")
    if x.dtype != torch.bfloat16 or B.dtype != torch.bfloat16:
        raise NotImplementedError("the MI355X shard state takes bf16 x and B")
    if dt.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("dt must be bf16 or fp32")
    if D not in (64, 128) or N not in (64, 128):
        raise NotImplementedError("head_dim and d_state must be 64 or 128")
    x3 = x.reshape(-1, T, H, D).contiguous()
    B3 = B.reshape(-1, T, G, N).contiguous()
    d3 = dt.reshape(-1, T, H).contiguous()
    lo, hi = (float(v) for v in dt_limit)
    if dt_softplus and lo <= 0.0 and hi == float("inf"):
        # softplus >= 0, so the clamp is the identity: the dt kernel computes the step
        b32 = dt_bias.float().contiguous() if dt_bias is not None else None
        cum, _, e = _DtCumsum.apply(d3, A.float().contiguous(), b32, True, True)
    else:
        # a bias without softplus, or a clamp that bites: the step in fp32 elementwise
        # ops first (mamba.py:143-148), then the kernel's cumsum over it
        step = d3.float() if dt_bias is None else d3.float() + dt_bias.float()
        if dt_softplus:
            step = torch.nn.functional.softplus(step)
        step = step.clamp(lo, hi).contiguous()
        cum, _, e = _DtCumsum.apply(step, A.float().contiguous(), None, False, True)
    t0 = None
    if seq_idx is not None:
        if tuple(seq_idx.shape) != (*lead, T):
            raise ValueError("seq_idx must be [..., T]")
        t0 = last_document_start(seq_idx.reshape(-1, T))
    state = _ChunkState.apply(x3, B3, e, cum, t0)
    return state.reshape(*lead, H, D, N)


def mamba2_cp_apply(scan_output: torch.Tensor, ssm_state: torch.Tensor, dt: torch.Tensor,
                    A: torch.Tensor, C: torch.Tensor, *, dt_bias: torch.Tensor | None = None,
                    dt_softplus: bool = False, seq_idx: torch.Tensor | None = None):
    """The CP correction the reference's ``mamba_chunk_scan_combined`` wrapper applies
    (strategies/mamba.py:250-300) for every rank at once: chunk decay from dt, the exact
    cross-rank entering state (single hop for packed sequences) and the output / state
    correction. Ranks stacked on a leading axis: ``scan_output`` bf16 ``[P, B, T, H, d]``
    (or ``[P, B, T, H*d]``), ``ssm_state`` fp32 ``[P, B, H, d, n]`` (each shard's scan
    from a zero state), ``dt`` ``[P, B, T, H]``, ``A`` ``[H]``, ``C`` bf16
    ``[P, B, T, G, n]``, ``seq_idx`` int32 ``[P, B, T]`` or None. Returns the corrected
    ``(scan_output, ssm_state)``; differentiable like the reference's torch ops."""
    P, B = ssm_state.shape[:2]
    H, d, n = ssm_state.shape[2:]
    T = dt.shape[2]
    cum_A, decay = mamba2_chunk_decay(dt, A, dt_bias, dt_softplus)          # [P,B,T,H], [P,B,H]
    h_prev = cp_state_prefix_all(ssm_state, decay, single_hop=seq_idx is not None)
    if seq_idx is None:
        # every rank's rows in one launch, stacked on the batch axis
        y, h_final = mamba2_cp_correction(
            scan_output.reshape(P * B, T, H * d), ssm_state.reshape(P * B, H, d, n),
            C.reshape(P * B, T, *C.shape[3:]), cum_A.reshape(P * B, T, H),
            h_prev.reshape(P * B, H, d, n), H, d)
        return y.reshape(scan_output.shape), h_final.reshape(ssm_state.shape)
    # packed: the state update is skipped when the last token of any of a rank's batch
    # rows starts a fresh sequence (seq_idx[:, -1].any() per rank, strategies/mamba.py:131),
    # so each rank gets its own launch
    ys, hs = [], []
    for r in range(P):
        y, h = mamba2_cp_correction(scan_output[r].reshape(B, T, H * d), ssm_state[r], C[r],
                                    cum_A[r], h_prev[r], H, d, seq_idx=seq_idx[r])
        ys.append(y)
        hs.append(h)
    return torch.stack(ys).reshape(scan_output.shape), torch.stack(hs)


def _validate_correction(out, h_final, C, cum_A, h_prev, num_heads, head_dim, seq_idx):
    abi.require_device(out, h_final, C, cum_A, h_prev)
    if out.dtype != torch.bfloat16 or C.dtype != torch.bfloat16:
        raise NotImplementedError("the MI355X Mamba2 correction takes bf16 out and C")
    if h_final.dtype != torch.float32 or h_prev.dtype != torch.float32 or \
            cum_A.dtype != torch.float32:
        raise NotImplementedError("states and cum_A must be fp32")
    if out.dim() != 3 or C.dim() != 4 or cum_A.dim() != 3 or h_prev.dim() != 4:
        raise ValueError("expected out [B,T,H*d], C [B,T,G,n], cum_A [B,T,H], h_prev [B,H,d,n]")
    Bsz, T, HD = out.shape
    G, n = C.shape[2], C.shape[3]
    if HD != num_heads * head_dim or cum_A.shape != (Bsz, T, num_heads) or \
            C.shape[:2] != (Bsz, T) or h_prev.shape != (Bsz, num_heads, head_dim, n) or \
            h_final.shape != h_prev.shape:
        raise ValueError("shapes of out/C/cum_A/h_prev/h_final do not agree")
    if num_heads % G:
        raise ValueError(f"ngroups {G} must divide num_heads {num_heads}")
    if seq_idx is None:
        return None
    if seq_idx.shape != (Bsz, T):
        raise ValueError("seq_idx must be [B, T]")
    abi.require_device(seq_idx)
    return seq_idx.to(torch.int32).contiguous()


def _bwd_workspace_bytes(Bsz, T, H, d, G, n) -> int:
    nbytes = abi.lib().rmx_mamba2_cp_correction_bwd_workspace(Bsz, T, H, d, G, n)
    if nbytes == 0:
        raise NotImplementedError(
            "the MI355X Mamba2 correction backward does not take this shape: "
            + (abi.lib().rmx_last_error() or b"").decode(errors="replace"))
    return nbytes


class _Correction(torch.autograd.Function):
    """y = out + bf16(e C.H_in), h_final_out = h_final + e_last H_in, with the gradients
    autograd takes through the reference's torch ops (strategies/mamba.py:116-137):
    dout = dy and dh_final = dh_final_out unchanged; dC, dcumA and dh_prev from the
    backward kernels."""

    @staticmethod
    def forward(ctx, out, h_final, C, cum_A, h_prev, num_heads, head_dim, sid):
        Bsz, T, _ = out.shape
        G, n = C.shape[2], C.shape[3]
        out_c, C_c, cum_c = out.contiguous(), C.contiguous(), cum_A.contiguous()
        hp_c, hf_c = h_prev.contiguous(), h_final.contiguous()
        y = torch.empty_like(out_c)
        hf_out = torch.empty_like(hf_c)
        abi.check(abi.lib().rmx_mamba2_cp_correction(
            out_c.data_ptr(), y.data_ptr(), hf_c.data_ptr(), hf_out.data_ptr(), C_c.data_ptr(),
            cum_c.data_ptr(), hp_c.data_ptr(), abi.ptr(sid), Bsz, T, num_heads, head_dim, G, n,
            abi.stream_of(out)))
        ctx.save_for_backward(C_c, cum_c, hp_c, sid)
        ctx.meta = (num_heads, head_dim)
        return y, hf_out

    @staticmethod
    def backward(ctx, gy, ghf):
        C, cum_A, h_prev, sid = ctx.saved_tensors
        num_heads, head_dim = ctx.meta
        need = ctx.needs_input_grad
        gC = g_cumA = g_hprev = None
        if need[2] or need[3] or need[4]:
            Bsz, T = C.shape[:2]
            G, n = C.shape[2], C.shape[3]
            if gy is None:
                gy = torch.zeros((Bsz, T, num_heads * head_dim), dtype=torch.bfloat16,
                                 device=C.device)
            gy_c = gy.to(torch.bfloat16).contiguous()
            ghf_c = None if ghf is None else ghf.to(torch.float32).contiguous()
            nbytes = _bwd_workspace_bytes(Bsz, T, num_heads, head_dim, G, n)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=C.device)
            gC = torch.empty_like(C)
            g_cumA = torch.empty_like(cum_A)
            g_hprev = torch.empty_like(h_prev)
            abi.check(abi.lib().rmx_mamba2_cp_correction_bwd(
                gy_c.data_ptr(), abi.ptr(ghf_c), C.data_ptr(), cum_A.data_ptr(), h_prev.data_ptr(),
                abi.ptr(sid), gC.data_ptr(), g_cumA.data_ptr(), g_hprev.data_ptr(), ws.data_ptr(),
                nbytes, Bsz, T, num_heads, head_dim, G, n, abi.stream_of(C)))
        return gy, ghf, gC, g_cumA, g_hprev, None, None, None


def mamba2_cp_correction(out: torch.Tensor, h_final: torch.Tensor, C: torch.Tensor,
                         cum_A: torch.Tensor, h_prev: torch.Tensor, num_heads: int,
                         head_dim: int, seq_idx: torch.Tensor | None = None):
    """Add the carried-in state's contribution to a shard's SSM output and final state.

    Same arguments, result and autograd as the reference (strategies/mamba.py:101-139):
    ``out`` bf16 ``[B, T, H*head_dim]``, ``h_final`` fp32 ``[B, H, head_dim, d_state]``,
    ``C`` bf16 ``[B, T, ngroups, d_state]``, ``cum_A`` fp32 ``[B, T, H]``, ``h_prev``
    fp32 like ``h_final``, ``seq_idx`` optional int ``[B, T]``. Returns
    ``(corrected_out, corrected_h_final)``; like the reference, an all-zero ``h_prev``
    returns ``(out, h_final)`` themselves (no graph to ``C``, ``cum_A``, ``h_prev``).
    Emulated ranks can be stacked on the batch axis (each batch row carries its own
    ``h_prev``). The backward takes head_dim 64 or 128 and d_state 64 or 128 (the
    forward any of the kernel's shapes); a graph that needs an unsupported backward
    fails here, at the forward, with NotImplementedError."""
    sid = _validate_correction(out, h_final, C, cum_A, h_prev, num_heads, head_dim, seq_idx)
    if not h_prev.any():
        return out, h_final
    if torch.is_grad_enabled() and any(t.requires_grad for t in (out, h_final, C, cum_A, h_prev)):
        Bsz, T, _ = out.shape
        _bwd_workspace_bytes(Bsz, T, num_heads, head_dim, C.shape[2], C.shape[3])
    return _Correction.apply(out, h_final, C, cum_A, h_prev, num_heads, head_dim, sid)


# ---------------------------------------------------------------- CP causal conv1d
_ACTIVATIONS = {None: 0, "silu": 1, "swish": 1}


class _CausalConv1dCP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, doc, act):
        y = torch.empty_like(x)
        P, B, C, L = x.shape
        abi.check(abi.lib().rmx_causal_conv1d_cp(
            x.data_ptr(), weight.data_ptr(), abi.ptr(bias), abi.ptr(doc), y.data_ptr(),
            P, B, C, L, weight.shape[1], act, abi.stream_of(x)))
        ctx.save_for_backward(x, weight, bias, doc)
        ctx.act = act
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, bias, doc = ctx.saved_tensors
        P, B, C, L = x.shape
        dy = dy.contiguous()
        dx = torch.empty_like(x)
        dw = torch.zeros(weight.shape, dtype=torch.float32, device=x.device)
        db = torch.zeros(C, dtype=torch.float32, device=x.device) if bias is not None else None
        abi.check(abi.lib().rmx_causal_conv1d_cp_bwd(
            x.data_ptr(), weight.data_ptr(), abi.ptr(bias), abi.ptr(doc), dy.data_ptr(),
            dx.data_ptr(), dw.data_ptr(), abi.ptr(db), P, B, C, L, weight.shape[1], ctx.act,
            abi.stream_of(x)))
        return (dx, dw.to(weight.dtype), None if db is None else db.to(bias.dtype), None, None)


def causal_conv1d_cp(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                     activation: str | None = None, cu_seqlens: torch.Tensor | None = None):
    """The Mamba2 CP convolution of the reference adapter (mamba.py:46-101) for every
    rank at once: ``x`` bf16 ``[world, batch, channels, local_len]`` (each rank's
    channels-first shard, as ``causal_conv1d_fn`` takes it), ``weight`` ``[channels,
    width]`` (or ``[channels, 1, width]``), ``bias`` ``[channels]`` or None, ``activation``
    None / "silu" / "swish". Shard r's first width-1 outputs read shard r-1's last tokens
    (the halo; zeros for rank 0); with ``cu_seqlens`` taps never cross a document
    boundary. Differentiable in x, weight and bias. Returns ``[world, batch, channels,
    local_len]``."""
    abi.require_device(x, weight, bias)
    if weight.dim() == 3 and weight.shape[1] == 1:
        weight = weight[:, 0]
    if x.dim() != 4 or weight.dim() != 2 or weight.shape[0] != x.shape[2]:
        raise ValueError("x must be [world, batch, channels, len] and weight [channels, width]")
    if bias is not None and bias.shape != (x.shape[2],):
        raise ValueError("bias must be [channels]")
    if activation not in _ACTIVATIONS:
        raise NotImplementedError(f"activation {activation!r}")
    width = weight.shape[1] - 1
    if x.shape[3] < width:
        raise ValueError("Mamba CP shards must be at least convolution width - 1 tokens")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or (
            bias is not None and bias.dtype != torch.bfloat16):
        raise NotImplementedError("the MI355X conv computes bf16 tensors")
    doc = None
    if cu_seqlens is not None:
        from ringmaster_amd.ring.zigzag import doc_ids_from_cu

        # the reference reshapes the ids of the packed batch to [batch, world * len]
        doc = doc_ids_from_cu(cu_seqlens, x.device)
        n = x.shape[0] * x.shape[3]
        if doc.numel() == x.shape[1] * n:
            doc = doc.reshape(x.shape[1], n)
        elif doc.numel() == n:
            doc = doc.reshape(1, n).expand(x.shape[1], n)
        else:
            raise ValueError("cu_seqlens must cover the full (padded) sequence")
        doc = doc.contiguous()
    x = x.contiguous()
    weight = weight.contiguous()
    bias = None if bias is None else bias.contiguous()
    return _CausalConv1dCP.apply(x, weight, bias, doc, _ACTIVATIONS[activation])
