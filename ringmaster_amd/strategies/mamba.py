"""Mamba2 context-parallel state passing on the MI355X (strategies/mamba.py:68-139).

Every rank runs the intra-chunk SSD on its shard from a zero state, which leaves
two things to fix up: the state entering the shard (the exact prefix of the
earlier ranks' chunk states) and that state's contribution to the shard's
outputs and final state. With the P ranks emulated on one GPU the rank axis is
a leading tensor axis:

* :func:`cp_state_prefix` — ``H_in_r = sum_{j<r} (prod_{j<k<r} A_k) B_j`` for all
  ranks at once, computed by the fp32 linear-scan kernel over the rank axis
  (the all-gather + local loop of ``cp_state_prefix``, strategies/mamba.py:68-98);
* :func:`mamba2_cp_correction` — ``y += C . (e^{cumA} H_in)`` and
  ``h_final += e^{cumA_last} H_in`` (strategies/mamba.py:101-139), one MFMA kernel
  over every (batch, head) and token.
"""

from __future__ import annotations

import torch

from ringmaster_amd import abi
from ringmaster_amd.strategies.state_passing import linear_scan_forward


def cp_state_prefix(ssm_states: torch.Tensor, chunk_decays: torch.Tensor, *,
                    single_hop: bool = False) -> torch.Tensor:
    """State entering every rank's shard.

    ``ssm_states``: fp32 ``[world, b, nheads, head_dim, d_state]``, each rank's local
    final state (computed from h0 = 0); ``chunk_decays``: fp32 ``[world, b, nheads]``,
    each rank's chunk decay ``A_r = exp(sum_t A dt_t)``. Returns ``h_prev`` shaped like
    ``ssm_states`` (rank 0 receives zeros). ``single_hop`` keeps only the immediate
    predecessor (packed sequences), as the reference does."""
    abi.require_device(ssm_states, chunk_decays)
    if ssm_states.dim() != 5 or chunk_decays.shape != ssm_states.shape[:3]:
        raise ValueError("ssm_states must be [world, b, H, d, n] and chunk_decays [world, b, H]")
    if ssm_states.dtype != torch.float32 or chunk_decays.dtype != torch.float32:
        raise NotImplementedError("the MI355X state passing carries fp32 states")
    world, b, H = ssm_states.shape[:3]
    h_prev = torch.zeros_like(ssm_states)
    if world == 1:
        return h_prev
    if single_hop:
        h_prev[1:] = ssm_states[:-1]
        return h_prev
    # scan h_r = A_r h_{r-1} + B_r over the rank axis (one decay per head): then
    # H_in_r = h_{r-1}. Only ranks 0..world-2 feed a later rank.
    a = chunk_decays[:-1].permute(1, 0, 2).contiguous()                       # [b, world-1, H]
    bst = ssm_states[:-1].permute(1, 0, 2, 3, 4).reshape(b, world - 1, -1).contiguous()
    h = linear_scan_forward(a, bst, 1)                                         # [b, world-1, H*d*n]
    h_prev[1:] = h.reshape(b, world - 1, *ssm_states.shape[2:]).transpose(0, 1)
    return h_prev


def mamba2_cp_correction(out: torch.Tensor, h_final: torch.Tensor, C: torch.Tensor,
                         cum_A: torch.Tensor, h_prev: torch.Tensor, num_heads: int,
                         head_dim: int, seq_idx: torch.Tensor | None = None):
    """Add the carried-in state's contribution to a shard's SSM output and final state.

    Same arguments and result as the reference (strategies/mamba.py:101-139):
    ``out`` bf16 ``[B, T, H*head_dim]``, ``h_final`` fp32 ``[B, H, head_dim, d_state]``,
    ``C`` bf16 ``[B, T, ngroups, d_state]``, ``cum_A`` fp32 ``[B, T, H]``, ``h_prev``
    fp32 like ``h_final``, ``seq_idx`` optional int ``[B, T]``. Returns
    ``(corrected_out, corrected_h_final)`` as new tensors. Emulated ranks can be
    stacked on the batch axis (each batch row carries its own ``h_prev``). Forward
    only: the autograd of the correction is not implemented here."""
    abi.require_device(out, h_final, C, cum_A, h_prev)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (out, h_final, C, cum_A, h_prev)):
        raise NotImplementedError("the MI355X Mamba2 correction is forward-only")
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
    sid = None
    if seq_idx is not None:
        if seq_idx.shape != (Bsz, T):
            raise ValueError("seq_idx must be [B, T]")
        abi.require_device(seq_idx)
        sid = seq_idx.to(torch.int32).contiguous()
    out_c, C_c, cum_c = out.contiguous(), C.contiguous(), cum_A.contiguous()
    hp_c, hf_c = h_prev.contiguous(), h_final.contiguous()
    y = torch.empty_like(out_c)
    hf_out = torch.empty_like(hf_c)
    abi.check(abi.lib().rmx_mamba2_cp_correction(
        out_c.data_ptr(), y.data_ptr(), hf_c.data_ptr(), hf_out.data_ptr(), C_c.data_ptr(),
        cum_c.data_ptr(), hp_c.data_ptr(), abi.ptr(sid), Bsz, T, num_heads, head_dim, G, n,
        abi.stream_of(out)))
    return y, hf_out
