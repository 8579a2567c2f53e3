"""Mamba2 CP state passing on the GPU: the rank-axis prefix (scan kernel) and the
output/state correction kernel against the oracle (strategies/mamba.py:68-139)."""

import math

import pytest
import torch

from oracle import state_passing as sp
from tests.gpu_util import BF16_REL_L2, assert_f32_rel, rel_l2, seeded

pytestmark = pytest.mark.gpu


def _inputs(Bsz, T, H, d, G, n, seed, strong_decay=False):
    out = seeded((Bsz, T, H * d), seed).to(torch.bfloat16)
    C = seeded((Bsz, T, G, n), seed + 1).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 2)
    if strong_decay:   # configs[4]: dt = softplus(N(0,1)), A = -exp(U(0, ln 16))
        A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
        dt = torch.nn.functional.softplus(torch.randn(Bsz, T, H, generator=g))
    else:              # the reference tests' weak decay: dt in [0, 0.1), A in (-1, 0]
        A = -torch.rand(H, generator=g)
        dt = torch.rand(Bsz, T, H, generator=g) * 0.1
    cum_A = torch.cumsum(A[None, None, :] * dt, dim=1).float()
    h_prev = seeded((Bsz, H, d, n), seed + 3)
    h_final = seeded((Bsz, H, d, n), seed + 4)
    return out, h_final, C, cum_A, h_prev


def _assert_y_close(y, ref_y, out):
    """y = bf16(out + bf16(dy)) may differ from the oracle only by the roundings of the
    fp32 product: rel-L2 within the bf16 bar and elementwise within 2^-6 of the size of
    the terms (|out| + |y|). (The correction reaches |y| ~ 40 at d_state = 128, where one
    bf16 step is 0.25, so the attention outputs' 2e-2 max-abs bar does not apply.)"""
    y, ref_y, out = y.float(), ref_y.float().to(y.device), out.float().to(y.device)
    assert torch.isfinite(y).all(), "y: non-finite values"
    rl = rel_l2(y, ref_y)
    assert rl < BF16_REL_L2, f"y: rel-L2 {rl:.3e}"
    scale = out.abs() + ref_y.abs() + 1e-6
    worst = ((y - ref_y).abs() / scale).max().item()
    assert worst <= 2.0 ** -6, f"y: elementwise error {worst:.3e} of the term size"


def _check(args, H, d, seq_idx=None):
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    out, h_final, C, cum_A, h_prev = args
    ref_y, ref_h = sp.mamba2_cp_correction(out, h_final, C, cum_A, h_prev, H, d, seq_idx=seq_idx)
    dev = [t.cuda() for t in args]
    y, hf = mamba2_cp_correction(*dev, H, d, seq_idx=None if seq_idx is None else seq_idx.cuda())
    torch.cuda.synchronize()
    y = y.cpu()
    _assert_y_close(y, ref_y, out)
    assert_f32_rel(hf, ref_h, "h_final")


# Streaming kernel (d_state <= 128, 4 units of min(d, 64) channels per workgroup in one
# C group): (200,4,64,1,128), (70,8,32,2,32), (300,4,128,2,64) (two units per head),
# (2100,4,64,1,16) (two 2048-token blocks, the second a ragged 52 tokens), (64,4,64,1,64) (two
# steps), (1,4,64,1,128) (one token). General kernel: (96,6,32,2,16), (130,2,128,2,64)
# (one head per group), (1,3,64,3,32), (40,2,64,1,256) (d_state 256).
@pytest.mark.parametrize("T,H,d,G,n", [(200, 4, 64, 1, 128), (70, 8, 32, 2, 32),
                                       (300, 4, 128, 2, 64), (2100, 4, 64, 1, 16),
                                       (64, 4, 64, 1, 64), (1, 4, 64, 1, 128),
                                       (96, 6, 32, 2, 16), (130, 2, 128, 2, 64),
                                       (1, 3, 64, 3, 32), (40, 2, 64, 1, 256)])
def test_correction_matches_oracle(T, H, d, G, n):
    _check(_inputs(2, T, H, d, G, n, seed=10), H, d)


@pytest.mark.parametrize("H,G", [(4, 1), (2, 2)])   # streaming kernel, general kernel
@pytest.mark.parametrize("fresh_last", [False, True])
def test_correction_seq_idx(fresh_last, H, G):
    Bsz, T, d, n = 2, 160, 64, 32
    args = _inputs(Bsz, T, H, d, G, n, seed=20)
    seq_idx = torch.zeros(Bsz, T, dtype=torch.int32)
    seq_idx[0, 70:] = 1                    # a new packed sequence starts at token 70
    if fresh_last:
        seq_idx[1, 150:] = 2               # and the last tokens of row 1 are a fresh one
    _check(args, H, d, seq_idx=seq_idx)


def test_correction_zero_prefix_is_identity():
    """Rank 0 (h_prev = 0): out and h_final pass through unchanged."""
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    out, h_final, C, cum_A, h_prev = _inputs(1, 64, 2, 64, 1, 16, seed=30)
    y, hf = mamba2_cp_correction(out.cuda(), h_final.cuda(), C.cuda(), cum_A.cuda(),
                                 torch.zeros_like(h_prev).cuda(), 2, 64)
    assert torch.equal(y.cpu(), out) and torch.equal(hf.cpu(), h_final)


def test_correction_configs4_full_size():
    """configs[4] shapes (8 shards stacked on the batch axis, 8192 tokens each,
    nheads=64, headdim=64, d_state=128, strong decay) against an fp32 torch
    reference of the same product on the GPU (the oracle's [B,T,H,d,n] temporary
    would need 137 GB)."""
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    Bsz, T, H, d, G, n = 8, 8192, 64, 64, 1, 128
    out, h_final, C, cum_A, h_prev = (t.cuda() for t in _inputs(Bsz, T, H, d, G, n, seed=40,
                                                                strong_decay=True))
    y, hf = mamba2_cp_correction(out, h_final, C, cum_A, h_prev, H, d)
    dy = torch.einsum("btn,bhdn->bthd", C[:, :, 0].float(), h_prev) * torch.exp(cum_A)[..., None]
    ref_y = out + dy.reshape(Bsz, T, H * d).to(torch.bfloat16)
    ref_h = h_final + torch.exp(cum_A[:, -1])[:, :, None, None] * h_prev
    torch.cuda.synchronize()
    _assert_y_close(y, ref_y, out)
    assert_f32_rel(hf, ref_h, "h_final")


@pytest.mark.parametrize("world", [1, 2, 5, 8])
def test_state_prefix_matches_oracle(world):
    from ringmaster_amd.strategies.mamba import cp_state_prefix_all

    b, H, d, n = 2, 4, 8, 16
    finals = seeded((world, b, H, d, n), 50)
    decays = torch.rand(world, b, H, generator=torch.Generator().manual_seed(51))
    ref = sp.cp_state_prefix_emulated(list(finals.double()), list(decays.double()))
    got = cp_state_prefix_all(finals.cuda(), decays.cuda()).cpu()
    for r in range(world):
        assert_f32_rel(got[r], ref[r], f"h_prev rank {r}")
    hop = cp_state_prefix_all(finals.cuda(), decays.cuda(), single_hop=True).cpu()
    assert torch.equal(hop[0], torch.zeros_like(hop[0]))
    for r in range(1, world):
        assert torch.equal(hop[r], finals[r - 1])


@pytest.mark.parametrize("single_hop", [False, True])
def test_state_prefix_per_rank_interface(single_hop):
    """The reference's per-rank return (strategies/mamba.py:68-98): every rank's
    ``(h_prev, zero_keep)`` from the gathered pairs; zero_keep a zero scalar on rank 0
    only, whose gradient reaches every gathered entry (as zeros); the single-rank call
    returns zeros."""
    from ringmaster_amd.strategies.mamba import cp_state_prefix, cp_state_prefix_gathered

    world, b, H, d, n = 5, 2, 3, 8, 16
    finals = seeded((world, b, H, d, n), 52).cuda()
    decays = torch.rand(world, b, H, generator=torch.Generator().manual_seed(53)).cuda()
    ref = sp.cp_state_prefix_emulated(list(finals.double().cpu()), list(decays.double().cpu()))
    for r in range(world):
        h_prev, keep = cp_state_prefix_gathered(finals, decays, r, single_hop=single_hop)
        want = (finals[r - 1].cpu() if r else torch.zeros_like(finals[0].cpu())) if single_hop \
            else ref[r]
        assert_f32_rel(h_prev.cpu(), want, f"h_prev rank {r}")
        if r == 0:
            assert keep.dim() == 0 and keep.item() == 0.0
        else:
            assert keep is None
    fs = finals.clone().requires_grad_(True)
    ds = decays.clone().requires_grad_(True)
    h_prev, keep = cp_state_prefix_gathered(fs, ds, 0, single_hop=single_hop)
    (h_prev.sum() + keep).backward()
    torch.cuda.synchronize()
    assert fs.grad is not None and not fs.grad.any() and ds.grad is not None
    h1, k1 = cp_state_prefix(finals[2], decays[2], single_hop=single_hop)
    assert torch.equal(h1, torch.zeros_like(h1)) and k1.item() == 0.0
    with pytest.raises(ValueError, match="rank"):
        cp_state_prefix_gathered(finals, decays, world)


# ---- backward: gradients of C, cum_A and h_prev against autograd through the oracle
# (the reference's torch ops, run in fp32 on the CPU). dC is bf16: rel-L2 within the
# bf16 bar and max error within 2^-7 of the largest |dC|; dcumA and dh_prev are fp32:
# the north-star 1e-4 relative bound (absolute below magnitude 1).

def _oracle_grads(args, H, d, gy, ghf, seq_idx=None):
    out, h_final, C, cum_A, h_prev = args
    Cf = C.float().requires_grad_(True)          # bf16 values held in fp32: unrounded dC
    ca = cum_A.clone().requires_grad_(True)
    hp = h_prev.clone().requires_grad_(True)
    y, hf = sp.mamba2_cp_correction(out, h_final, Cf, ca, hp, H, d, seq_idx=seq_idx)
    outs, gouts = [y], [gy]
    if ghf is not None and hf.requires_grad:
        outs.append(hf)
        gouts.append(ghf)
    return torch.autograd.grad(outs, (Cf, ca, hp), gouts, allow_unused=True)


def _check_bwd(args, H, d, seq_idx=None, with_ghf=True, seed=90):
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    out, h_final, C, cum_A, h_prev = args
    Bsz, T, _ = out.shape
    gy = seeded((Bsz, T, H * d), seed).to(torch.bfloat16)
    ghf = seeded(h_prev.shape, seed + 1) if with_ghf else None
    rC, rA, rH = _oracle_grads(args, H, d, gy, ghf, seq_idx)
    dC, dA, dH = (t.cuda().requires_grad_(True) for t in (C, cum_A, h_prev))
    y, hf = mamba2_cp_correction(out.cuda(), h_final.cuda(), dC, dA, dH, H, d,
                                 seq_idx=None if seq_idx is None else seq_idx.cuda())
    outs, gouts = [y], [gy.cuda()]
    if with_ghf:
        outs.append(hf)
        gouts.append(ghf.cuda())
    gC, gA, gH = torch.autograd.grad(outs, (dC, dA, dH), gouts)
    torch.cuda.synchronize()
    assert gC.dtype == torch.bfloat16 and gA.dtype == torch.float32 and gH.dtype == torch.float32
    gC = gC.float().cpu()
    assert torch.isfinite(gC).all()
    rl = rel_l2(gC, rC)
    worst = (gC - rC).abs().max().item() / rC.abs().max().clamp_min(1e-30).item()
    assert rl < BF16_REL_L2 and worst <= 2.0 ** -7, f"dC: rel-L2 {rl:.3e}, max err {worst:.3e}"
    assert_f32_rel(gA, rA, "dcumA")
    assert_f32_rel(gH, rH, "dh_prev")


@pytest.mark.parametrize("T,H,d,G,n", [(200, 4, 64, 1, 128), (300, 4, 128, 2, 64),
                                       (4500, 4, 64, 1, 64), (70, 8, 64, 2, 128),
                                       (33, 4, 128, 1, 128)])
def test_correction_backward_matches_oracle(T, H, d, G, n):
    _check_bwd(_inputs(2, T, H, d, G, n, seed=60), H, d)


@pytest.mark.parametrize("fresh_last", [False, True])
def test_correction_backward_seq_idx(fresh_last):
    Bsz, T, H, d, G, n = 2, 160, 4, 64, 1, 64
    seq_idx = torch.zeros(Bsz, T, dtype=torch.int32)
    seq_idx[0, 70:] = 1
    if fresh_last:
        seq_idx[1, 150:] = 2
    _check_bwd(_inputs(Bsz, T, H, d, G, n, seed=70), H, d, seq_idx=seq_idx)


def test_correction_backward_without_state_gradient():
    """Only y reaches the loss: no dL/dh_final_out (the kernels take a null pointer)."""
    _check_bwd(_inputs(2, 96, 4, 64, 1, 128, seed=80), 4, 64, with_ghf=False)


def test_correction_backward_zero_prefix_has_no_graph():
    """As in the reference, an all-zero h_prev returns (out, h_final) themselves."""
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    out, h_final, C, cum_A, h_prev = (t.cuda() for t in _inputs(1, 64, 4, 64, 1, 64, seed=85))
    C.requires_grad_(True)
    y, hf = mamba2_cp_correction(out, h_final, C, cum_A, torch.zeros_like(h_prev), 4, 64)
    assert y is out and hf is h_final


def test_correction_backward_unsupported_shape_raises_at_forward():
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    out, h_final, C, cum_A, h_prev = (t.cuda() for t in _inputs(1, 64, 4, 64, 1, 32, seed=86))
    C.requires_grad_(True)
    with pytest.raises(NotImplementedError, match="d_state"):
        mamba2_cp_correction(out, h_final, C, cum_A, h_prev, 4, 64)


def test_correction_backward_configs4_full_size():
    """configs[4] shapes against fp32 torch GPU formulas of the same gradients:
    dC = sum_{h,d} e G H_in, dcumA = e sum_d G S (+ the state term at T-1),
    dh_prev = sum_t e G C + e_last dh_final_out."""
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    Bsz, T, H, d, G, n = 8, 8192, 64, 64, 1, 128
    out, h_final, C, cum_A, h_prev = (t.cuda() for t in _inputs(Bsz, T, H, d, G, n, seed=95,
                                                                strong_decay=True))
    gy = seeded((Bsz, T, H * d), 96).to(torch.bfloat16).cuda()
    ghf = seeded(h_prev.shape, 97).cuda()
    dC, dA, dH = (t.clone().requires_grad_(True) for t in (C, cum_A, h_prev))
    y, hf = mamba2_cp_correction(out, h_final, dC, dA, dH, H, d)
    gC, gA, gH = torch.autograd.grad((y, hf), (dC, dA, dH), (gy, ghf))
    C0 = C[:, :, 0].float()
    e = torch.exp(cum_A)
    Gy = gy.float().reshape(Bsz, T, H, d)
    Ge = Gy * e[..., None]
    S = torch.einsum("btn,bhdn->bthd", C0, h_prev)
    rA = (Ge * S).sum(-1)
    rA[:, -1] += e[:, -1] * (ghf * h_prev).sum((-1, -2))
    rH = torch.einsum("bthd,btn->bhdn", Ge, C0) + e[:, -1, :, None, None] * ghf
    rC = torch.einsum("bthd,bhdn->btn", Ge, h_prev)
    torch.cuda.synchronize()
    rl = rel_l2(gC[:, :, 0].float(), rC)
    assert rl < BF16_REL_L2, f"dC rel-L2 {rl:.3e}"
    assert_f32_rel(gA, rA, "dcumA")
    assert_f32_rel(gH, rH, "dh_prev")
