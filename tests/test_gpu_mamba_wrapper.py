"""The Mamba2 CP scan wrapper on the GPU (strategies/mamba.py:250-300): the chunk decay
from dt (rmx_mamba2_dt_cumsum and its backward), the differentiable rank-axis prefix,
and their composition with the correction, against the oracle restatement and
autograd through it."""

import pytest
import torch

from oracle import state_passing as sp
from tests.gpu_util import BF16_REL_L2, assert_f32_rel, rel_l2, seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("softplus,dt_f32,H", [(True, False, 64), (False, True, 8),
                                              (True, True, 130)])
def test_chunk_decay_values_and_grads(softplus, dt_f32, H):
    from ringmaster_amd.strategies.mamba import mamba2_chunk_decay

    print(f"case softplus={softplus} dt_f32={dt_f32} H={H}", flush=True)
    R, T = 3, 777
    g = torch.Generator().manual_seed(3)
    dt = (torch.randn(R, T, H, generator=g) - 1.0).to(torch.float32 if dt_f32 else torch.bfloat16)
    A = -0.01 * torch.exp(torch.rand(H, generator=g))   # decay exp(cum_A) stays ~1e-2
    bias = torch.randn(H, generator=g) * 0.5
    gc = seeded((R, T, H), 5) * 0.01
    gdec = seeded((R, H), 6)
    dtr, Ar, br = (t.double().requires_grad_(True) for t in (dt.float(), A, bias))
    cum_r, dec_r = sp.chunk_decay(dtr, Ar, br if softplus else None, softplus)
    (cum_r * gc.double()).sum().add((dec_r * gdec.double()).sum()).backward()
    dtd, Ad, bd = dt.cuda().requires_grad_(True), A.cuda().requires_grad_(True), \
        bias.cuda().requires_grad_(True)
    cum, dec = mamba2_chunk_decay(dtd, Ad, bd, softplus)
    torch.autograd.backward((cum, dec), (gc.cuda(), gdec.cuda()))
    torch.cuda.synchronize()
    assert_f32_rel(cum, cum_r, "cum_A")
    assert_f32_rel(dec, dec_r, "decay")
    ref_gdt = dtr.grad if dt_f32 else dtr.grad.to(torch.bfloat16).double()
    tol = 1e-4 if dt_f32 else 2.0 ** -8   # bf16 dt gets a bf16 gradient
    assert_f32_rel(dtd.grad.double(), ref_gdt, "g_dt", tol=tol)
    assert_f32_rel(Ad.grad, Ar.grad, "g_A")
    if softplus:
        assert_f32_rel(bd.grad, br.grad, "g_dt_bias")
    else:
        assert bd.grad is None


@pytest.mark.parametrize("single_hop", [False, True])
def test_state_prefix_grads(single_hop):
    from ringmaster_amd.strategies.mamba import cp_state_prefix_all

    P, b, H, d, n = 4, 2, 3, 8, 16
    states = seeded((P, b, H, d, n), 7)
    decays = torch.rand(P, b, H, generator=torch.Generator().manual_seed(8)) * 0.9 + 0.05
    gout = seeded((P, b, H, d, n), 9)
    sr, dr = states.double().requires_grad_(True), decays.double().requires_grad_(True)
    if single_hop:
        ref = torch.stack([torch.zeros_like(sr[0])] + [sr[r - 1] for r in range(1, P)])
    else:
        ref = torch.stack(sp.cp_state_prefix_emulated(list(sr.unbind(0)), list(dr.unbind(0))))
    (ref * gout.double()).sum().backward()
    sd, dd = states.cuda().requires_grad_(True), decays.cuda().requires_grad_(True)
    got = cp_state_prefix_all(sd, dd, single_hop=single_hop)
    got.backward(gout.cuda())
    torch.cuda.synchronize()
    assert_f32_rel(got, ref, "h_prev")
    assert_f32_rel(sd.grad, sr.grad, "g_states")
    if single_hop:  # the single-hop prefix does not depend on the decays
        assert dr.grad is None and not dd.grad.any()
    else:
        assert_f32_rel(dd.grad, dr.grad, "g_decays")


@pytest.mark.parametrize("seq", [False, True])
def test_cp_apply_matches_wrapper_oracle(seq):
    from ringmaster_amd.strategies.mamba import mamba2_cp_apply

    P, B, T, H, d, G, n = 4, 1, 96, 4, 64, 1, 64
    print(f"case P={P} T={T} H={H} d={d} n={n} seq_idx={seq}", flush=True)
    g = torch.Generator().manual_seed(11)
    out = seeded((P, B, T, H * d), 12).to(torch.bfloat16)
    states = seeded((P, B, H, d, n), 13)
    dt = (torch.randn(P, B, T, H, generator=g) - 2.0).to(torch.bfloat16)
    A = -torch.rand(H, generator=g) - 0.05
    bias = torch.randn(H, generator=g) * 0.1
    C = seeded((P, B, T, G, n), 14).to(torch.bfloat16)
    sid = None
    if seq:
        sid = torch.zeros(P, B, T, dtype=torch.int32)
        sid[2, :, 40:] = 1                   # rank 2 starts a new packed sequence at token 40
    gy = seeded((P, B, T, H * d), 15).to(torch.bfloat16).float()  # y is bf16: so is dL/dy
    gh = seeded((P, B, H, d, n), 16)
    # oracle (fp64 where it computes in the caller's dtype) with autograd
    Cr = C.double().requires_grad_(True)
    dtr, Ar, br = (t.double().requires_grad_(True) for t in (dt.float(), A, bias))
    sr = states.double().requires_grad_(True)
    res = sp.cp_scan_wrapper_emulated(
        list(out.double().unbind(0)), list(sr.unbind(0)), list(dtr.unbind(0)), Ar,
        list(Cr.unbind(0)), H, d, dt_bias=br, dt_softplus=True,
        seq_idxs=None if sid is None else list(sid.unbind(0)))
    ref_y = torch.stack([y for y, _ in res])
    ref_h = torch.stack([h for _, h in res])
    ((ref_y * gy.double()).sum() + (ref_h * gh.double()).sum()).backward()
    # product
    dev = dict(C=C.cuda().requires_grad_(True), dt=dt.cuda().requires_grad_(True),
               A=A.cuda().requires_grad_(True), bias=bias.cuda().requires_grad_(True),
               states=states.cuda().requires_grad_(True))
    y, h = mamba2_cp_apply(out.cuda(), dev["states"], dev["dt"], dev["A"], dev["C"],
                           dt_bias=dev["bias"], dt_softplus=True,
                           seq_idx=None if sid is None else sid.cuda())
    torch.autograd.backward((y, h), (gy.cuda().to(torch.bfloat16), gh.cuda()))
    torch.cuda.synchronize()
    yc, ryc = y.float().cpu(), ref_y.float()
    assert rel_l2(yc, ryc) < BF16_REL_L2, "y"
    assert ((yc - ryc).abs() / (out.float().abs() + ryc.abs() + 1e-6)).max().item() <= 2.0 ** -6
    assert_f32_rel(h, ref_h, "h_final")
    assert rel_l2(dev["C"].grad.float().cpu(), Cr.grad.float()) < BF16_REL_L2, "dC"
    assert_f32_rel(dev["states"].grad, sr.grad, "d ssm_state", tol=1e-3)
    assert_f32_rel(dev["A"].grad, Ar.grad, "dA", tol=1e-3)
    assert_f32_rel(dev["bias"].grad, br.grad, "d dt_bias", tol=1e-3)
    assert rel_l2(dev["dt"].grad.float().cpu(), dtr.grad.float()) < BF16_REL_L2, "d dt"
