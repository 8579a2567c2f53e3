"""Emulated zigzag ring on the MI355X vs the CPU oracle ring (fp32), dense and packed."""

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, assert_f32_rel, bf16_pair

pytestmark = pytest.mark.gpu


def _stack_interface(full, world, half):
    """[1, S, H, d] fp32 -> per-rank interface [b, H, L, d] list and the stacked device tensor."""
    idx = [rm.zigzag_gidx(r, half, world) for r in range(world)]
    per = [full[:, i].transpose(1, 2).contiguous() for i in idx]
    dev = torch.stack(per).to(torch.bfloat16).cuda()
    return per, dev, idx


def _run_ring(world, half, hq, hkv, d=128, cu=None, seed=0):
    from ringmaster_amd.ring.zigzag import zigzag_ring_attention

    S = 2 * world * half
    qf, _ = bf16_pair((1, S, hq, d), seed + 1)
    kf, _ = bf16_pair((1, S, hkv, d), seed + 2)
    vf, _ = bf16_pair((1, S, hkv, d), seed + 3)
    dof, _ = bf16_pair((1, S, hq, d), seed + 4)
    qs, qd, idx = _stack_interface(qf, world, half)
    ks, kd, _ = _stack_interface(kf, world, half)
    vs, vd, _ = _stack_interface(vf, world, half)
    dos = [dof[:, i] for i in idx]
    dod = torch.stack(dos).to(torch.bfloat16).cuda()
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    cu_dev = None if cu is None else cu.cuda()
    out = zigzag_ring_attention(qd, kd, vd, scaling=None, cu_seqlens=cu_dev)
    out.backward(dod)
    torch.cuda.synchronize()
    ref_out, ref_lse = rm.zigzag_ring_forward(qs, ks, vs, cu_seqlens=cu)
    rdq, rdk, rdv = rm.zigzag_ring_backward(dos, qs, ks, vs, ref_out, ref_lse, cu_seqlens=cu)
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(qd.grad[r], rdq[r], f"dq rank {r}")
        assert_bf16_close(kd.grad[r], rdk[r], f"dk rank {r}")
        assert_bf16_close(vd.grad[r], rdv[r], f"dv rank {r}")
    return out


@pytest.mark.parametrize("world", [1, 2, 4, 8])
def test_dense_ring(world):
    _run_ring(world, half=64, hq=2, hkv=2)


def test_dense_ring_ragged_tiles():
    _run_ring(4, half=100, hq=2, hkv=2)


def test_dense_ring_gqa():
    _run_ring(4, half=96, hq=4, hkv=2)


@pytest.mark.parametrize("world", [2, 4])
def test_dense_ring_d64(world):
    """head_dim 64: the forward's merge epilogues (ACC_INIT / MERGE / FINAL) and the fp32
    gradient accumulation of both backward kernels at D=64 (checked on the fp32 results,
    see tests/test_gpu_configs.py)."""
    from tests.test_gpu_configs import _ring_vs_oracle

    _ring_vs_oracle(world, half=96, hq=4, hkv=2, d=64, seed=40)


@pytest.mark.parametrize("world", [2, 4])
def test_varlen_ring_d64(world):
    from tests.test_gpu_configs import _ring_vs_oracle

    half = 96
    cu = torch.tensor([0, 70, 130, 131, 300, 2 * world * half], dtype=torch.int32)
    _ring_vs_oracle(world, half=half, hq=4, hkv=1, d=64, cu=cu, seed=50)


@pytest.mark.parametrize("docs", [[300, 212], [100, 50, 250, 112], [512]])
def test_varlen_ring(docs):
    world, half = 2, 128
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()], dtype=torch.int32)
    assert cu[-1].item() == 2 * world * half
    _run_ring(world, half, hq=2, hkv=1, cu=cu)


def test_varlen_ring_p4():
    world, half = 4, 64
    cu = torch.tensor([0, 37, 200, 201, 390, 512], dtype=torch.int32)
    _run_ring(world, half, hq=2, hkv=2, cu=cu)


def test_ring_lse_matches_oracle():
    from ringmaster_amd.ring.zigzag import ring_forward

    world, half, H, d = 4, 64, 2, 128
    S = 2 * world * half
    qf, _ = bf16_pair((1, S, H, d), 31)
    kf, _ = bf16_pair((1, S, H, d), 32)
    vf, _ = bf16_pair((1, S, H, d), 33)
    qs, qd, _ = _stack_interface(qf, world, half)
    ks, kd, _ = _stack_interface(kf, world, half)
    vs, vd, _ = _stack_interface(vf, world, half)
    out, lse, out32 = ring_forward(qd, kd, vd, d ** -0.5)
    torch.cuda.synchronize()
    ref_out, ref_lse = rm.zigzag_ring_forward(qs, ks, vs)
    for r in range(world):
        assert_f32_rel(lse[r], ref_lse[r], f"lse rank {r}")
        # the fp32 out the backward's delta reads is the merged out before bf16 rounding
        assert_bf16_close(out32[r], ref_out[r], f"fp32 out rank {r}")
        assert torch.equal(out32[r].to(torch.bfloat16), out[r]), f"bf16(out32) != out rank {r}"


def test_one_rank_alone_matches_the_full_ring():
    """``only_ranks`` (the per-rank timing mode) launches one rank's blocks at that rank's own
    grid: its out / lse / fp32 out and its dQ must equal the batched ring's bit for bit."""
    from ringmaster_amd.ring.zigzag import ring_backward, ring_forward

    world, half, h, d = 4, 160, 2, 128
    L = 2 * half
    g = torch.Generator(device="cuda").manual_seed(11)
    mk = lambda *s: torch.randn(*s, generator=g, device="cuda").to(torch.bfloat16)  # noqa: E731
    q, k, v = mk(world, 1, h, L, d), mk(world, 1, h, L, d), mk(world, 1, h, L, d)
    dout = mk(world, 1, L, h, d)
    scale = d ** -0.5
    out, lse, out32 = ring_forward(q, k, v, scale)
    dq, _, _ = ring_backward(dout, q, k, v, out32, lse, scale)
    for r in range(world):
        o1, l1, a1 = ring_forward(q, k, v, scale, only_ranks={r})
        dq1, _, _ = ring_backward(dout, q, k, v, out32, lse, scale, only_ranks={r})
        torch.cuda.synchronize()
        assert torch.equal(o1[r], out[r]), f"out rank {r}"
        assert torch.equal(l1[r], lse[r]), f"lse rank {r}"
        assert torch.equal(a1[r], out32[r]), f"fp32 out rank {r}"
        assert torch.equal(dq1[r], dq[r]), f"dq rank {r}"
