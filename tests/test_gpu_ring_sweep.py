"""A seeded sweep of zigzag rings on the MI355X vs the oracle ring (fp32), dense and packed.

Each case draws the world size (1, 2, 3, 4 or 8 ranks), the zigzag chunk length (1 to 100
tokens: chunks far below one tile, ragged against every tile), GQA ratio, head dim (64, 96,
128, 256) and either the dense causal ring or packed documents with a random split of the
sequence (`ring/zigzag.py:70-254`), and checks every rank's out and dq / dk / dv against
``zigzag_ring_forward`` / ``zigzag_ring_backward``. Bars as in tests/test_gpu_sweep.py."""

import numpy as np
import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, bf16_pair, rel_l2

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        world = int(rng.choice([1, 2, 3, 4, 8]))
        half = int(rng.choice([1, 7, 33, 64, 100]))
        hkv = int(rng.choice([1, 2]))
        hq = hkv * int(rng.choice([1, 2, 4]))
        d = int(rng.choice([64, 96, 128, 256]))
        S = 2 * world * half
        docs = None
        if rng.random() < 0.5 and S > 2:
            cuts = np.sort(rng.choice(np.arange(1, S), size=int(rng.integers(1, min(6, S - 1) + 1)),
                                      replace=False))
            docs = [0, *cuts.tolist(), S]
        out.append((i, world, half, hq, hkv, d, docs))
    return out


def _id(c):
    i, world, half, hq, hkv, d, docs = c
    return f"{i}-P{world}-h{half}-{hq}:{hkv}-d{d}-{'docs' + str(len(docs) - 1) if docs else 'dense'}"


def _grad_close(got, ref, what):
    g, ref = got.detach().float().cpu(), ref.detach().float()
    assert torch.isfinite(g).all(), f"{what}: non-finite values"
    diff = (g - ref).abs()
    bar = (ref.abs() * 2.0 ** -6).clamp_min(2e-2)
    over = (diff / bar).max().item()
    if over >= 1:
        i = int((diff / bar).flatten().argmax())
        print(f"  {what}: worst element {i} ref {ref.flatten()[i].item():.4f} got "
              f"{g.flatten()[i].item():.4f} (|ref| max {ref.abs().max().item():.3f})", flush=True)
    rl = rel_l2(g, ref) if ref.abs().max().item() >= 1e-3 else 0.0
    assert over < 1 and rl < 1e-2, f"{what}: max-abs {diff.max().item():.3e} ({over:.2f} of the bar) rel-L2 {rl:.3e}"


@pytest.mark.parametrize("case", _cases(), ids=_id)
def test_ring_sweep(case):
    from ringmaster_amd.ring.zigzag import zigzag_ring_attention

    i, world, half, hq, hkv, d, docs = case
    print(f"case ring sweep {_id(case)} docs={docs}", flush=True)
    S = 2 * world * half
    cu = None if docs is None else torch.tensor(docs, dtype=torch.int32)
    idx = [rm.zigzag_gidx(r, half, world) for r in range(world)]

    def stack(full):
        per = [full[:, j].transpose(1, 2).contiguous() for j in idx]
        return per, torch.stack(per).to(torch.bfloat16).cuda()

    qf, _ = bf16_pair((1, S, hq, d), 500 + i)
    kf, _ = bf16_pair((1, S, hkv, d), 600 + i)
    vf, _ = bf16_pair((1, S, hkv, d), 700 + i)
    dof, _ = bf16_pair((1, S, hq, d), 800 + i)
    (qs, qd), (ks, kd), (vs, vd) = stack(qf), stack(kf), stack(vf)
    dos = [dof[:, j] for j in idx]
    dod = torch.stack(dos).to(torch.bfloat16).cuda()
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    out = zigzag_ring_attention(qd, kd, vd, scaling=None,
                                cu_seqlens=None if cu is None else cu.cuda())
    out.backward(dod)
    torch.cuda.synchronize()
    ref_out, ref_lse = rm.zigzag_ring_forward(qs, ks, vs, cu_seqlens=cu)
    rdq, rdk, rdv = rm.zigzag_ring_backward(dos, qs, ks, vs, ref_out, ref_lse, cu_seqlens=cu)
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        _grad_close(qd.grad[r], rdq[r], f"dq rank {r}")
        _grad_close(kd.grad[r], rdk[r], f"dk rank {r}")
        _grad_close(vd.grad[r], rdv[r], f"dv rank {r}")
