"""fp16 attention on the MI355X (v_mfma_f32_32x32x16_f16) vs the CPU oracle in fp32: the
provider contract's dtype (ring/kernels.py:52-78 computes in fp32 from any input dtype
and returns q.dtype), through the block provider, the Dao op pair, the emulated rings
and the standalone merge. Inputs hold fp16-representable values; the bar is the fp16
one of tests/gpu_util.py."""

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_f16_close, assert_f32_rel, f16_pair

pytestmark = pytest.mark.gpu


def _block(causal, hq, hkv, sq, sk, d, window=None, b=1, seed=0):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    print(f"case fp16 block causal={causal} hq={hq} hkv={hkv} sq={sq} sk={sk} d={d} "
          f"window={window}", flush=True)
    qf, qd = f16_pair((b, sq, hq, d), seed + 1)
    kf, kd = f16_pair((b, sk, hkv, d), seed + 2)
    vf, vd = f16_pair((b, sk, hkv, d), seed + 3)
    dof, dod = f16_pair((b, sq, hq, d), seed + 4)
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None, window=window)
    out.backward(dod)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and qd.grad.dtype == torch.float16
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None, window=window,
                                 flash=True)
    ref.backward(dof)
    assert_f16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_f16_close(qd.grad, qr.grad, "dq")
    assert_f16_close(kd.grad, kr.grad, "dk")
    assert_f16_close(vd.grad, vr.grad, "dv")


@pytest.mark.parametrize("causal,hq,hkv,sq,sk,d", [
    (True, 2, 2, 256, 256, 128),
    (False, 4, 1, 192, 320, 128),
    (True, 2, 2, 100, 300, 128),
    (True, 4, 2, 200, 200, 64),
    (False, 8, 2, 128, 64, 96),
])
def test_fp16_block(causal, hq, hkv, sq, sk, d):
    _block(causal, hq, hkv, sq, sk, d)


def test_fp16_block_window():
    _block(True, 4, 2, 400, 400, 128, window=(100, 0))
    _block(False, 4, 2, 256, 300, 128, window=(-1, 33))  # bounded on the right only


def test_fp16_dao_ops():
    from ringmaster_amd.ring.kernels import flash_ops

    fwd, bwd = flash_ops()
    qf, q = f16_pair((1, 192, 4, 128), 11)
    kf, k = f16_pair((1, 192, 2, 128), 12)
    vf, v = f16_pair((1, 192, 2, 128), 13)
    dof, do = f16_pair((1, 192, 4, 128), 14)
    out, lse, _, _ = fwd(q, k, v, 0.0, 0.125, True, -1, -1, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.0, 0.125, True, -1, -1, 0.0, None, False, None)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=True, scaling=0.125)
    ref.backward(dof)
    assert_f16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_f16_close(dq, qr.grad, "dq")
    assert_f16_close(dk, kr.grad, "dk")
    assert_f16_close(dv, vr.grad, "dv")


@pytest.mark.parametrize("cu", [None, [0, 100, 300, 512]])
def test_fp16_zigzag_ring(cu):
    from ringmaster_amd.ring import zigzag_ring_attention

    world, L, hq, hkv, d = 4, 128, 4, 2, 128
    print(f"case fp16 zigzag world={world} L={L} docs={cu}", flush=True)
    cut = None if cu is None else torch.tensor(cu, dtype=torch.int32)
    per, dev = [], []
    for i, h in enumerate((hq, hkv, hkv)):
        ts = [f16_pair((1, h, L, d), 20 + 10 * i + r)[0] for r in range(world)]
        per.append(ts)
        dev.append(torch.stack(ts).to(torch.float16).cuda().requires_grad_(True))
    dos = [f16_pair((1, L, hq, d), 60 + r)[0] for r in range(world)]
    out = zigzag_ring_attention(*dev, cu_seqlens=None if cut is None else cut.cuda())
    out.backward(torch.stack(dos).to(torch.float16).cuda())
    torch.cuda.synchronize()
    ref_out, ref_lse = rm.zigzag_ring_forward(*per, cu_seqlens=cut)
    rdq, rdk, rdv = rm.zigzag_ring_backward(dos, *per, ref_out, ref_lse, cu_seqlens=cut)
    assert out.dtype == torch.float16
    for r in range(world):
        assert_f16_close(out[r], ref_out[r], f"out rank {r}")
        assert_f16_close(dev[0].grad[r], rdq[r], f"dq rank {r}")
        assert_f16_close(dev[1].grad[r], rdk[r], f"dk rank {r}")
        assert_f16_close(dev[2].grad[r], rdv[r], f"dv rank {r}")


def test_fp16_merge():
    from ringmaster_amd.ring.merge import update_out_and_lse

    b, s, h, d = 1, 64, 4, 128
    o1f, o1 = f16_pair((b, s, h, d), 70)
    o2f, o2 = f16_pair((b, s, h, d), 71)
    l1 = torch.randn(b, h, s, generator=torch.Generator().manual_seed(72))
    l2 = torch.randn(b, h, s, generator=torch.Generator().manual_seed(73))
    out, lse = update_out_and_lse(None, None, o1, l1.cuda())
    out, lse = update_out_and_lse(out, lse, o2, l2.cuda())
    torch.cuda.synchronize()
    ro, rl = rm.update_out_and_lse(None, None, o1f, l1)
    ro, rl = rm.update_out_and_lse(ro, rl, o2f, l2)
    assert_f32_rel(out, ro, "merged out")
    assert_f32_rel(lse, rl, "merged lse")
