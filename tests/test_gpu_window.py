"""Sliding windows and head dims other than 64/128 on the MI355X vs the CPU oracle (fp32).

The provider contract's ``window`` on single blocks and through the Dao op pair: flash
attention's ``window_size = (left, right)`` (the flash provider passes it on,
ring/kernels.py:37-38; ``pos_q - pos_k > left`` and ``pos_k - pos_q > right`` masked,
bottom-right aligned, causal calls bounded at right = 0; the oracle is ``math_block`` with
``flash=True``, which reads ``left`` as ring/kernels.py:68-72 does), the gather ring and
the packed gather ring with windows (ring/loop.py:175-228), and head dims that are
multiples of 8 up to 128 (the kernels compute at 64 or 128 and read the columns past
head_dim as zeros; head dims above 128: tests/test_gpu_head256.py)."""

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, assert_f32_rel, bf16_pair, keyless_prefix

pytestmark = pytest.mark.gpu


def _block(causal, hq, hkv, sq, sk, d, window, b=1, seed=0):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    print(f"case block causal={causal} hq={hq} hkv={hkv} sq={sq} sk={sk} d={d} "
          f"window={window}", flush=True)
    qf, qd = bf16_pair((b, sq, hq, d), seed + 1)
    kf, kd = bf16_pair((b, sk, hkv, d), seed + 2)
    vf, vd = bf16_pair((b, sk, hkv, d), seed + 3)
    dof, dod = bf16_pair((b, sq, hq, d), seed + 4)
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None, window=window)
    out.backward(dod)
    torch.cuda.synchronize()
    s0 = keyless_prefix(sq, sk, causal, window)
    assert torch.isneginf(lse[:, :, :s0].cpu()).all(), "rows without keys: lse"
    assert not out[:, :s0].float().abs().sum().item(), "rows without keys: out"
    assert not qd.grad[:, :s0].float().abs().sum().item(), "rows without keys: dq"
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf[:, s0:], kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None, window=window,
                                 flash=True)
    ref.backward(dof[:, s0:])
    assert_bf16_close(out[:, s0:], ref, "out")
    assert_f32_rel(lse[:, :, s0:], ref_lse, "lse")
    assert_bf16_close(qd.grad[:, s0:], qr.grad, "dq")
    assert_bf16_close(kd.grad, kr.grad, "dk", ulp_floor=hq != hkv)
    assert_bf16_close(vd.grad, vr.grad, "dv", ulp_floor=hq != hkv)


@pytest.mark.parametrize("causal,hq,hkv,sq,sk,d,left,right", [
    (True, 2, 2, 300, 300, 128, 64, 0),     # the window's edge crosses key tiles
    (True, 4, 2, 200, 517, 64, 100, 0),     # bottom-right aligned, sq < sk
    (False, 2, 1, 256, 256, 128, 17, -1),   # non-causal: only the left edge
    (True, 2, 2, 1100, 1100, 128, 255, 0),  # whole key tiles below the window skipped
    (False, 4, 4, 320, 96, 128, 40, -1),    # sk < sq: flash bounds the right at sk keys
    (False, 2, 1, 256, 256, 128, 17, 0),    # non-causal (17, 0): the causal band
    (False, 4, 4, 320, 96, 128, 40, 0),     # sk < sq, right 0: the first 224 rows keyless
])
def test_block_window(causal, hq, hkv, sq, sk, d, left, right):
    _block(causal, hq, hkv, sq, sk, d, (left, right))


def test_block_window_zero_attends_itself():
    """A causal window of 0 on a square block: each query sees only its own key, so
    out = v, lse = scale q.k, dv = dout and dq = dk = 0 (dS = P (dP - delta) with P = 1
    and delta = dout.v = dP)."""
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    qf, q = bf16_pair((1, 256, 2, 128), 8)
    kf, k = bf16_pair((1, 256, 2, 128), 9)
    vf, v = bf16_pair((1, 256, 2, 128), 10)
    dof, do = bf16_pair((1, 256, 2, 128), 11)
    for t in (q, k, v):
        t.requires_grad_(True)
    out, lse = mi355x_hip_block(q, k, v, causal=True, scaling=0.1, window=(0, 0))
    out.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), v.detach().cpu())
    assert_f32_rel(lse, 0.1 * (qf * kf).sum(-1).transpose(1, 2), "lse")
    assert torch.equal(v.grad.cpu(), do.cpu())
    assert q.grad.abs().max().item() < 1e-4 and k.grad.abs().max().item() < 1e-4


def test_block_window_covering_everything_is_no_window():
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    _, q = bf16_pair((1, 200, 2, 128), 5)
    _, k = bf16_pair((1, 200, 2, 128), 6)
    _, v = bf16_pair((1, 200, 2, 128), 7)
    a, la = mi355x_hip_block(q, k, v, causal=True, scaling=None, window=(199, 0))
    b, lb = mi355x_hip_block(q, k, v, causal=True, scaling=None)
    c, lc = mi355x_hip_block(q, k, v, causal=True, scaling=None, window=(-1, -1))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)
    assert torch.equal(c, b) and torch.equal(lc, lb)


@pytest.mark.parametrize("d", [8, 32, 48, 80, 96, 112])
def test_block_head_dims(d):
    _block(True, 4, 2, 230, 230, d, None)


def test_block_head_dim_96_window_gqa_batch2():
    _block(False, 6, 2, 190, 260, 96, (70, 0), b=2)


def test_dao_ops_window():
    from ringmaster_amd.ring.kernels import flash_ops

    fwd, bwd = flash_ops()
    qf, q = bf16_pair((1, 300, 4, 128), 11)
    kf, k = bf16_pair((1, 300, 2, 128), 12)
    vf, v = bf16_pair((1, 300, 2, 128), 13)
    dof, do = bf16_pair((1, 300, 4, 128), 14)
    out, lse, _, _ = fwd(q, k, v, 0.0, 0.125, True, 90, 0, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.0, 0.125, True, 90, 0, 0.0, None, False, None)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=True, scaling=0.125, window=(90, 0),
                                 flash=True)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(dq, qr.grad, "dq")
    assert_bf16_close(dk, kr.grad, "dk", ulp_floor=True)
    assert_bf16_close(dv, vr.grad, "dv", ulp_floor=True)


def test_dao_ops_right_window():
    """The Dao op pair with window_size_right on a non-causal block (the flash provider's
    (left, right), GQA 2:1, sq != sk)."""
    from ringmaster_amd.ring.kernels import flash_ops

    fwd, bwd = flash_ops()
    print("case dao right window 260x300 (40, 25)", flush=True)
    qf, q = bf16_pair((1, 260, 4, 128), 21)
    kf, k = bf16_pair((1, 300, 2, 128), 22)
    vf, v = bf16_pair((1, 300, 2, 128), 23)
    dof, do = bf16_pair((1, 260, 4, 128), 24)
    out, lse, _, _ = fwd(q, k, v, 0.0, 0.125, False, 40, 25, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.0, 0.125, False, 40, 25, 0.0, None, False, None)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=False, scaling=0.125, window=(40, 25),
                                 flash=True)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(dq, qr.grad, "dq")
    assert_bf16_close(dk, kr.grad, "dk", ulp_floor=True)
    assert_bf16_close(dv, vr.grad, "dv", ulp_floor=True)


@pytest.mark.parametrize("hq,hkv,sq,sk,d,window", [
    (2, 2, 300, 300, 128, (-1, 0)),     # right 0 alone: the causal block
    (4, 2, 200, 517, 64, (-1, 70)),     # right only, sq < sk
    (2, 1, 513, 400, 128, (33, 100)),   # both bounds, sk < sq: the first 13 rows keyless
    (2, 2, 1100, 1100, 128, (64, 64)),  # symmetric band: whole key tiles skipped both sides
    (4, 4, 96, 320, 40, (0, 5)),        # a narrow band at head dim 40
])
def test_block_right_window(hq, hkv, sq, sk, d, window):
    """Non-causal blocks bounded on the right: the kernels run the causal mask with its
    diagonal moved right by the bound."""
    _block(False, hq, hkv, sq, sk, d, window)


# ---- rings
def _ring_inputs(world, L, hq, hkv, d, seed=0):
    per, dev = [], []
    for i, h in enumerate((hq, hkv, hkv)):
        ts = [bf16_pair((1, h, L, d), seed + 10 * i + r)[0] for r in range(world)]
        per.append(ts)
        dev.append(torch.stack(ts).to(torch.bfloat16).cuda().requires_grad_(True))
    dos = [bf16_pair((1, L, hq, d), seed + 40 + r)[0] for r in range(world)]
    return per, dev, dos, torch.stack(dos).to(torch.bfloat16).cuda()


def _check_ring(fn, ref_fn, world, L, hq=2, hkv=2, d=128, seed=0, what=""):
    print(f"case ring {what} world={world} L={L} hq={hq} hkv={hkv} d={d}", flush=True)
    per, (qd, kd, vd), dos, dod = _ring_inputs(world, L, hq, hkv, d, seed)
    out = fn(qd, kd, vd)
    out.backward(dod)
    torch.cuda.synchronize()
    refs = [[t.clone().requires_grad_(True) for t in ts] for ts in per]
    ref_out, _ = ref_fn(*refs)
    sum((o * g).sum() for o, g in zip(ref_out, dos)).backward()
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(qd.grad[r], refs[0][r].grad, f"dq rank {r}")
        assert_bf16_close(kd.grad[r], refs[1][r].grad, f"dk rank {r}", ulp_floor=hq != hkv)
        assert_bf16_close(vd.grad[r], refs[2][r].grad, f"dv rank {r}", ulp_floor=hq != hkv)


@pytest.mark.parametrize("causal,left,right", [
    (True, 150, 0), (True, 40, 0), (False, 300, -1), (False, 700, -1),
    (False, 300, 0),    # non-causal, right 0: the band behind rank r's position (P-1) L + i
    (False, 100, 200),  # both bounds: every block of a rank masked on its own side
    (False, -1, 50),    # bounded on the right only
])
def test_allgather_ring_window(causal, left, right):
    """The gather ring hands the window to one block call over the gathered keys
    (ring/loop.py:218-228), so the block provider's (flash) window applies at the
    bottom-right aligned positions."""
    from ringmaster_amd.ring import ring_attention

    world, L = 4, 128
    w = (left, right)
    _check_ring(lambda q, k, v: ring_attention(q, k, v, causal=causal, rotate_method="allgather",
                                               window=w),
                lambda qs, ks, vs: rm.allgather_ring_forward(qs, ks, vs, causal=causal,
                                                             window=w, flash=True),
                world, L, hq=4, hkv=2, what=f"allgather causal={causal} window={w}")


def test_varlen_ring_window():
    from ringmaster_amd.ring import varlen_ring_attention

    cu = torch.tensor([0, 37, 200, 201, 390, 512], dtype=torch.int32)
    _check_ring(lambda q, k, v: varlen_ring_attention(q, k, v, scaling=None, cu_seqlens=cu.cuda(),
                                                      window=(60, 0)),
                lambda qs, ks, vs: rm.varlen_ring_forward(qs, ks, vs, cu, window=(60, 0)),
                4, 128, what="varlen window=60")


def test_zigzag_ring_head_dim_96():
    """The zigzag ring at head dim 96 against the oracle ring's forward and its explicit
    reverse-ring backward."""
    from ringmaster_amd.ring import zigzag_ring_attention

    world, L, hq, hkv, d = 4, 128, 4, 2, 96
    print(f"case ring zigzag world={world} L={L} hq={hq} hkv={hkv} d={d}", flush=True)
    per, (qd, kd, vd), dos, dod = _ring_inputs(world, L, hq, hkv, d)
    out = zigzag_ring_attention(qd, kd, vd)
    out.backward(dod)
    torch.cuda.synchronize()
    ref_out, ref_lse = rm.zigzag_ring_forward(*per)
    rdq, rdk, rdv = rm.zigzag_ring_backward(dos, *per, ref_out, ref_lse)
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(qd.grad[r], rdq[r], f"dq rank {r}")
        assert_bf16_close(kd.grad[r], rdk[r], f"dk rank {r}", ulp_floor=True)
        assert_bf16_close(vd.grad[r], rdv[r], f"dv rank {r}", ulp_floor=True)


def test_allgather_ring_head_dim_80_window():
    from ringmaster_amd.ring import ring_attention

    _check_ring(lambda q, k, v: ring_attention(q, k, v, causal=True, rotate_method="allgather",
                                               window=(100, 0)),
                lambda qs, ks, vs: rm.allgather_ring_forward(qs, ks, vs, causal=True,
                                                             window=(100, 0)),
                2, 192, d=80, what="allgather d=80 window=100")
