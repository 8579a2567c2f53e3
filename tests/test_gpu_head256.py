"""Head dims above 128 (up to 256, e.g. Gemma's 256) on the MI355X vs the CPU oracle (fp32).

The provider contract's head dims (ring/kernels.py:52-78: any head dim for ``math``;
flash takes up to 256) on single blocks (causal, bottom-right aligned with sq != sk,
GQA, windows, ragged lengths, fp16, dropout), through the Dao op pair, and in the rings
(the zigzag ring's merged forward and fp32 gradient accumulation, the packed document
ring). The kernels compute at 256 and read the columns past head_dim as zeros."""

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import (assert_bf16_close, assert_f16_close, assert_f32_rel, bf16_pair,
                            f16_pair)

pytestmark = pytest.mark.gpu


def _block(causal, hq, hkv, sq, sk, d, window=None, b=1, seed=0, half=torch.bfloat16,
           dropout=0.0):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    print(f"case block d={d} causal={causal} hq={hq} hkv={hkv} sq={sq} sk={sk} b={b} "
          f"window={window} dtype={half} dropout={dropout}", flush=True)
    pair = f16_pair if half == torch.float16 else bf16_pair
    close = assert_f16_close if half == torch.float16 else assert_bf16_close
    qf, qd = pair((b, sq, hq, d), seed + 1)
    kf, kd = pair((b, sk, hkv, d), seed + 2)
    vf, vd = pair((b, sk, hkv, d), seed + 3)
    dof, dod = pair((b, sq, hq, d), seed + 4)
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    seed_d = 4321 + seed if dropout else None
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None, window=window,
                                dropout=dropout, dropout_seed=seed_d)
    out.backward(dod)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None, window=window,
                                 dropout=dropout, drop_seed=seed_d, flash=True)
    ref.backward(dof)
    close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    kw = {} if half == torch.float16 else {"ulp_floor": hq != hkv or bool(dropout)}
    close(qd.grad, qr.grad, "dq")
    close(kd.grad, kr.grad, "dk", **kw)
    close(vd.grad, vr.grad, "dv", **kw)


@pytest.mark.parametrize("causal,hq,hkv,sq,sk,d", [
    (True, 2, 2, 256, 256, 256),    # whole tiles
    (False, 4, 2, 192, 320, 256),   # GQA 2:1, sq < sk
    (True, 4, 1, 300, 517, 256),    # ragged, bottom-right aligned, GQA 4:1
    (False, 2, 2, 333, 100, 256),   # sk < sq: ragged key block
    (True, 2, 2, 230, 230, 136),    # head dims between 128 and 256: zero columns
    (False, 4, 2, 160, 200, 192),
    (True, 2, 1, 129, 129, 248),
])
def test_block_head_dim_above_128(causal, hq, hkv, sq, sk, d):
    _block(causal, hq, hkv, sq, sk, d)


def test_block_head_dim_256_batch2_window():
    _block(True, 4, 2, 400, 400, 256, window=(90, 0), b=2)
    _block(False, 2, 2, 190, 260, 256, window=(70, 0), seed=5)
    _block(False, 2, 2, 190, 260, 256, window=(-1, 40), seed=6)  # right-bounded only
    _block(False, 2, 1, 260, 190, 256, window=(64, 90), seed=7)  # both bounds, sk < sq


def test_block_head_dim_256_fp16():
    _block(True, 4, 2, 300, 300, 256, half=torch.float16)


@pytest.mark.parametrize("causal", [True, False])
def test_block_head_dim_256_dropout(causal):
    _block(causal, 4, 2, 200, 264, 256, dropout=0.2, seed=7)


def test_dao_ops_head_dim_256():
    from ringmaster_amd.ring.kernels import flash_ops

    print("case dao ops d=256", flush=True)
    fwd, bwd = flash_ops()
    qf, q = bf16_pair((1, 300, 4, 256), 11)
    kf, k = bf16_pair((1, 300, 2, 256), 12)
    vf, v = bf16_pair((1, 300, 2, 256), 13)
    dof, do = bf16_pair((1, 300, 4, 256), 14)
    out, lse, _, _ = fwd(q, k, v, 0.0, 0.0625, True, -1, -1, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.0, 0.0625, True, -1, -1, 0.0, None, False, None)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=True, scaling=0.0625)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(dq, qr.grad, "dq")
    assert_bf16_close(dk, kr.grad, "dk", ulp_floor=True)
    assert_bf16_close(dv, vr.grad, "dv", ulp_floor=True)


def _ring_inputs(world, L, hq, hkv, d, seed=0):
    per, dev = [], []
    for i, h in enumerate((hq, hkv, hkv)):
        ts = [bf16_pair((1, h, L, d), seed + 10 * i + r)[0] for r in range(world)]
        per.append(ts)
        dev.append(torch.stack(ts).to(torch.bfloat16).cuda().requires_grad_(True))
    dos = [bf16_pair((1, L, hq, d), seed + 40 + r)[0] for r in range(world)]
    return per, dev, dos, torch.stack(dos).to(torch.bfloat16).cuda()


def test_zigzag_ring_head_dim_256():
    """The zigzag ring at head dim 256 (merged forward across steps, fp32 dK/dV
    accumulation) against the oracle ring's forward and its explicit reverse-ring
    backward."""
    from ringmaster_amd.ring import zigzag_ring_attention

    world, L, hq, hkv, d = 4, 128, 4, 2, 256
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


def test_varlen_ring_head_dim_256():
    """Packed documents (document masks on global indices) at head dim 256."""
    from ringmaster_amd.ring import varlen_ring_attention

    world, L, hq, hkv, d = 4, 128, 2, 2, 256
    cu = torch.tensor([0, 37, 200, 201, 390, 512], dtype=torch.int32)
    print(f"case ring varlen world={world} L={L} d={d}", flush=True)
    per, (qd, kd, vd), dos, dod = _ring_inputs(world, L, hq, hkv, d, seed=3)
    out = varlen_ring_attention(qd, kd, vd, scaling=None, cu_seqlens=cu.cuda())
    out.backward(dod)
    torch.cuda.synchronize()
    refs = [[t.clone().requires_grad_(True) for t in ts] for ts in per]
    ref_out, _ = rm.varlen_ring_forward(*refs, cu)
    sum((o * g).sum() for o, g in zip(ref_out, dos)).backward()
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(qd.grad[r], refs[0][r].grad, f"dq rank {r}")
        assert_bf16_close(kd.grad[r], refs[1][r].grad, f"dk rank {r}")
        assert_bf16_close(vd.grad[r], refs[2][r].grad, f"dv rank {r}")


@pytest.mark.parametrize("causal", [True, False])
def test_dkdv_head_dim_256_unaligned_gradient_buffers(causal):
    """dK/dV written into caller buffers below vector alignment (fp32 views 4 bytes and bf16
    views 2 bytes past an aligned base: the ABI asks only for element-aligned strides) equal,
    bit for bit, the same gradients written into aligned buffers."""
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops
    from ringmaster_amd.ring.kernels import block_forward

    b, sq, sk, hq, hkv, d = 1, 200, 264, 4, 2, 256
    print(f"case unaligned dkdv causal={causal} d={d}", flush=True)
    _, q = bf16_pair((b, sq, hq, d), 21)
    _, k = bf16_pair((b, sk, hkv, d), 22)
    _, v = bf16_pair((b, sk, hkv, d), 23)
    _, do = bf16_pair((b, sq, hq, d), 24)
    sc = d ** -0.5
    mask = abi.MASK_CAUSAL if causal else abi.MASK_FULL
    out, lse, out32 = block_forward(q, k, v, sc, causal, keep_f32=True)
    delta = torch.empty((b, hq, sq), device="cuda")
    nlse = torch.empty_like(delta)
    ops.attn_bwd_delta(out32, do, delta, hkv, lse=lse, nlse=nlse)
    n = b * sk * hkv * d
    shape = (b, sk, hkv, d)

    def run(off, f32):
        dt = torch.float32 if f32 else torch.bfloat16
        bufs = [torch.zeros(n + 8, dtype=dt, device="cuda") for _ in range(2)]
        dk, dv = (t[off:off + n].view(shape) for t in bufs)
        kw = dict(dk_acc=dk, dv_acc=dv) if f32 else dict(dk=dk, dv=dv)
        ops.attn_bwd([ops.BwdJob(q=q, k=k, v=v, dout=do, lse=lse, delta=delta, nlse=nlse,
                                 dq_mode=abi.GRAD_NONE,
                                 dkv_mode=abi.GRAD_WRITE_F32 if f32 else abi.GRAD_WRITE_BF16,
                                 **kw)], scale=sc, mask=mask)
        torch.cuda.synchronize()
        return dk.clone(), dv.clone()

    for f32 in (True, False):
        ak, av = run(0, f32)
        uk, uv = run(1, f32)
        assert torch.equal(ak, uk) and torch.equal(av, uv), f"f32={f32}"
        assert ak.abs().sum() > 0
