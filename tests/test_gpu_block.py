"""Block provider parity: mi355x_hip_block (HIP, bf16) vs the oracle math_block (fp32)."""

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, assert_f32_rel, bf16_pair

pytestmark = pytest.mark.gpu


def _run(causal, hq, hkv, sq, sk, d, b=1, seed=0):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    qf, qd = bf16_pair((b, sq, hq, d), seed + 1)
    kf, kd = bf16_pair((b, sk, hkv, d), seed + 2)
    vf, vd = bf16_pair((b, sk, hkv, d), seed + 3)
    dof, dod = bf16_pair((b, sq, hq, d), seed + 4)
    qd.requires_grad_(True)
    kd.requires_grad_(True)
    vd.requires_grad_(True)
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None)
    out.backward(dod)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(qd.grad, qr.grad, "dq")
    assert_bf16_close(kd.grad, kr.grad, "dk")
    assert_bf16_close(vd.grad, vr.grad, "dv")


@pytest.mark.parametrize("causal,hq,hkv,sq,sk,d", [
    (True, 2, 2, 256, 256, 128),
    (False, 2, 2, 256, 256, 128),
    (False, 4, 1, 192, 320, 128),   # GQA 4:1, ragged tiles
    (True, 2, 2, 100, 300, 128),    # bottom-right causal, sq < sk, tails
    (False, 8, 2, 128, 64, 128),    # sk < sq
    (True, 4, 2, 200, 200, 64),     # head_dim 64
    (False, 2, 1, 1, 77, 128),      # single query row
])
def test_block_fwd_bwd(causal, hq, hkv, sq, sk, d):
    _run(causal, hq, hkv, sq, sk, d)


def test_block_batch2():
    _run(True, 2, 1, 130, 130, 128, b=2)


def test_block_config1_shape_small():
    # configs[1] head geometry (Hq=32, Hkv=8, D=128) at a short sequence, non-causal
    _run(False, 32, 8, 256, 256, 128)


def test_dao_signature_ops():
    from ringmaster_amd.ring.kernels import flash_ops

    fwd, bwd = flash_ops()
    qf, q = bf16_pair((1, 128, 4, 128), 11)
    kf, k = bf16_pair((1, 128, 2, 128), 12)
    vf, v = bf16_pair((1, 128, 2, 128), 13)
    dof, do = bf16_pair((1, 128, 4, 128), 14)
    out, lse, _, _ = fwd(q, k, v, 0.0, 0.125, True, -1, -1, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.0, 0.125, True, -1, -1, 0.0, None, False, None)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=True, scaling=0.125)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(dq, qr.grad, "dq")
    assert_bf16_close(dk, kr.grad, "dk")
    assert_bf16_close(dv, vr.grad, "dv")


def test_errors_match_reference_contract():
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    q = torch.zeros(1, 8, 3, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="divisible"):
        mi355x_hip_block(q, k, k, causal=True, scaling=None)
    with pytest.raises(RuntimeError):
        mi355x_hip_block(q.cpu(), k.cpu(), k.cpu(), causal=True, scaling=None)


def test_doc_mask_block():
    """Document-masked block (global indices) vs the oracle masked_block_fwd/bwd."""
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops

    S, h, H, d = 512, 128, 2, 128
    cu = torch.tensor([0, 70, 200, 333, 512], dtype=torch.int32)
    doc = rm.doc_ids_from_cu(cu)
    qg = torch.cat([torch.arange(0, 128), torch.arange(384, 512)])   # a zigzag-like q set
    kg = torch.arange(128, 384)
    qf, qd = bf16_pair((1, 256, H, d), 21)
    kf, kd = bf16_pair((1, 256, H, d), 22)
    vf, vd = bf16_pair((1, 256, H, d), 23)
    m = rm.additive_doc_mask(qg, kg, doc, True)
    ref, ref_lse = rm.masked_block_fwd(qf, kf, vf, m, d ** -0.5)
    out = torch.empty_like(qd)
    lse = torch.empty(1, H, 256, device="cuda")
    dev_i32 = lambda t: t.to(torch.int32).cuda()  # noqa: E731
    ops.attn_fwd([ops.FwdJob(q=qd, k=kd, v=vd, mode=abi.FWD_WRITE, out=out, lse=lse,
                             q_gidx=dev_i32(qg), k_gidx=dev_i32(kg),
                             q_doc=dev_i32(doc[qg]), k_doc=dev_i32(doc[kg]))],
                 scale=d ** -0.5, mask=abi.MASK_DOC)
    torch.cuda.synchronize()
    assert_bf16_close(out, ref, "doc out")
    assert_f32_rel(lse, ref_lse, "doc lse")
    del h, S
