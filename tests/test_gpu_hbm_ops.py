"""HBM-bound ops on the MI355X vs the oracle: LSE merge, zigzag shard/unshard (bit-exact),
context-parallel linear scan (fp32, 1e-4 relative)."""

import pytest
import torch

from oracle import ring_math as rm
from oracle import shard as osh
from oracle import state_passing as sp
from tests.gpu_util import assert_f32_rel, seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("blk_dtype", [torch.bfloat16, torch.float32])
def test_lse_merge(blk_dtype):
    from ringmaster_amd.ring.merge import update_out_and_lse

    b, s, h, d = 2, 96, 4, 128
    o1 = seeded((b, s, h, d), 1).to(blk_dtype)
    l1 = seeded((b, h, s), 2) + 3.0
    o2 = seeded((b, s, h, d), 3).to(blk_dtype)
    l2 = seeded((b, h, s), 4) + 3.0
    l2[0, 0, :5] = float("-inf")  # masked rows: the merge must keep the running pair
    ro, rl = rm.update_out_and_lse(None, None, o1.float(), l1)
    ro, rl = rm.update_out_and_lse(ro, rl, o2.float(), l2)
    go, gl = update_out_and_lse(None, None, o1.cuda(), l1.cuda())
    go, gl = update_out_and_lse(go, gl, o2.cuda(), l2.cuda())
    torch.cuda.synchronize()
    assert_f32_rel(go, ro, "merged out")
    assert_f32_rel(gl, rl, "merged lse")


@pytest.mark.parametrize("world", [2, 4, 8])
@pytest.mark.parametrize("seq_len", [32, 48])
def test_zigzag_shard_roundtrip_small(world, seq_len):
    from ringmaster_amd.shard import zigzag_shard, zigzag_unshard

    ids = torch.arange(seq_len).view(1, seq_len)
    dev = zigzag_shard(ids.cuda(), world, pad_value=-100)
    for r in range(world):
        ref = osh.zigzag_shard_tensor(ids, world, r, pad_value=-100)
        assert torch.equal(dev[r].cpu(), ref)
    back = zigzag_unshard(dev, seq_len)
    assert torch.equal(back.cpu(), ids)


def test_zigzag_shard_batch_matches_oracle():
    """The product's batch shard against the oracle (every key, including a mask, a 3-D
    feature tensor and a tensor the caller padded already) and through the pinned rules
    of tests/test_shard_oracle.py (positions, pads, global shift labels, cover, unshard)."""
    from ringmaster_amd.shard import zigzag_shard, zigzag_shard_batch, zigzag_unshard
    from tests.test_shard_oracle import check_shard_batch

    for cp, seq in ((2, 16), (4, 22), (8, 48), (8, 37)):
        total = seq + (-seq) % (2 * cp)
        base = {"input_ids": torch.arange(seq).view(1, seq) + 1000,
                "labels": torch.arange(seq).view(1, seq) * 3,
                "attention_mask": torch.ones(1, seq, dtype=torch.long),
                "features": torch.randn(1, seq, 5, generator=torch.Generator().manual_seed(seq)),
                "prepadded": torch.arange(total).view(1, total) + 7}
        for r in range(cp):
            ref, (orig, pad) = osh.zigzag_shard_batch({k: v.clone() for k, v in base.items()}, r, cp)
            got, info = zigzag_shard_batch({k: v.cuda() for k, v in base.items()}, r, cp)
            assert info.original_seq_len == orig and info.pad_len == pad
            assert set(got) == set(ref)
            for key in ref:
                assert torch.equal(got[key].cpu(), ref[key]), (cp, seq, r, key)

    def shard_fn(batch, r, w):
        out, info = zigzag_shard_batch({k: v.cuda() for k, v in batch.items()}, r, w)
        return {k: v.cpu() for k, v in out.items()}, (info.original_seq_len, info.pad_len)

    check_shard_batch(
        shard_fn,
        unshard_fn=lambda shards, seq: zigzag_unshard(torch.stack(shards).cuda(), seq).cpu(),
        shard_tensor_fn=lambda x, w, r, pad_value=0: zigzag_shard(
            x.cuda(), w, rank=r, pad_value=pad_value).cpu())


def test_zigzag_shard_full_size_bit_exact():
    """configs[2] q-shaped tensor [1, 131072, 16, 128] bf16: shard -> unshard is the identity
    and every shard row equals the source row at its global index (checksum on samples)."""
    from ringmaster_amd.shard import zigzag_shard, zigzag_unshard

    world, S, H, d = 8, 131072, 16, 128
    x = torch.randint(-30000, 30000, (1, S, H, d), dtype=torch.int16, device="cuda").view(
        torch.bfloat16)
    sh = zigzag_shard(x, world)
    half = S // (2 * world)
    for r in (0, 3, 7):
        idx = rm.zigzag_gidx(r, half, world).cuda()
        assert torch.equal(sh[r, 0].view(torch.int16), x[0, idx].view(torch.int16))
    back = zigzag_unshard(sh, S)
    assert torch.equal(back.view(torch.int16), x.view(torch.int16))


@pytest.mark.parametrize("groups_mode", ["elementwise", "grouped", "scalar"])
@pytest.mark.parametrize("world", [1, 2, 8])
def test_linear_scan_small(groups_mode, world):
    from ringmaster_amd.strategies.state_passing import cp_linear_scan

    g = torch.Generator().manual_seed(5)
    T, d = 32, {"elementwise": 12, "grouped": 1024, "scalar": 6}[groups_mode]
    groups = {"elementwise": d, "grouped": 4, "scalar": 3}[groups_mode]
    a = torch.rand(2, T, groups, generator=g) * 0.9 + 0.05
    b = torch.randn(2, T, d, generator=g)
    dh = torch.randn(2, T, d, generator=g)
    af = a.repeat_interleave(d // groups, dim=2).double().requires_grad_(True)
    bf = b.double().requires_grad_(True)
    ref = sp.cp_linear_scan_emulated(af, bf, world)
    ref.backward(dh.double())
    ad, bd = a.cuda().requires_grad_(True), b.cuda().requires_grad_(True)
    h = cp_linear_scan(ad, bd, world=world)
    h.backward(dh.cuda())
    torch.cuda.synchronize()
    assert_f32_rel(h, ref, "h")
    ref_da = af.grad.reshape(2, T, groups, d // groups).sum(-1)
    assert_f32_rel(bd.grad, bf.grad, "db")
    assert_f32_rel(ad.grad, ref_da, "da", tol=1e-3 if groups_mode == "grouped" else 1e-4)


@pytest.mark.parametrize("groups_mode", ["elementwise", "grouped"])
def test_linear_scan_per_rank_with_h_in(groups_mode):
    """The per-rank boundary of cp_linear_scan(a, b, group) (strategies/state_passing.py:
    29-59): rank r's local chunk with the carried-in state H_in (the rank-ordered prefix of
    the earlier ranks' (A_j, B_j)) equals the global scan's slice; its gradients (da, db and
    dh_in = a_0 g_0) equal autograd through the oracle's per-rank scan; cp_scan_prefix
    folds the kernel's chunk states into the same H_in."""
    from ringmaster_amd.strategies.state_passing import (cp_linear_scan, cp_scan_prefix,
                                                         linear_scan_forward)

    g = torch.Generator().manual_seed(8)
    world, n = 4, 48
    d, groups = (12, 12) if groups_mode == "elementwise" else (1024, 4)
    a = torch.rand(2, world * n, groups, generator=g) * 0.9 + 0.05
    b = torch.randn(2, world * n, d, generator=g)
    af = a.repeat_interleave(d // groups, dim=2).double()
    glob = sp.local_linear_scan(af, b.double())
    pre = sp.scan_prefix(af, b.double(), world)
    _, cs = linear_scan_forward(a.cuda(), b.cuda(), world, return_chunk_state=True)
    assert_f32_rel(cp_scan_prefix(cs), pre, "H_in from the chunk states")
    for r in range(world):
        sl = slice(r * n, (r + 1) * n)
        dh = torch.randn(2, n, d, generator=g)
        ar, br = a[:, sl].cuda().requires_grad_(True), b[:, sl].cuda().requires_grad_(True)
        hin = pre[r].float().cuda().requires_grad_(True)
        h = cp_linear_scan(ar, br, None, h_in=hin)
        h.backward(dh.cuda())
        assert_f32_rel(h, glob[:, sl], f"rank {r}: h vs the global scan")
        ra = af[:, sl].clone().requires_grad_(True)
        rb = b[:, sl].double().requires_grad_(True)
        rh = pre[r].clone().requires_grad_(True)
        sp.rank_linear_scan(ra, rb, rh).backward(dh.double())
        assert_f32_rel(br.grad, rb.grad, f"rank {r}: db")
        assert_f32_rel(hin.grad, rh.grad, f"rank {r}: dh_in")
        ref_da = ra.grad.reshape(2, n, groups, d // groups).sum(-1)
        assert_f32_rel(ar.grad, ref_da, f"rank {r}: da", tol=1e-3 if groups > 12 else 1e-4)


def test_linear_scan_config4_full_size():
    """256 chunk states x 524288 fp32, world 8, per-head decay (64 groups)."""
    from ringmaster_amd.strategies.state_passing import linear_scan_forward

    L, d, G, world = 256, 524288, 64, 8
    g = torch.Generator().manual_seed(6)
    a = torch.rand(1, L, G, generator=g) * 0.9 + 0.05      # weak-decay parity variant
    b = torch.randn(1, L, d, generator=g)
    h, cs = linear_scan_forward(a.cuda(), b.cuda(), world, return_chunk_state=True)
    torch.cuda.synchronize()
    ref = sp.local_linear_scan_vec(a.repeat_interleave(d // G, dim=2), b)
    assert_f32_rel(h, ref, "h full size")
    n = L // world
    for r in (0, 7):
        cum = a[:, r * n:(r + 1) * n].prod(1).repeat_interleave(d // G, dim=1)
        assert_f32_rel(cs[r, :, 0], cum, f"A_{r}")


def test_linear_scan_config4_full_size_backward():
    """configs[4] backward at full size (256 chunk states x 524288 fp32, 64 decay groups,
    world 8): db, da (sums over 8192 channels per group) and the forward, against autograd
    through the oracle's emulated ranks in fp64 (strategies/state_passing.py:19-59)."""
    from ringmaster_amd.strategies.state_passing import cp_linear_scan

    L, d, G, world = 256, 524288, 64, 8
    g = torch.Generator().manual_seed(9)
    a = torch.rand(1, L, G, generator=g) * 0.9 + 0.05
    b = torch.randn(1, L, d, generator=g)
    dh = torch.randn(1, L, d, generator=g)
    ad, bd = a.cuda().requires_grad_(True), b.cuda().requires_grad_(True)
    h = cp_linear_scan(ad, bd, world=world)
    h.backward(dh.cuda())
    torch.cuda.synchronize()
    h, da, db = h.detach().cpu(), ad.grad.cpu(), bd.grad.cpu()
    af = a.double().repeat_interleave(d // G, dim=2).requires_grad_(True)
    bf = b.double().requires_grad_(True)
    ref = sp.cp_linear_scan_emulated(af, bf, world)
    ref.backward(dh.double())
    assert_f32_rel(h, ref.detach(), "h")
    del ref
    assert_f32_rel(db, bf.grad, "db")
    ref_da = af.grad.reshape(1, L, G, d // G).sum(-1)
    assert_f32_rel(da, ref_da, "da", tol=1e-3)
