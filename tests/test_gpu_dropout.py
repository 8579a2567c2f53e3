"""Attention dropout on the MI355X vs the CPU oracle.

The kernels draw the dropout mask from a hash of (seed, batch, head, query, key)
(oracle.ring_math.dropout_keep restates it), so a given seed is checked exactly: the
mask bit for bit, the dropped outputs and gradients to the bf16 bar, through the block
provider, the Dao op pair (its rng_state) and the gather ring. Agreement with the
reference's torch dropout is distributional (tests/test_oracle_pinning.py)."""

import numpy as np
import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, assert_f16_close, assert_f32_rel, bf16_pair, f16_pair

pytestmark = pytest.mark.gpu


def _block(causal, hq, hkv, sq, sk, d, p, seed, window=None, half=torch.bfloat16):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    print(f"case dropout block causal={causal} hq={hq} hkv={hkv} sq={sq} sk={sk} d={d} p={p} "
          f"seed={seed} window={window} dtype={half}", flush=True)
    pair = f16_pair if half == torch.float16 else bf16_pair
    close = assert_f16_close if half == torch.float16 else assert_bf16_close
    qf, qd = pair((1, sq, hq, d), 1)
    kf, kd = pair((1, sk, hkv, d), 2)
    vf, vd = pair((1, sk, hkv, d), 3)
    dof, dod = pair((1, sq, hq, d), 4)
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None, dropout=p,
                                dropout_seed=seed, window=window)
    out.backward(dod)
    torch.cuda.synchronize()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None, dropout=p,
                                 drop_seed=seed, window=window, flash=True)
    ref.backward(dof)
    close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse (undropped)")
    kw = {} if half == torch.float16 else {"ulp_floor": hq != hkv}
    close(qd.grad, qr.grad, "dq")
    close(kd.grad, kr.grad, "dk", **kw)
    close(vd.grad, vr.grad, "dv", **kw)


@pytest.mark.parametrize("causal,hq,hkv,sq,sk,d,p", [
    (True, 2, 2, 256, 256, 128, 0.1),
    (False, 4, 2, 192, 320, 128, 0.5),
    (True, 2, 2, 100, 300, 64, 0.2),
    (False, 8, 2, 128, 64, 96, 0.3),
])
def test_dropout_block(causal, hq, hkv, sq, sk, d, p):
    _block(causal, hq, hkv, sq, sk, d, p, seed=1234 + sq)


def test_dropout_block_fp16_window():
    _block(True, 4, 2, 300, 300, 128, 0.25, seed=77, window=(90, 0), half=torch.float16)


def test_dropout_block_right_window():
    _block(False, 4, 2, 300, 280, 128, 0.2, seed=91, window=(50, 20))


@pytest.mark.parametrize("b,hq,sq,sk,p,seed", [
    (2, 2, 512, 128, 0.4, 0xDEADBEEFCAFE),
    # element (b 1, h 8, q 202, k 74) hashes between floor(p 2^32) of the fp32 p the ABI
    # carries and that of the float64 p: dropped by the fp32 threshold
    (2, 16, 256, 128, 0.3, 1145),
])
def test_dropout_mask_bits_exact(b, hq, sq, sk, p, seed):
    """q = 0 makes every probability 1 / sk; with V = I (sk = d) the output row q is the
    mask row scaled by 1 / (sk (1 - p)), so the kernel's keep bits are read off the output
    and compared with the oracle's hash, bit for bit (every head and batch row)."""
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    print(f"case dropout mask bits b={b} hq={hq} sq={sq} sk={sk} p={p} seed={seed}", flush=True)
    q = torch.zeros(b, sq, hq, sk, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(b, sk, hq, sk, dtype=torch.bfloat16, device="cuda")
    v = torch.eye(sk, dtype=torch.bfloat16, device="cuda")[None, :, None, :].expand(b, sk, hq, sk)
    out, _ = mi355x_hip_block(q, k, v.contiguous(), causal=False, scaling=None, dropout=p,
                              dropout_seed=seed)
    torch.cuda.synchronize()
    got = (out.float().cpu() * sk * (1 - p)) > 0.5  # [b, sq, hq, sk]
    for bi in range(b):
        for h in range(hq):
            want = rm.dropout_keep(seed, bi * hq + h, np.arange(sq), np.arange(sk), p)
            assert np.array_equal(got[bi, :, h].numpy(), want), f"mask of (b={bi}, h={h})"
    assert abs(got.float().mean().item() - (1 - p)) < 0.01
    if seed == 1145:
        assert not bool(got[1, 202, 8, 74])


def test_dropout_seed_determinism():
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    _, q = bf16_pair((1, 256, 2, 128), 5)
    _, k = bf16_pair((1, 256, 2, 128), 6)
    _, v = bf16_pair((1, 256, 2, 128), 7)
    a, _ = mi355x_hip_block(q, k, v, causal=True, scaling=None, dropout=0.3, dropout_seed=11)
    b, _ = mi355x_hip_block(q, k, v, causal=True, scaling=None, dropout=0.3, dropout_seed=11)
    c, _ = mi355x_hip_block(q, k, v, causal=True, scaling=None, dropout=0.3, dropout_seed=12)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


def _drop_grad_bar(qf, kf, vf, dof, p, seed, scale):
    """Per-element bars of dK and dV [b, sk, hkv, d] for a causal dropout block: max(2e-2,
    two bf16 ulps of the element) plus the rounding the backward adds before its sums, from
    fp64 summands: it takes (P M)^T and dS = P (M dP - delta) as bf16 operands (2^-9
    relative each, M the kept mask times 1 / (1 - p)), so dK gains up to 4 2^-8
    RSS_q(scale dS Q) and dV 4 2^-8 RSS_q(P M dO), over the queries and folded heads.
    Elements whose summands cancel (|dK| far below the sum of |summands|) need that term:
    the two-ulp bar alone is a bar on the result's own size."""
    q, k, v, do = (t.double() for t in (qf, kf, vf, dof))
    b, sq, hq, d = q.shape
    sk, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    kx, vx = k.repeat_interleave(g, 2), v.repeat_interleave(g, 2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, kx) * scale
    s = s.masked_fill(torch.ones(sq, sk, dtype=torch.bool).triu(sk - sq + 1), float("-inf"))
    pr = torch.softmax(s, -1)
    m = rm.dropout_scale_mask(seed, b, hq, sq, sk, p).double()
    dpm = m * torch.einsum("bqhd,bkhd->bhqk", do, vx)
    out = torch.einsum("bhqk,bkhd->bqhd", pr * m, vx)
    dlt = (do * out).sum(-1).transpose(1, 2)[..., None]
    ds = pr * (dpm - dlt)

    def fold(x, y):
        return torch.einsum("bhqk,bqhd->bkhd", x, y).unflatten(2, (hkv, g)).sum(3)

    extra_k = 4 * 2.0 ** -8 * scale * fold(ds ** 2, q ** 2).sqrt()
    extra_v = 4 * 2.0 ** -8 * fold((pr * m) ** 2, do ** 2).sqrt()
    return extra_k.float(), extra_v.float()


def _close_with(got, ref, extra, what):
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    diff = (g - r).abs()
    bar = (r.abs() * 2 * 2.0 ** -7).clamp_min(2e-2) + extra
    over = (diff / bar).max().item()
    rl = float(((g - r).norm() / r.norm().clamp_min(1e-30)).item())
    assert over < 1 and rl < 1e-2, f"{what}: max-abs {diff.max().item():.3e} ({over:.2f} of the bar) rel-L2 {rl:.3e}"


def test_dropout_dao_ops_rng_state():
    from ringmaster_amd.ring.kernels import flash_ops

    # the mask follows the device generator's (seed, offset): seed it, so the case does not
    # depend on how many draws earlier tests made
    torch.cuda.manual_seed(20)
    fwd, bwd = flash_ops()
    qf, q = bf16_pair((1, 192, 4, 128), 11)
    kf, k = bf16_pair((1, 192, 2, 128), 12)
    vf, v = bf16_pair((1, 192, 2, 128), 13)
    dof, do = bf16_pair((1, 192, 4, 128), 14)
    out, lse, _, rng_state = fwd(q, k, v, 0.2, 0.125, True, -1, -1, 0.0, None, False)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd(do, q, k, v, out, lse, dq, dk, dv, 0.2, 0.125, True, -1, -1, 0.0, None, False, rng_state)
    torch.cuda.synchronize()
    from ringmaster_amd.ring.kernels import seed_of_rng_state

    # rng_state: the device generator's (seed, offset), as flash returns it
    seed = seed_of_rng_state(int(rng_state[0]) & ((1 << 64) - 1), int(rng_state[1]))
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf, kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=True, scaling=0.125, dropout=0.2,
                                 drop_seed=seed)
    ref.backward(dof)
    assert_bf16_close(out, ref, "out")
    assert_f32_rel(lse, ref_lse, "lse")
    assert_bf16_close(dq, qr.grad, "dq")
    # GQA-folded, with kept probabilities scaled by 1 / (1 - p) = 1.25: dK / dV values near 3
    # (two bf16 ulps of 2^-6 each) and elements whose summands cancel
    extra_k, extra_v = _drop_grad_bar(qf, kf, vf, dof, 0.2, seed, 0.125)
    _close_with(dk, kr.grad, extra_k, "dk")
    _close_with(dv, vr.grad, extra_v, "dv")
    with pytest.raises(ValueError, match="rng_state"):
        bwd(do, q, k, v, out, lse, dq, dk, dv, 0.2, 0.125, True, -1, -1, 0.0, None, False, None)


@pytest.mark.parametrize("causal", [True, False])
def test_dropout_allgather_ring(causal):
    """The gather ring with dropout: one mask over (global query, gathered key), drawn from
    a seed of torch's CPU generator, against the oracle's gather ring with that seed."""
    from ringmaster_amd.ring import ring_attention
    from ringmaster_amd.ring.kernels import new_dropout_seed

    world, L, hq, hkv, d, p = 4, 128, 4, 2, 128, 0.15
    print(f"case dropout allgather causal={causal} world={world} L={L}", flush=True)
    per, dev = [], []
    for i, h in enumerate((hq, hkv, hkv)):
        ts = [bf16_pair((1, h, L, d), 30 + 10 * i + r)[0] for r in range(world)]
        per.append(ts)
        dev.append(torch.stack(ts).to(torch.bfloat16).cuda().requires_grad_(True))
    dos = [bf16_pair((1, L, hq, d), 70 + r)[0] for r in range(world)]
    torch.manual_seed(2024)
    out = ring_attention(*dev, causal=causal, rotate_method="allgather", dropout=p)
    out.backward(torch.stack(dos).to(torch.bfloat16).cuda())
    torch.cuda.synchronize()
    torch.manual_seed(2024)
    seed = new_dropout_seed()
    refs = [[t.clone().requires_grad_(True) for t in ts] for ts in per]
    ref_out, _ = rm.allgather_ring_forward(*refs, causal=causal, dropout=p, drop_seed=seed)
    sum((o * g).sum() for o, g in zip(ref_out, dos)).backward()
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(dev[0].grad[r], refs[0][r].grad, f"dq rank {r}")
        assert_bf16_close(dev[1].grad[r], refs[1][r].grad, f"dk rank {r}", ulp_floor=True)
        assert_bf16_close(dev[2].grad[r], refs[2][r].grad, f"dv rank {r}", ulp_floor=True)


def test_dropout_seeds_leave_the_cpu_stream_alone():
    """Dropout draws its seed from the device generator's (seed, offset), as flash does: the
    CPU generator's stream is unchanged, consecutive calls get different masks, and
    torch.manual_seed makes the draws repeat."""
    from ringmaster_amd.ring.kernels import mi355x_hip_block, new_dropout_seed

    _, q = bf16_pair((1, 128, 2, 64), 21)
    torch.manual_seed(7)
    expect = torch.rand(4)
    torch.manual_seed(7)
    a, _ = mi355x_hip_block(q, q, q, causal=True, scaling=None, dropout=0.25)
    b, _ = mi355x_hip_block(q, q, q, causal=True, scaling=None, dropout=0.25)
    assert torch.equal(torch.rand(4), expect)
    torch.manual_seed(7)
    a2, _ = mi355x_hip_block(q, q, q, causal=True, scaling=None, dropout=0.25)
    torch.cuda.synchronize()
    assert torch.equal(a, a2) and not torch.equal(a, b)
    torch.manual_seed(7)
    assert new_dropout_seed() != new_dropout_seed()
