"""A seeded sweep of block shapes through the provider on the MI355X vs the CPU oracle (fp32).

Each case draws batch 1-2, query and key lengths from 1 to 700 (ragged against every tile
size, sk < sq included: bottom-right causal then leaves the first rows without keys, out 0 and
lse -inf), GQA ratios 1-8, head dims that are multiples of 8 up to 256 (all three kernel
sets), causal or not, a window or none (flash attention's ``(left, right)``: every other
non-causal windowed case bounded on the right too, the others by the left bound and flash's
right bound at sk), bf16 or fp16, and dropout or none, and checks out,
lse and the three gradients against ``math_block`` (ring/kernels.py:52-78) at the bf16 / fp16
bars: max(2e-2, two ulps of the element) for bf16 gradients (5e-3 and fp16 ulps for fp16),
wider only for the dK of the named cancellation cases (``_CANCEL``). The draw is fixed (numpy
seed 20261202), so a failure names a reproducible case."""

import math

import numpy as np
import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import (assert_bf16_close, assert_f16_close, assert_f32_rel, bf16_pair,
                            f16_pair, keyless_prefix, rel_l2)

pytestmark = pytest.mark.gpu


def _cases(n=48, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2]))
        g = int(rng.choice([1, 2, 4, 8]))
        d = int(rng.choice([8, 40, 64, 72, 128, 136, 200, 256]))
        sq = int(rng.choice([1, 2, 31, 64, 65, 129, 257, 300, 511, 700]))
        sk = int(rng.choice([1, 3, 32, 64, 100, 128, 250, 513, 700]))
        causal = bool(rng.random() < 0.5)
        left = int(rng.choice([0, 5, 63, 200])) if rng.random() < 0.3 else None
        half = "f16" if rng.random() < 0.25 else "bf16"
        p = float(rng.choice([0.1, 0.3])) if rng.random() < 0.2 else 0.0
        b = int(rng.choice([1, 2]))
        # the right bound: derived from the index, so the draws above stay as they were
        right = (7 * i) % 61 if (left is not None and not causal and i % 2) else -1
        out.append((i, b, sq, sk, hkv * g, hkv, d, causal, left, right, half, p))
    return out


def _id(c):
    i, b, sq, sk, hq, hkv, d, causal, left, right, half, p = c
    win = f"w{left}" + (f",{right}" if right >= 0 else "")
    return f"{i}-b{b}-q{sq}-k{sk}-h{hq}:{hkv}-d{d}-{'c' if causal else 'f'}-{win}-{half}-p{p}"


# Cases whose dK and dV sum many query rows onto few keys (700 queries onto 3 keys; 511
# queries x 8 folded heads onto 32): the summands of such an element cancel, e.g. a dK of 0.65
# from an absolute sum of 102, a dV of 1.08 from signed dO rows. The backward's GEMMs take dS
# and P in bf16 (relative rounding up to 2^-8), and delta inherits the forward's rounding of P
# (2^-8 sum_k P |dP| per row), so the error of a cancelling element scales with its summands,
# not with the result: measured 1.4-1.8 times 2^-8 RSS(scale dS Q) at the worst dK elements.
# Their bars add 4 2^-8 RSS(scale dS Q) + RSS(scale P d_delta Q) (dK) and 4 2^-8 RSS(P dO)
# (dV), computed in fp64 from the oracle's inputs.
_CANCEL = {8, 24}


def _grad_spread(qf, kf, vf, dof, causal, left):
    """Per element of dK [b, sk, hkv, d]: 4 2^-8 RSS_q(scale dS_qk Q_q) + RSS_q(scale P_qk
    d_q Q_q), d_q = 2^-8 sum_k P_qk |dP_qk|; of dV: 4 2^-8 RSS_q(P_qk dO_q) (the backward
    takes P in bf16); over the queries and folded heads (fp64). Also |dK| and |dV| over the
    absolute sums of their summands (how far each element cancels)."""
    q, k, v, do = (t.double() for t in (qf, kf, vf, dof))
    b, sq, hq, d = q.shape
    sk, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    kx, vx = k.repeat_interleave(g, 2), v.repeat_interleave(g, 2)
    scale = 1.0 / math.sqrt(d)
    s = torch.einsum("bqhd,bkhd->bhqk", q, kx) * scale
    iq, ik = torch.arange(sq)[:, None] + (sk - sq), torch.arange(sk)[None, :]
    masked = torch.zeros(sq, sk, dtype=torch.bool)
    if causal:
        masked |= ik > iq
    if left is not None:
        masked |= iq - ik > left
    pr = torch.softmax(s.masked_fill(masked, float("-inf")), -1)
    dp = torch.einsum("bqhd,bkhd->bhqk", do, vx)
    dlt = (do * torch.einsum("bhqk,bkhd->bqhd", pr, vx)).sum(-1).transpose(1, 2)[..., None]
    ds = pr * (dp - dlt)
    dd = 2.0 ** -8 * (pr * dp.abs()).sum(-1, keepdim=True)

    def fold(x, y):
        return torch.einsum("bhqk,bqhd->bkhd", x, y).unflatten(2, (hkv, g)).sum(3)

    extra_k = 4 * 2.0 ** -8 * scale * fold(ds ** 2, q ** 2).sqrt() + scale * fold((pr * dd) ** 2, q ** 2).sqrt()
    extra_v = 4 * 2.0 ** -8 * fold(pr ** 2, do ** 2).sqrt()
    # how far the elements cancel: |dK| (|dV|) over the absolute sum of its summands
    ratio_k = fold(ds, q).abs() / fold(ds.abs(), q.abs()).clamp_min(1e-30)
    ratio_v = fold(pr, do).abs() / fold(pr, do.abs()).clamp_min(1e-30)
    return extra_k.float(), extra_v.float(), ratio_k, ratio_v


@pytest.mark.parametrize("case", _cases(), ids=_id)
def test_block_sweep(case):
    from ringmaster_amd.ring.kernels import mi355x_hip_block

    i, b, sq, sk, hq, hkv, d, causal, left, right, half, p = case
    print(f"case sweep {_id(case)}", flush=True)
    f16 = half == "f16"
    pair = f16_pair if f16 else bf16_pair
    close = assert_f16_close if f16 else assert_bf16_close
    window = None if left is None else (left, right)
    qf, qd = pair((b, sq, hq, d), 100 + i)
    kf, kd = pair((b, sk, hkv, d), 200 + i)
    vf, vd = pair((b, sk, hkv, d), 300 + i)
    dof, dod = pair((b, sq, hq, d), 400 + i)
    for t in (qd, kd, vd):
        t.requires_grad_(True)
    seed = 777 + i if p else None
    out, lse = mi355x_hip_block(qd, kd, vd, causal=causal, scaling=None, window=window,
                                dropout=p, dropout_seed=seed)
    out.backward(dod)
    torch.cuda.synchronize()
    # rows without any key (a right bound R with sk + R < sq, R = 0 for causal blocks): the
    # prefix i < sq - sk - R. The oracle runs on the other rows, which keep their positions
    # (and dropout coordinates, drop_q0 = s0); the kernels give those rows out 0, lse -inf
    # and dq 0 (the convention of the reference's masked blocks, ring/varlen_blocks.py:70-79)
    s0 = keyless_prefix(sq, sk, causal, window)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (qf[:, s0:], kf, vf))
    ref, ref_lse = rm.math_block(qr, kr, vr, causal=causal, scaling=None, window=window,
                                 dropout=p, drop_seed=seed, drop_q0=s0, flash=True)
    ref.backward(dof[:, s0:])
    got_l = lse.detach().cpu()
    assert torch.isneginf(got_l[:, :, :s0]).all(), "rows without keys: lse"
    assert torch.equal(out[:, :s0].float().cpu(), torch.zeros_like(out[:, :s0].float().cpu()))
    assert torch.equal(qd.grad[:, :s0].float().cpu(), torch.zeros_like(qd.grad[:, :s0].float().cpu()))
    if s0 == sq:
        return
    assert_f32_rel(got_l[:, :, s0:], ref_lse, "lse")

    def check(got, ref, what, grad, extra=None):
        # references that are exactly 0 in exact arithmetic (one key per row: dS = 0) get the
        # max-abs bar only. Gradients: max(2e-2, two bf16 ulps of the element) (fp16: 5e-3
        # and fp16 ulps, rel-L2 2.5e-3), plus ``extra`` for the named cancellation cases.
        # Outputs (bf16) are floored at one ulp of the value: dropout's 1 / (1 - p) lifts them
        # past 4, where half a bf16 ulp is 1.6e-2
        ref = ref.detach().float()
        floor, ulp, rl_bar = (5e-3, 2.0 ** -10, 2.5e-3) if f16 else (2e-2, 2.0 ** -7, 1e-2)
        if ref.abs().max().item() < 1e-3:
            err = (got.detach().float().cpu() - ref).abs().max().item()
            assert err < floor, f"{what}: max-abs {err:.3e} against a zero reference"
        elif not grad:
            close(got, ref, what) if f16 else close(got, ref, what, ulp_floor=True)
        else:
            g = got.detach().float().cpu()
            assert torch.isfinite(g).all(), f"{what}: non-finite values"
            diff = (g - ref).abs()
            bar = (ref.abs() * 2 * ulp).clamp_min(floor)
            if extra is not None:
                bar = bar + extra
            over = (diff / bar).max().item()
            if over >= 1:
                i = int((diff / bar).flatten().argmax())
                print(f"  {what}: worst element {i} ref {ref.flatten()[i].item():.4f} got "
                      f"{g.flatten()[i].item():.4f} (|ref| max {ref.abs().max().item():.3f})",
                      flush=True)
            rl = rel_l2(g, ref)
            assert over < 1 and rl < rl_bar, \
                f"{what}: max-abs {diff.max().item():.3e} ({over:.2f} of the bar) rel-L2 {rl:.3e}"

    check(out[:, s0:], ref, "out", False)
    check(qd.grad[:, s0:], qr.grad, "dq", True)
    extra_k = extra_v = None
    if i in _CANCEL:
        assert not p and not f16, "the named cancellation cases are bf16 without dropout"
        extra_k, extra_v, ratio_k, ratio_v = _grad_spread(qf, kf, vf, dof, causal, left)
        # the cancellation itself: some elements are under 2% of their summands' absolute sum
        assert ratio_k.min() < 0.02 and ratio_v.min() < 0.02
    check(kd.grad, kr.grad, "dk", True, extra_k)
    check(vd.grad, vr.grad, "dv", True, extra_v)
    assert math.isfinite(float(out.detach().float().abs().sum()))
