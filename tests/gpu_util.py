"""Helpers shared by the GPU parity tests (seeded inputs, tolerance checks)."""

import torch

# bf16 outputs vs an fp32 reference, fp32 LSE / states
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 1e-2
F32_REL = 1e-4
# fp16 outputs (10 mantissa bits, 8 times bf16's resolution): a bar 4 times tighter in both
# measures, floored at two fp16 ulps of the value (2^-9 |ref|) for gradients above 2
F16_MAX_ABS = 5e-3
F16_REL_L2 = 2.5e-3


def seeded(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * scale


def bf16_pair(shape, seed, scale=1.0):
    """(fp32 CPU tensor holding bf16-representable values, bf16 device tensor)."""
    x = seeded(shape, seed, scale).to(torch.bfloat16)
    return x.float(), x.cuda()


def f16_pair(shape, seed, scale=1.0):
    """(fp32 CPU tensor holding fp16-representable values, fp16 device tensor)."""
    x = seeded(shape, seed, scale).to(torch.float16)
    return x.float(), x.cuda()


def rel_l2(got, ref):
    got, ref = got.double(), ref.double()
    return ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def assert_bf16_close(got, ref, what="", ulp_floor=False):
    """bf16 result vs an fp32 reference: max-abs < 2e-2 and rel-L2 < 1e-2. With
    ``ulp_floor`` (True, or a number n of ulps) the max-abs bar of an element is
    max(2e-2, n 2^-7 |ref|), n to 2n bf16 ulps of the value: for GQA-folded gradients,
    which reach |x| > 4 where one bf16 ulp (2^-5) alone exceeds 2e-2."""
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    diff = (got - ref).abs()
    err = diff.max().item()
    rl = rel_l2(got, ref)
    if ulp_floor:
        ulps = 1.0 if ulp_floor is True else float(ulp_floor)
        over = (diff / torch.clamp(ref.abs() * ulps * 2.0 ** -7, min=BF16_MAX_ABS)).max().item()
        assert over < 1 and rl < BF16_REL_L2, \
            f"{what}: max-abs {err:.3e} ({over:.2f} of the ulp-floored bar) rel-L2 {rl:.3e}"
        return
    assert err < BF16_MAX_ABS and rl < BF16_REL_L2, f"{what}: max-abs {err:.3e} rel-L2 {rl:.3e}"


def assert_f32_rel(got, ref, what="", tol=F32_REL):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got)), f"{what}: finiteness differs"
    err = ((got[fin] - ref[fin]).abs() / ref[fin].abs().clamp_min(1.0)).max().item() \
        if fin.any() else 0.0
    assert err < tol, f"{what}: rel err {err:.3e}"


def assert_f16_close(got, ref, what=""):
    """fp16 result vs an fp32 reference: per element |got - ref| < max(5e-3, 2^-9 |ref|)
    and rel-L2 < 2.5e-3."""
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    diff = (got - ref).abs()
    over = (diff / torch.clamp(ref.abs() * 2.0 ** -9, min=F16_MAX_ABS)).max().item()
    rl = rel_l2(got, ref)
    assert over < 1 and rl < F16_REL_L2, \
        f"{what}: max-abs {diff.max().item():.3e} ({over:.2f} of the bar) rel-L2 {rl:.3e}"


def keyless_prefix(sq, sk, causal, window=None):
    """The number of leading rows of a block that attend no key: with a right bound R on
    ``pos_k - pos_q`` (causal: R = 0; a flash window's right bound) the rows with
    ``q + sk - sq + R < 0``, none without one (a left bound never empties a row, since
    every bottom-right aligned ``pos_q`` is at most sk - 1). The kernels give those rows
    out 0, lse -inf and dq 0; the oracle runs on the others, whose positions are kept."""
    from oracle import ring_math as rm

    right = 0 if causal else None
    if window is not None:
        right = rm.flash_window(window, causal, sk)[1]
    return min(sq, max(0, sq - sk - right)) if right is not None else 0
