"""Pin the CPU restatement of the Mamba2 CP convolution (oracle/conv.py): the textbook
depthwise causal conv against a brute-force loop, and the per-rank halo algorithm of
mamba.py:46-101 against the convolution of the whole sequence (or of every document).
Planted mistakes in the halo must fail these checks."""

import pytest
import torch

from oracle import conv as oc


def _rnd(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def _brute(x, w, b, act):
    B, C, T = x.shape
    W = w.shape[1]
    y = torch.zeros_like(x)
    for bb in range(B):
        for c in range(C):
            for t in range(T):
                z = b[c].item() if b is not None else 0.0
                for i in range(W):
                    s = t - (W - 1) + i
                    if s >= 0:
                        z += w[c, i].item() * x[bb, c, s].item()
                y[bb, c, t] = z / (1 + torch.exp(torch.tensor(-z)).item()) if act else z
    return y


@pytest.mark.parametrize("act", [None, "silu"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_causal_conv_vs_brute_force(act, with_bias):
    x, w = _rnd(2, 3, 9, seed=1), _rnd(3, 4, seed=2)
    b = _rnd(3, seed=3) if with_bias else None
    assert torch.allclose(oc.causal_conv1d_fn(x, w, b, act), _brute(x, w, b, act), atol=1e-12)


def _split(x, world):
    return list(x.chunk(world, dim=-1))


@pytest.mark.parametrize("world", [1, 2, 3, 4])
@pytest.mark.parametrize("W", [1, 2, 4])
def test_cp_conv_equals_whole_sequence(world, W):
    x, w, b = _rnd(2, 5, 8 * world, seed=4), _rnd(5, W, seed=5), _rnd(5, seed=6)
    ref = oc.causal_conv1d_fn(x, w, b, "silu")
    got = torch.cat(oc.cp_conv(_split(x, world), w, b, "silu"), dim=-1)
    assert torch.allclose(got, ref, atol=1e-12)


def _per_document(x, w, b, act, cu):
    bounds = torch.as_tensor(cu).tolist()
    return torch.cat([oc.causal_conv1d_fn(x[..., s:e], w, b, act)
                      for s, e in zip(bounds[:-1], bounds[1:])], dim=-1)


@pytest.mark.parametrize("docs,world", [([5, 11], 2), ([2, 1, 9, 4], 2), ([3, 8, 1, 12], 4),
                                        ([24], 3)])
def test_cp_conv_packed_equals_per_document(docs, world):
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()])
    S = int(cu[-1])
    x, w, b = _rnd(1, 4, S, seed=7), _rnd(4, 4, seed=8), _rnd(4, seed=9)
    got = torch.cat(oc.cp_conv(_split(x, world), w, b, None, cu_seqlens=cu), dim=-1)
    assert torch.allclose(got, _per_document(x, w, b, None, cu), atol=1e-12)


def test_cp_conv_mutants_are_caught(monkeypatch):
    docs, world = [3, 8, 1, 12], 4
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()])
    x, w = _rnd(1, 4, 24, seed=10), _rnd(4, 4, seed=11)
    ref = _per_document(x, w, None, None, cu)
    real = oc.cp_conv

    # the halo kept across a document boundary (no mask)
    def unmasked(xs, weight, bias=None, activation=None, cu_seqlens=None):
        return real(xs, weight, bias, activation)
    got = torch.cat(unmasked(_split(x, world), w), dim=-1)
    assert not torch.allclose(got, ref, atol=1e-6)
    # the halo taken from the next rank instead of the previous one
    whole = oc.causal_conv1d_fn(x, w)
    xs = _split(x, world)
    wrong = real(xs[1:] + xs[:1], w)  # every rank prepends the wrong neighbour's tail
    assert not torch.allclose(torch.cat(wrong[-1:] + wrong[:-1], dim=-1), whole, atol=1e-6)
