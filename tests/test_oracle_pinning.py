"""Pin the CPU oracle before trusting it: fp64 brute force, torch SDPA, closed forms
and invariants (ring == full attention, merge associativity, scan == recurrence).
Each check is chosen so that a plausible mistake (dropped term, wrong sign or
index, transposed operand, wrong ring direction) fails it; test_oracle_mutants.py
plants such mistakes and asserts these checks catch them."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ring_math as rm
from oracle import state_passing as sp

TOL32 = 2e-5


def rnd(*shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


def brute_block(q, k, v, causal, scale, left=None, right=None):
    """Pure-Python loops over (b, h, i): softmax by its definition, fp64, over the keys
    j of row i that the causal rule (j <= i + sk - sq) and the window (i + sk - sq - j
    <= left, j - (i + sk - sq) <= right) leave; a row left without keys gets out 0 and
    lse -inf."""
    b, sq, hq, d = q.shape
    sk, hkv = k.shape[1], k.shape[2]
    out = torch.zeros(b, sq, hq, d, dtype=torch.float64)
    lse = torch.zeros(b, hq, sq, dtype=torch.float64)
    for bi in range(b):
        for h in range(hq):
            kh = h // (hq // hkv)
            for i in range(sq):
                pos = i + (sk - sq)
                js = [j for j in range(sk) if ((not causal) or j <= pos)
                      and (left is None or pos - j <= left)
                      and (right is None or j - pos <= right)]
                if not js:
                    lse[bi, h, i] = -math.inf
                    continue
                s = [float((q[bi, i, h] * k[bi, j, kh]).sum()) * scale for j in js]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                z = sum(w)
                lse[bi, h, i] = m + math.log(z)
                for wj, j in zip(w, js):
                    out[bi, i, h] += (wj / z) * v[bi, j, kh]
    return out, lse


def check_block(block_fn, causal, hq, hkv, sq, sk, d=8):
    q, k, v = rnd(1, sq, hq, d, seed=1), rnd(1, sk, hkv, d, seed=2), rnd(1, sk, hkv, d, seed=3)
    out, lse = block_fn(q, k, v, causal=causal, scaling=None)
    ref_out, ref_lse = brute_block(q, k, v, causal, 1.0 / math.sqrt(d))
    assert torch.allclose(out.double(), ref_out, atol=TOL32, rtol=TOL32)
    assert torch.allclose(lse.double(), ref_lse, atol=TOL32, rtol=TOL32)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv,sq,sk", [(2, 2, 5, 5), (4, 2, 3, 7), (4, 1, 6, 6)])
def test_math_block_vs_brute_force(causal, hq, hkv, sq, sk):
    check_block(rm.math_block, causal, hq, hkv, sq, sk)


@pytest.mark.parametrize("causal", [False, True])
def test_math_block_vs_sdpa(causal):
    # library routine: SDPA with GQA; square blocks so top-left == bottom-right causal
    q, k, v = rnd(2, 16, 8, 32, seed=4), rnd(2, 16, 2, 32, seed=5), rnd(2, 16, 2, 32, seed=6)
    out, _ = rm.math_block(q, k, v, causal=causal, scaling=0.3)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         is_causal=causal, scale=0.3, enable_gqa=True)
    assert torch.allclose(out.double(), ref.transpose(1, 2), atol=TOL32)


@pytest.mark.parametrize("causal,sq,sk,left", [
    (True, 7, 7, 2), (False, 7, 7, 3), (True, 4, 9, 1), (False, 4, 9, 0), (False, 9, 4, 2),
    (True, 6, 6, 0)])
def test_math_block_window_vs_brute_force(causal, sq, sk, left):
    """The window of ring/kernels.py:68-72 (bottom-right aligned positions) against the
    row loop over the keys it leaves."""
    check_window_block(rm.math_block, causal, sq, sk, left)


def check_window_block(block_fn, causal, sq, sk, left):
    q, k, v = rnd(1, sq, 4, 8, seed=15), rnd(1, sk, 2, 8, seed=16), rnd(1, sk, 2, 8, seed=17)
    out, lse = block_fn(q, k, v, causal=causal, scaling=None, window=(left, 0))
    ref_out, ref_lse = brute_block(q, k, v, causal, 1.0 / math.sqrt(8), left)
    assert torch.allclose(out.double(), ref_out, atol=TOL32, rtol=TOL32)
    assert torch.allclose(lse.double(), ref_lse, atol=TOL32, rtol=TOL32)


def test_math_block_window_special_cases():
    """A window covering every key is no window; a causal window of 0 on a square block
    leaves each query its own key: out = v, lse = scale q.k."""
    q, k, v = rnd(1, 6, 2, 8, seed=18), rnd(1, 6, 2, 8, seed=19), rnd(1, 6, 2, 8, seed=20)
    for causal in (False, True):
        wide, _ = rm.math_block(q, k, v, causal=causal, scaling=0.4, window=(5, 0))
        plain, _ = rm.math_block(q, k, v, causal=causal, scaling=0.4)
        assert torch.allclose(wide, plain, atol=TOL32)
    out, lse = rm.math_block(q, k, v, causal=True, scaling=0.4, window=(0, 0))
    assert torch.allclose(out.double(), v, atol=TOL32)
    assert torch.allclose(lse.double(), 0.4 * (q * k).sum(-1).transpose(1, 2), atol=TOL32)


# flash attention 2's window arguments, worked by hand from its published rules (a bound
# of at least sk keys is -1; causal sets right 0; a -1 facing a bound >= 0 becomes sk):
# (causal, sq, sk, window) -> (left, right) as math_block(flash=True) applies them
_FLASH_BOUNDS = [
    (False, 7, 7, (3, -1), (3, 7)),    # left only: right bounded at sk (no effect here)
    (False, 7, 7, (-1, 2), (7, 2)),    # right only
    (False, 7, 7, (2, 1), (2, 1)),     # a band around the diagonal
    (True, 7, 7, (3, 5), (3, 0)),      # causal: right 0 whatever was asked
    (True, 6, 9, (-1, -1), (9, 0)),    # causal, no window: plain causal
    (False, 4, 9, (10, 3), (9, 3)),    # left >= sk is -1, then sk
    (False, 9, 4, (2, -1), (2, 4)),    # sq > sk + 1: the right bound sk empties rows 0..2
    (False, 9, 4, (1, 0), (1, 0)),     # non-causal (l, 0): causal band, rows 0..4 keyless
    (False, 5, 5, (-1, -1), (None, None)),
    (False, 5, 5, (6, 9), (None, None)),  # both bounds past sk: no window
]


@pytest.mark.parametrize("causal,sq,sk,window,bounds", _FLASH_BOUNDS)
def test_flash_window_vs_brute_force(causal, sq, sk, window, bounds):
    """The flash provider's window (ring/kernels.py:37-38 hands it to flash_attn_func):
    the bounds against the hand-worked table, and the block against the row loop over the
    keys they leave (rows left without keys: lse -inf, compared on the others)."""
    assert rm.flash_window(window, causal, sk) == bounds
    q, k, v = rnd(1, sq, 4, 8, seed=85), rnd(1, sk, 2, 8, seed=86), rnd(1, sk, 2, 8, seed=87)
    out, lse = rm.math_block(q, k, v, causal=causal, scaling=None, window=window, flash=True)
    ref_out, ref_lse = brute_block(q, k, v, causal, 1.0 / math.sqrt(8), *bounds)
    rows = torch.isfinite(ref_lse[0, 0])
    assert torch.isneginf(lse[:, :, ~rows]).all()
    assert torch.allclose(out[:, rows].double(), ref_out[:, rows], atol=TOL32, rtol=TOL32)
    assert torch.allclose(lse[:, :, rows].double(), ref_lse[:, :, rows], atol=TOL32, rtol=TOL32)


def test_flash_window_special_cases():
    """Where the flash window reduces to known forms: (l, -1) with sq <= sk is math_block's
    window l; a non-causal (-1, 0) is the causal block; a causal call ignores the right
    bound; a symmetric band (w, w) is SDPA with the band mask built from tril and triu."""
    q, k, v = rnd(1, 6, 2, 8, seed=88), rnd(1, 9, 2, 8, seed=89), rnd(1, 9, 2, 8, seed=90)
    for causal in (False, True):
        a, la = rm.math_block(q, k, v, causal=causal, scaling=0.4, window=(2, -1), flash=True)
        b, lb = rm.math_block(q, k, v, causal=causal, scaling=0.4, window=(2, 0))
        assert torch.allclose(a, b, atol=TOL32) and torch.allclose(la, lb, atol=TOL32)
    a, _ = rm.math_block(q, k, v, causal=False, scaling=0.4, window=(-1, 0), flash=True)
    b, _ = rm.math_block(q, k, v, causal=True, scaling=0.4)
    assert torch.allclose(a, b, atol=TOL32)
    a, _ = rm.math_block(q, k, v, causal=True, scaling=0.4, window=(3, 4), flash=True)
    b, _ = rm.math_block(q, k, v, causal=True, scaling=0.4, window=(3, 0))
    assert torch.allclose(a, b, atol=TOL32)
    w, sq, sk = 2, 6, 9
    ones = torch.ones(sq, sk, dtype=torch.bool)
    band = ones.tril(sk - sq + w) & ones.triu(sk - sq - w)
    out, _ = rm.math_block(q, k, v, causal=False, scaling=0.4, window=(w, w), flash=True)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         attn_mask=band, scale=0.4)
    assert torch.allclose(out.double(), ref.transpose(1, 2), atol=TOL32)


@pytest.mark.parametrize("causal", [True, False])
def test_allgather_ring_window_positions(causal):
    """The gather ring's one block per rank (ring/loop.py:201-228): causal, rank r's
    query i sits at global position r L + i, so the ranks together are the global
    windowed attention (brute force over the whole sequence); non-causal, every rank's
    queries sit at (P - 1) L + i against all keys."""
    P, L, left = 3, 4, 5
    qs = [rnd(1, 2, L, 8, seed=21 + r) for r in range(P)]
    ks = [rnd(1, 1, L, 8, seed=31 + r) for r in range(P)]
    vs = [rnd(1, 1, L, 8, seed=41 + r) for r in range(P)]
    outs, lses = rm.allgather_ring_forward(qs, ks, vs, causal=causal, scaling=None, window=(left, 0))
    kf = torch.cat([t.transpose(1, 2) for t in ks], 1)
    vf = torch.cat([t.transpose(1, 2) for t in vs], 1)
    sc = 1.0 / math.sqrt(8)
    if causal:
        qf = torch.cat([t.transpose(1, 2) for t in qs], 1)
        ref_o, ref_l = brute_block(qf, kf, vf, True, sc, left)
        for r in range(P):
            assert torch.allclose(outs[r].double(), ref_o[:, r * L:(r + 1) * L], atol=TOL32)
            assert torch.allclose(lses[r].double(), ref_l[:, :, r * L:(r + 1) * L], atol=TOL32)
    else:
        for r in range(P):
            ref_o, ref_l = brute_block(qs[r].transpose(1, 2), kf, vf, False, sc, left)
            assert torch.allclose(outs[r].double(), ref_o, atol=TOL32)
            assert torch.allclose(lses[r].double(), ref_l, atol=TOL32)


def test_allgather_ring_flash_window_positions():
    """The gather ring with the flash provider's window, non-causal: rank r's queries at
    (P - 1) L + i against every gathered key, bounded on both sides (brute force)."""
    P, L, left, right = 3, 4, 5, 2
    qs = [rnd(1, 2, L, 8, seed=91 + r) for r in range(P)]
    ks = [rnd(1, 1, L, 8, seed=94 + r) for r in range(P)]
    vs = [rnd(1, 1, L, 8, seed=97 + r) for r in range(P)]
    outs, lses = rm.allgather_ring_forward(qs, ks, vs, causal=False, scaling=None,
                                           window=(left, right), flash=True)
    kf = torch.cat([t.transpose(1, 2) for t in ks], 1)
    vf = torch.cat([t.transpose(1, 2) for t in vs], 1)
    for r in range(P):
        ref_o, ref_l = brute_block(qs[r].transpose(1, 2), kf, vf, False, 1.0 / math.sqrt(8),
                                   left, right)
        assert torch.allclose(outs[r].double(), ref_o, atol=TOL32)
        assert torch.allclose(lses[r].double(), ref_l, atol=TOL32)


def test_varlen_ring_window_equals_per_document():
    """The packed gather ring with a window (ring/loop.py:175-198) is, per document, the
    causal windowed attention of that document alone."""
    P, L, left = 2, 8, 3
    cu = torch.tensor([0, 5, 11, 16])
    qs = [rnd(1, 2, L, 8, seed=51 + r) for r in range(P)]
    ks = [rnd(1, 2, L, 8, seed=61 + r) for r in range(P)]
    vs = [rnd(1, 2, L, 8, seed=71 + r) for r in range(P)]
    outs, lses = rm.varlen_ring_forward(qs, ks, vs, cu, scaling=None, window=(left, 0))
    out = torch.cat(outs, 1)
    lse = torch.cat(lses, 2)
    qf, kf, vf = (torch.cat([t.transpose(1, 2) for t in ts], 1) for ts in (qs, ks, vs))
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        ref_o, ref_l = brute_block(qf[:, a:b], kf[:, a:b], vf[:, a:b], True, 1 / math.sqrt(8), left)
        assert torch.allclose(out[:, a:b].double(), ref_o, atol=TOL32)
        assert torch.allclose(lse[:, :, a:b].double(), ref_l, atol=TOL32)


def _varlen_rows_case(b=2, P=2, L=8, hq=2, hkv=1, d=8):
    """Per-row documents (ring/loop.py:178): row 0 packs [5, 6, 5], row 1 [9, 7]; the
    flattened cu_seqlens covers both rows."""
    cu = torch.tensor([0, 5, 11, 16, 25, 32])
    qs = [rnd(b, hq, L, d, seed=81 + r).requires_grad_(True) for r in range(P)]
    ks = [rnd(b, hkv, L, d, seed=91 + r).requires_grad_(True) for r in range(P)]
    vs = [rnd(b, hkv, L, d, seed=101 + r).requires_grad_(True) for r in range(P)]
    return cu, qs, ks, vs


def check_varlen_rows(fwd, causal):
    """``fwd(qs, ks, vs, cu, causal=...)`` against brute-force attention of every document
    alone in its own row (fp64 loops), values; and its autograd gradients against those of
    per-document attention (fp64 torch)."""
    cu, qs, ks, vs = _varlen_rows_case()
    b, P, L = qs[0].shape[0], len(qs), qs[0].shape[2]
    S = P * L
    outs, lses = fwd(qs, ks, vs, cu, causal=causal)
    out, lse = torch.cat(outs, 1), torch.cat(lses, 2)
    qf, kf, vf = (torch.cat([t.transpose(1, 2) for t in ts], 1) for ts in (qs, ks, vs))
    sc = 1 / math.sqrt(qf.shape[-1])
    bounds = cu.tolist()
    ref = torch.zeros_like(out, dtype=torch.float64)
    for row in range(b):
        for a, z in zip(bounds[:-1], bounds[1:]):
            lo, hi = max(a, row * S) - row * S, min(z, (row + 1) * S) - row * S
            if lo >= hi:
                continue
            ro, rl = brute_block(qf[row:row + 1, lo:hi].detach(), kf[row:row + 1, lo:hi].detach(),
                                 vf[row:row + 1, lo:hi].detach(), causal, sc)
            assert torch.allclose(out[row:row + 1, lo:hi].detach().double(), ro, atol=TOL32)
            assert torch.allclose(lse[row:row + 1, :, lo:hi].detach().double(), rl, atol=TOL32)
            # differentiable per-document reference for the gradients
            qd, kd, vd = qf[row:row + 1, lo:hi], kf[row:row + 1, lo:hi], vf[row:row + 1, lo:hi]
            od, _ = rm.full_attention(qd, kd, vd, causal=causal, scaling=sc)
            ref[row:row + 1, lo:hi] = od
    dout = rnd(*out.shape, seed=111)
    g_ref = torch.autograd.grad((ref * dout).sum(), [*qs, *ks, *vs])
    g_got = torch.autograd.grad((out * dout).sum(), [*qs, *ks, *vs])
    for a, z in zip(g_got, g_ref):
        assert torch.allclose(a, z, atol=TOL32)


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_ring_per_row_documents(causal):
    """The packed ring gives each batch row its own documents (ring/loop.py:178) and, with
    ``causal=False``, every key of the query's document (:149,183-184)."""
    check_varlen_rows(rm.varlen_ring_forward, causal)


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_ring_dropout_coordinates(causal):
    """One document per row: the packed ring with a dropout seed equals the gather ring
    with that seed (the same mask over (row, head, r L + i, gathered key))."""
    P, L, b, p, seed = 3, 8, 2, 0.3, 1234
    cu = torch.tensor([0, P * L, 2 * P * L])
    qs = [rnd(b, 2, L, 8, seed=121 + r) for r in range(P)]
    ks = [rnd(b, 2, L, 8, seed=131 + r) for r in range(P)]
    vs = [rnd(b, 2, L, 8, seed=141 + r) for r in range(P)]
    o1, l1 = rm.varlen_ring_forward(qs, ks, vs, cu, causal=causal, dropout=p, drop_seed=seed)
    o2, l2 = rm.allgather_ring_forward(qs, ks, vs, causal=causal, dropout=p, drop_seed=seed)
    o0, _ = rm.varlen_ring_forward(qs, ks, vs, cu, causal=causal)
    for r in range(P):
        assert torch.allclose(o1[r], o2[r], atol=TOL32)
        assert torch.allclose(l1[r], l2[r], atol=TOL32)
        assert not torch.allclose(o1[r], o0[r], atol=1e-3)  # the mask drops something


def _fmix32_int(x):
    """MurmurHash3's fmix32 on a Python int (an implementation independent of numpy's
    wrap-around arithmetic)."""
    m = 0xFFFFFFFF
    x &= m
    x ^= x >> 16
    x = (x * 0x85EBCA6B) & m
    x ^= x >> 13
    x = (x * 0xC2B2AE35) & m
    x ^= x >> 16
    return x


def test_fmix32_matches_integer_arithmetic_and_is_a_bijection():
    import numpy as np

    g = np.random.default_rng(0)
    xs = np.concatenate([g.integers(0, 1 << 32, 2000, dtype=np.uint64).astype(np.uint32),
                         np.array([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF], dtype=np.uint32)])
    got = rm.fmix32(xs)
    assert [int(v) for v in got] == [_fmix32_int(int(x)) for x in xs]
    # each step (xor-shift, odd multiply) is invertible: no two inputs share an output
    assert len(np.unique(rm.fmix32(np.arange(1 << 20, dtype=np.uint32)))) == 1 << 20


def test_dropout_keep_matches_its_definition():
    """dropout_keep on a few elements, recomputed from the formula with Python ints; the
    threshold is floor(p 2^32) of p as the C ABI's fp32 ``dropout_p`` holds it (struct
    round trip), and an element whose hash falls between that threshold and the float64 one
    is dropped."""
    import struct

    seed, bh, p = 0x0123456789ABCDEF, 7, 0.3
    keep = rm.dropout_keep(seed, bh, [0, 5, 1000], [3, 64, 77777], p)
    bhmix = _fmix32_int((seed & 0xFFFFFFFF) ^ _fmix32_int((seed >> 32) ^ (bh * 0x9E3779B9)))
    p32 = struct.unpack("f", struct.pack("f", p))[0]
    thr = int(p32 * 2 ** 32)
    assert thr == 1288490240 and int(p * 2 ** 32) == 1288490188
    for i, q in enumerate([0, 5, 1000]):
        for j, k in enumerate([3, 64, 77777]):
            u = _fmix32_int(bhmix ^ ((q * 0x85EBCA77) & 0xFFFFFFFF) ^ ((k * 0xC2B2AE3D) & 0xFFFFFFFF))
            assert bool(keep[i, j]) == (u >= thr)
    # seed 1145, bh 24, query 202, key 74: hash 1288490235, between the two thresholds
    u = _fmix32_int(_fmix32_int((1145 & 0xFFFFFFFF) ^ _fmix32_int(0 ^ (24 * 0x9E3779B9)))
                    ^ ((202 * 0x85EBCA77) & 0xFFFFFFFF) ^ ((74 * 0xC2B2AE3D) & 0xFFFFFFFF))
    assert 1288490188 <= u < 1288490240
    assert not rm.dropout_keep(1145, 24, [202], [74], 0.3)[0, 0]


@pytest.mark.parametrize("p", [0.1, 0.3, 0.7])
def test_dropout_keep_rate_and_independence(p):
    """Keep rate 1 - p within 5 sigma over 4M elements; neighbouring elements (along q and
    along k) and two heads kept together at rate (1 - p)^2, as independent draws are."""
    import numpy as np

    n = 2048
    keep = rm.dropout_keep(99, 3, np.arange(n), np.arange(n), p)
    sig = math.sqrt(p * (1 - p) / keep.size)
    assert abs(keep.mean() - (1 - p)) < 5 * sig
    pair_sig = math.sqrt((1 - p) ** 2 * (1 - (1 - p) ** 2) / keep.size)
    assert abs((keep[:, 1:] & keep[:, :-1]).mean() - (1 - p) ** 2) < 6 * pair_sig
    assert abs((keep[1:] & keep[:-1]).mean() - (1 - p) ** 2) < 6 * pair_sig
    other = rm.dropout_keep(99, 4, np.arange(n), np.arange(n), p)
    assert abs((keep & other).mean() - (1 - p) ** 2) < 6 * pair_sig
    rows = keep.mean(1)  # per-row rates: binomial spread, no biased rows
    assert rows.std() < 1.5 * math.sqrt(p * (1 - p) / n)


def check_dropout_unbiased(block_fn):
    """Averaged over seeds, the dropped block equals the undropped one (E[M / (1 - p)] = 1,
    lse undropped)."""
    p = 0.25
    q, k, v = rnd(1, 16, 2, 8, seed=80), rnd(1, 16, 2, 8, seed=81), rnd(1, 16, 2, 8, seed=82)
    ref, ref_lse = rm.math_block(q, k, v, causal=True, scaling=None)
    acc = torch.zeros_like(ref, dtype=torch.float64)
    n = 400
    for sd in range(n):
        o, lse = block_fn(q, k, v, causal=True, scaling=None, dropout=p, drop_seed=sd)
        assert torch.allclose(lse.double(), ref_lse.double(), atol=TOL32)
        acc += o.double()
    # standard error of the mean of out_i = sum_j P_ij m_ij v_j, m in {0, 1/(1-p)}:
    # Var = sum_j P_ij^2 v_j^2 p / (1 - p)
    scores = q.transpose(1, 2).double() @ k.transpose(1, 2).double().transpose(-1, -2)
    pr = torch.exp(scores / math.sqrt(8) - ref_lse[..., None].double())
    pr = pr.masked_fill(~torch.ones(16, 16, dtype=torch.bool).tril(), 0.0)
    var = (pr ** 2) @ (v.transpose(1, 2).double() ** 2) * p / (1 - p)
    se = (var / n).sqrt().transpose(1, 2)
    z = ((acc / n - ref.double()).abs() / (se + 1e-9)).max().item()
    assert z < 5.5, f"mean of dropped outputs is {z:.1f} standard errors off"


def test_dropout_block_unbiased_and_lse_undropped():
    check_dropout_unbiased(rm.math_block)


def test_dropout_block_gradients_are_the_derivative():
    """The dropped block's autograd gradients against finite differences (fp64, one seed)."""
    q, k, v = (rnd(1, 5, 2, 4, seed=s).requires_grad_(True) for s in (83, 84, 85))

    def f(q, k, v):
        return rm.math_block(q, k, v, causal=False, scaling=0.7, dropout=0.4, drop_seed=5,
                             drop_q0=3, drop_k0=11)[0].double()

    qt, kt, vt = (t.detach().double().requires_grad_(True) for t in (q, k, v))
    # the oracle computes in fp32: gradcheck an fp64 copy of its dropped path, then check
    # the oracle's own autograd against that copy's gradients
    assert torch.autograd.gradcheck(_math_block_f64, (qt, kt, vt), eps=1e-6, atol=1e-5)
    f(q, k, v).sum().backward()
    _math_block_f64(qt, kt, vt).sum().backward()
    for a, b in ((q, qt), (k, kt), (v, vt)):
        assert torch.allclose(a.grad.double(), b.grad, atol=1e-4)


def _math_block_f64(q, k, v):
    """math_block's dropped path in fp64 (same mask), for gradcheck."""
    qt, kt, vt = (t.transpose(1, 2) for t in (q, k, v))
    scores = (qt @ kt.transpose(-1, -2)) * 0.7
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.exp(scores - lse.unsqueeze(-1))
    probs = probs * rm.dropout_scale_mask(5, 1, 2, 5, 5, 0.4, 3, 11).double()
    return (probs @ vt).transpose(1, 2)


def check_merge(merge_fn):
    """merge(attn(Q, K1), attn(Q, K2)) == attn(Q, [K1; K2]) in out and lse."""
    q = rnd(1, 6, 2, 8, seed=7)
    k1, v1 = rnd(1, 5, 2, 8, seed=8), rnd(1, 5, 2, 8, seed=9)
    k2, v2 = rnd(1, 4, 2, 8, seed=10) + 1.5, rnd(1, 4, 2, 8, seed=11)
    o1, l1 = rm.math_block(q, k1, v1, causal=False, scaling=None)
    o2, l2 = rm.math_block(q, k2, v2, causal=False, scaling=None)
    out, lse = merge_fn(None, None, o1, l1)
    out, lse = merge_fn(out, lse, o2, l2)
    ref_o, ref_l = rm.math_block(q, torch.cat([k1, k2], 1), torch.cat([v1, v2], 1), causal=False,
                                 scaling=None)
    assert torch.allclose(out.double(), ref_o.double(), atol=TOL32)
    assert torch.allclose(lse.squeeze(-1).transpose(1, 2).double(), ref_l.double(), atol=TOL32)


def test_merge_equals_concatenated_attention():
    check_merge(rm.update_out_and_lse)


def test_merge_neg_inf_block_is_noop_and_commutes():
    q = rnd(1, 3, 1, 4, seed=12)
    o1, l1 = rm.math_block(q, rnd(1, 3, 1, 4, seed=13), rnd(1, 3, 1, 4, seed=14), causal=False,
                           scaling=None)
    o2, l2 = rm.math_block(q, rnd(1, 2, 1, 4, seed=15), rnd(1, 2, 1, 4, seed=16), causal=False,
                           scaling=None)
    a, la = rm.update_out_and_lse(*rm.update_out_and_lse(None, None, o1, l1), o2, l2)
    b, lb = rm.update_out_and_lse(*rm.update_out_and_lse(None, None, o2, l2), o1, l1)
    assert torch.allclose(a, b, atol=1e-6) and torch.allclose(la, lb, atol=1e-6)
    c, lc = rm.update_out_and_lse(a, la, torch.zeros_like(o1), torch.full_like(l1, -math.inf))
    assert torch.equal(c, a) and torch.equal(lc, la)


def zigzag_case(world, half, hq=4, hkv=4, d=8, seed=0, cu=None):
    S = 2 * world * half
    q, k, v = rnd(1, S, hq, d, seed=seed + 1), rnd(1, S, hkv, d, seed=seed + 2), \
        rnd(1, S, hkv, d, seed=seed + 3)
    dout = rnd(1, S, hq, d, seed=seed + 4)
    return q, k, v, dout


def check_ring(world, half, hq=4, hkv=4, cu=None, fwd=rm.zigzag_ring_forward,
               bwd=rm.zigzag_ring_backward, tol=1e-5):
    """The emulated zigzag ring equals full (doc-)causal attention, values and grads."""
    q, k, v, dout = zigzag_case(world, half, hq, hkv)
    idx = [rm.zigzag_gidx(r, half, world) for r in range(world)]
    shard = lambda t: [t[:, i].transpose(1, 2).contiguous() for i in idx]  # noqa: E731
    outs, lses = fwd(shard(q), shard(k), shard(v), cu_seqlens=cu)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref, ref_lse = rm.full_attention(qr, kr, vr, causal=True, cu_seqlens=cu)
    ref.backward(dout)
    err = 0.0
    for r in range(world):
        err = max(err, (outs[r].double() - ref.detach()[:, idx[r]]).abs().max().item())
        err = max(err, (lses[r].double() - ref_lse.detach()[:, :, idx[r]]).abs().max().item())
    dqs, dks, dvs = bwd([dout[:, i] for i in idx], shard(q), shard(k), shard(v), outs, lses,
                        cu_seqlens=cu)
    for r in range(world):
        err = max(err, (dqs[r].double() - qr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
        err = max(err, (dks[r].double() - kr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
        err = max(err, (dvs[r].double() - vr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
    assert err < tol, f"ring vs full attention err {err}"


@pytest.mark.parametrize("world", [1, 2, 4, 8])
def test_zigzag_ring_equals_full_causal(world):
    check_ring(world, half=3)


def test_zigzag_ring_gqa():
    check_ring(4, half=2, hq=4, hkv=2)


@pytest.mark.parametrize("seq_len,docs,world", [(16, [6, 10], 2), (16, [5, 7, 4], 2),
                                                (32, [10, 9, 13], 4), (24, [3, 3, 6, 4, 8], 4)])
def test_zigzag_varlen_equals_per_document(seq_len, docs, world):
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()], dtype=torch.int32)
    half = seq_len // (2 * world)
    check_ring(world, half, cu=cu)


def check_contiguous(world, L, *, causal=True, hq=4, hkv=4, cu=None, fwd=None, bwd=None,
                     tol=1e-5):
    """An emulated contiguous ring (p2p or DistFlash restatement) equals full (doc-)causal
    or full non-causal attention, values and grads."""
    fwd = fwd or (lambda *a, **kw: rm.contiguous_ring_forward(*a, causal=causal, **kw))
    bwd = bwd or (lambda *a, **kw: rm.contiguous_ring_backward(*a, causal=causal, **kw))
    S = world * L
    q, k, v = rnd(1, S, hq, 8, seed=1), rnd(1, S, hkv, 8, seed=2), rnd(1, S, hkv, 8, seed=3)
    dout = rnd(1, S, hq, 8, seed=4)
    idx = [rm.contiguous_gidx(r, L) for r in range(world)]
    shard = lambda t: [t[:, i].transpose(1, 2).contiguous() for i in idx]  # noqa: E731
    outs, lses = fwd(shard(q), shard(k), shard(v), cu_seqlens=cu)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref, ref_lse = rm.full_attention(qr, kr, vr, causal=causal, cu_seqlens=cu)
    ref.backward(dout)
    err = 0.0
    for r in range(world):
        err = max(err, (outs[r].double() - ref.detach()[:, idx[r]]).abs().max().item())
        err = max(err, (lses[r].double() - ref_lse.detach()[:, :, idx[r]]).abs().max().item())
    dqs, dks, dvs = bwd([dout[:, i] for i in idx], shard(q), shard(k), shard(v), outs, lses,
                        cu_seqlens=cu)
    for r in range(world):
        err = max(err, (dqs[r].double() - qr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
        err = max(err, (dks[r].double() - kr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
        err = max(err, (dvs[r].double() - vr.grad[:, idx[r]].transpose(1, 2)).abs().max().item())
    assert err < tol, f"contiguous ring vs full attention err {err}"


@pytest.mark.parametrize("world", [1, 2, 3, 4])
@pytest.mark.parametrize("causal", [True, False])
def test_contiguous_ring_equals_full(world, causal):
    check_contiguous(world, 5, causal=causal)


def test_contiguous_ring_gqa():
    check_contiguous(4, 4, hq=4, hkv=2)


@pytest.mark.parametrize("docs,world", [([6, 10], 2), ([10, 9, 13], 4), ([3, 3, 6, 4, 8], 4)])
def test_contiguous_varlen_equals_per_document(docs, world):
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()], dtype=torch.int32)
    check_contiguous(world, sum(docs) // world, cu=cu)


@pytest.mark.parametrize("world", [1, 2, 3, 4, 5])
def test_distflash_equals_full_causal(world):
    check_contiguous(world, 4, fwd=rm.distflash_forward, bwd=rm.distflash_backward)


def test_distflash_varlen_and_gqa():
    cu = torch.tensor([0, 7, 9, 20, 24], dtype=torch.int32)
    check_contiguous(4, 6, hq=4, hkv=2, cu=cu, fwd=rm.distflash_forward,
                     bwd=rm.distflash_backward)


def test_full_attention_per_doc_equals_sdpa_per_doc():
    docs = [5, 7, 4]
    cu = torch.tensor([0, 5, 12, 16])
    q, k, v = rnd(1, 16, 2, 8, seed=20), rnd(1, 16, 2, 8, seed=21), rnd(1, 16, 2, 8, seed=22)
    out, _ = rm.full_attention(q, k, v, causal=True, cu_seqlens=cu)
    parts = []
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        parts.append(F.scaled_dot_product_attention(
            q[:, a:b].transpose(1, 2), k[:, a:b].transpose(1, 2), v[:, a:b].transpose(1, 2),
            is_causal=True).transpose(1, 2))
    assert sum(docs) == 16
    assert torch.allclose(out, torch.cat(parts, 1), atol=1e-10)


def test_attention_rows_matches_full():
    q, k, v = rnd(1, 24, 4, 8, seed=30), rnd(1, 24, 2, 8, seed=31), rnd(1, 24, 2, 8, seed=32)
    ref, ref_lse = rm.full_attention(q, k, v, causal=True)
    pos = torch.tensor([0, 5, 23])
    out, lse = rm.attention_rows(q[:, pos], k, v, pos)
    assert torch.allclose(out, ref[:, pos], atol=1e-10)
    assert torch.allclose(lse, ref_lse[:, :, pos], atol=1e-10)


# ---------------------------------------------------------------- scan
def check_scan(scan_fn, world=2, T=8, d=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = (torch.rand(1, T, d, generator=g, dtype=torch.float64) * 0.9 + 0.05).requires_grad_(True)
    b = torch.randn(1, T, d, generator=g, dtype=torch.float64).requires_grad_(True)
    ref = sp.local_linear_scan(a, b)
    got = scan_fn(a, b, world)
    assert torch.allclose(got, ref, atol=1e-10)
    ga = torch.autograd.grad(ref.square().sum(), (a, b))
    gb = torch.autograd.grad(got.square().sum(), (a, b))
    for x, y in zip(ga, gb):
        assert torch.allclose(x, y, atol=1e-10)


@pytest.mark.parametrize("world", [1, 2, 4, 8])
def test_cp_linear_scan_equals_global(world):
    check_scan(sp.cp_linear_scan_emulated, world=world, T=16)


def test_local_scan_closed_forms():
    b = rnd(2, 10, 3, seed=40)
    assert torch.allclose(sp.local_linear_scan(torch.ones_like(b), b), b.cumsum(1), atol=1e-12)
    a = torch.rand(2, 10, 3, dtype=torch.float64) + 0.5
    b0 = torch.zeros_like(b)
    b0[:, 0] = 1.0
    assert torch.allclose(sp.local_linear_scan(a, b0), a.cumprod(1) / a[:, :1], atol=1e-12)
    assert torch.allclose(sp.local_linear_scan_vec(a, b), sp.local_linear_scan(a, b), atol=1e-12)


def test_gated_linear_attention_cast():
    """S_t = g_t S_{t-1} + k_t v_t^T, o_t = q_t S_t via the scan (tests/test_state_passing.py:61-115)."""
    g = torch.Generator().manual_seed(1)
    T, dk, dv = 8, 4, 5
    q, k, v = (torch.randn(T, n, generator=g, dtype=torch.float64) for n in (dk, dk, dv))
    gate = torch.rand(T, generator=g, dtype=torch.float64) * 0.9 + 0.05
    S = torch.zeros(dk, dv, dtype=torch.float64)
    ref = []
    for t in range(T):
        S = gate[t] * S + torch.outer(k[t], v[t])
        ref.append(q[t] @ S)
    ref = torch.stack(ref)
    kv = torch.einsum("ti,tj->tij", k, v).reshape(1, T, dk * dv)
    a = gate.reshape(1, T, 1).expand(1, T, dk * dv)
    states = sp.cp_linear_scan_emulated(a, kv, 2).reshape(T, dk, dv)
    assert torch.allclose(torch.einsum("ti,tij->tj", q, states), ref, atol=1e-10)


@pytest.mark.parametrize("world", [2, 4, 8])
def test_mamba2_prefix_equals_global_ssd(world):
    torch.manual_seed(0)
    b, T, H, d, G, n = 1, 16, 2, 3, 1, 4
    x = torch.randn(b, T, H, d, dtype=torch.float64)
    dt = torch.rand(b, T, H, dtype=torch.float64) * 0.1
    A = -torch.rand(H, dtype=torch.float64)
    B = torch.randn(b, T, G, n, dtype=torch.float64)
    C = torch.randn(b, T, G, n, dtype=torch.float64)
    ref_out, _ = sp.ssd_reference(x, dt, A, B, C)
    n_loc = T // world
    finals, decays, parts = [], [], []
    for r in range(world):
        sl = slice(r * n_loc, (r + 1) * n_loc)
        out_c, h_final = sp.ssd_reference(x[:, sl], dt[:, sl], A, B[:, sl], C[:, sl])
        cum_A = torch.cumsum(A[None, None, :] * dt[:, sl], dim=1)
        finals.append(h_final)
        decays.append(torch.exp(cum_A[:, -1]))
        parts.append((out_c, h_final, sl, cum_A))
    prefixes = sp.cp_state_prefix_emulated(finals, decays)
    for r, (out_c, h_final, sl, cum_A) in enumerate(parts):
        corrected, _ = sp.mamba2_cp_correction(out_c, h_final, C[:, sl], cum_A, prefixes[r], H, d)
        assert (corrected - ref_out[:, sl]).abs().max().item() < 1e-6


@pytest.mark.parametrize("world", [1, 2, 4])
@pytest.mark.parametrize("softplus", [False, True])
def test_cp_scan_wrapper_equals_global_ssd_values_and_grads(world, softplus):
    """The CP wrapper (chunk decay from dt, prefix, correction) applied to each shard's
    zero-state SSD equals the global SSD, in values and in the gradients w.r.t. dt, A,
    dt_bias, x and C (the shards' SSD runs inside the same graph)."""
    torch.manual_seed(1)
    b, T, H, d, G, n = 1, 16, 2, 3, 1, 4
    x = torch.randn(b, T, H, d, dtype=torch.float64, requires_grad=True)
    dt_raw = (torch.randn(b, T, H, dtype=torch.float64) * 0.5 - 2.0).requires_grad_(True)
    bias = (torch.randn(H, dtype=torch.float64) * 0.1).requires_grad_(True)
    A = (-torch.rand(H, dtype=torch.float64) - 0.1).requires_grad_(True)
    B = torch.randn(b, T, G, n, dtype=torch.float64)
    C = torch.randn(b, T, G, n, dtype=torch.float64, requires_grad=True)
    dt_eff = torch.nn.functional.softplus(dt_raw + bias) if softplus else dt_raw.abs() * 0.1
    ref_out, ref_state = sp.ssd_reference(x, dt_eff, A, B, C)
    n_loc = T // world
    outs, finals, dts, Cs = [], [], [], []
    for r in range(world):
        sl = slice(r * n_loc, (r + 1) * n_loc)
        o, h = sp.ssd_reference(x[:, sl], dt_eff[:, sl], A, B[:, sl], C[:, sl])
        outs.append(o)
        finals.append(h)
        dts.append(dt_raw[:, sl] if softplus else dt_eff[:, sl])
        Cs.append(C[:, sl])
    res = sp.cp_scan_wrapper_emulated(outs, finals, dts, A, Cs, H, d,
                                      dt_bias=bias if softplus else None, dt_softplus=softplus)
    got = torch.cat([o for o, _ in res], dim=1)
    assert (got - ref_out).abs().max().item() < 1e-6
    assert (res[-1][1] - ref_state).abs().max().item() < 1e-6
    w = torch.randn_like(ref_out)
    gs = torch.autograd.grad((got * w).sum() + res[-1][1].sum(), (x, dt_raw, A, C, bias),
                             allow_unused=True, retain_graph=True)
    rs = torch.autograd.grad((ref_out * w).sum() + ref_state.sum(), (x, dt_raw, A, C, bias),
                             allow_unused=True)
    for g, r in zip(gs, rs):
        if r is None:
            continue
        assert (g - r).abs().max().item() < 1e-5, (g - r).abs().max().item()


def _ssd_segments(x, dt, A, B, C, seg):
    """SSD with the state reset at every segment start (packed sequences): per-segment
    ssd_reference runs, concatenated; returns (out, final state of the last segment)."""
    outs, h = [], None
    bounds = [0] + [t for t in range(1, seg.numel()) if seg[t] != seg[t - 1]] + [seg.numel()]
    for lo, hi in zip(bounds, bounds[1:]):
        o, h = sp.ssd_reference(x[:, lo:hi], dt[:, lo:hi], A, B[:, lo:hi], C[:, lo:hi])
        outs.append(o)
    return torch.cat(outs, 1), h


@pytest.mark.parametrize("cut", [5, 11])
def test_mamba2_correction_packed_sequences(cut):
    """Two packed documents over two ranks: per-rank SSD with resets at the document
    boundary, the single-hop prefix and the seq_idx-masked correction equal the
    per-document SSD (strategies/mamba.py:68-98,101-139)."""
    torch.manual_seed(1)
    b, T, H, d, G, n = 1, 16, 2, 3, 1, 4
    x = torch.randn(b, T, H, d, dtype=torch.float64)
    dt = torch.rand(b, T, H, dtype=torch.float64) * 0.1
    A = -torch.rand(H, dtype=torch.float64)
    B = torch.randn(b, T, G, n, dtype=torch.float64)
    C = torch.randn(b, T, G, n, dtype=torch.float64)
    doc = (torch.arange(T) >= cut).long()                 # document id per token
    ref_out, _ = _ssd_segments(x, dt, A, B, C, doc)
    world, n_loc = 2, T // 2
    shards = [slice(r * n_loc, (r + 1) * n_loc) for r in range(world)]
    finals, decays, parts = [], [], []
    for sl in shards:
        seg = doc[sl]
        out_c, h_final = _ssd_segments(x[:, sl], dt[:, sl], A, B[:, sl], C[:, sl], seg)
        cum_A = torch.cumsum(A[None, None, :] * dt[:, sl], dim=1)
        finals.append(h_final)
        decays.append(torch.exp(cum_A[:, -1]))
        seq_idx = (seg - seg[0]).reshape(1, -1)             # 0 = continues the incoming document
        parts.append((out_c, h_final, sl, cum_A, seq_idx))
    # single hop: rank 1 receives rank 0's final state
    prefixes = [torch.zeros_like(finals[0]), finals[0]]
    for r, (out_c, h_final, sl, cum_A, seq_idx) in enumerate(parts):
        corrected, _ = sp.mamba2_cp_correction(out_c, h_final, C[:, sl], cum_A, prefixes[r], H, d,
                                               seq_idx=seq_idx)
        assert (corrected - ref_out[:, sl]).abs().max().item() < 1e-6


def _correction_case(seed, seq_kind):
    g = torch.Generator().manual_seed(seed)
    b, T, H, d, G, n = 2, 12, 4, 3, 2, 5
    out = torch.randn(b, T, H * d, generator=g, dtype=torch.float64)   # fp64: no output rounding
    h_final = torch.randn(b, H, d, n, generator=g, dtype=torch.float64)
    C = torch.randn(b, T, G, n, generator=g, dtype=torch.float64)
    cum_A = torch.cumsum(-torch.rand(b, T, H, generator=g, dtype=torch.float64) * 0.3, dim=1)
    h_prev = torch.randn(b, H, d, n, generator=g, dtype=torch.float64)
    seq_idx = None
    if seq_kind != "none":
        seq_idx = torch.zeros(b, T, dtype=torch.long)
        seq_idx[0, 7:] = 1
        if seq_kind == "fresh_last":
            seq_idx[1, 10:] = 3
    gy = torch.randn(b, T, H * d, generator=g, dtype=torch.float64)
    ghf = torch.randn(b, H, d, n, generator=g, dtype=torch.float64)
    return (out, h_final, C, cum_A, h_prev, H, d), seq_idx, gy, ghf


def _correction_loss(args, seq_idx, gy, ghf, C, cum_A, h_prev):
    out, h_final, _, _, _, H, d = args
    y, hf = sp.mamba2_cp_correction(out, h_final, C, cum_A, h_prev, H, d, seq_idx=seq_idx)
    return (y.double() * gy).sum() + (hf.double() * ghf).sum()


@pytest.mark.parametrize("seq_kind", ["none", "packed", "fresh_last"])
def test_mamba2_correction_backward_pinned(seq_kind):
    """The gradients the correction's backward kernels produce (dC, dcumA, dh_prev) are
    autograd through the oracle's restatement of strategies/mamba.py:101-139; pin them
    (a) against central finite differences of the same loss and (b) against the closed
    forms the kernels implement: with e = mask exp(cumA), S = C.H_in,
    dC = sum_{h in g} e G H_in, dcumA = e sum_d G S (+ e_last sum Gs H_in at T-1 when the
    state is updated), dh_prev = sum_t e G C (+ e_last Gs)."""
    args, seq_idx, gy, ghf = _correction_case(5, seq_kind)
    out, h_final, C, cum_A, h_prev, H, d = args
    leaves = [t.clone().requires_grad_(True) for t in (C, cum_A, h_prev)]
    grads = torch.autograd.grad(_correction_loss(args, seq_idx, gy, ghf, *leaves), leaves)

    # (a) finite differences (the oracle computes in fp32 inside: eps 1e-3, loose bound)
    g = torch.Generator().manual_seed(6)
    for which, base in enumerate((C, cum_A, h_prev)):
        for _ in range(6):
            idx = tuple(int(torch.randint(s, (1,), generator=g)) for s in base.shape)
            vals = []
            for sgn in (1.0, -1.0):
                pert = [C, cum_A, h_prev]
                t = base.clone()
                t[idx] += sgn * 1e-3
                pert[which] = t
                vals.append(_correction_loss(args, seq_idx, gy, ghf, *pert).item())
            fd = (vals[0] - vals[1]) / 2e-3
            an = grads[which][idx].item()
            assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (which, idx, fd, an)

    # (b) closed forms
    b, T = C.shape[:2]
    G, n = C.shape[2], C.shape[3]
    hpg = H // G
    mask = torch.ones(b, T, dtype=torch.float64) if seq_idx is None else (seq_idx == 0).double()
    e = mask[..., None] * torch.exp(cum_A)                              # [b, T, H]
    Cx = C.repeat_interleave(hpg, dim=2)                                # [b, T, H, n]
    Gy = gy.reshape(b, T, H, d)
    S = torch.einsum("bthn,bhdn->bthd", Cx, h_prev)
    dA = e * (Gy * S).sum(-1)
    dH = torch.einsum("bthd,bthn->bhdn", Gy * e[..., None], Cx)
    dCx = torch.einsum("bthd,bhdn->bthn", Gy * e[..., None], h_prev)
    dC = dCx.reshape(b, T, G, hpg, n).sum(3)
    upd = seq_idx is None or not bool(seq_idx[:, -1].any())
    if upd:
        el = torch.exp(cum_A[:, -1])
        dA[:, -1] += el * (ghf * h_prev).sum((-1, -2))
        dH = dH + el[..., None, None] * ghf
    for got, ref in zip(grads, (dC, dA, dH)):
        assert (got - ref).abs().max().item() <= 1e-4 * max(1.0, ref.abs().max().item())


@pytest.mark.parametrize("G", [1, 2])
def test_chunk_state_equals_ssd_final_state(G):
    """The closed-form shard state equals the SSD recurrence's final state, and with a
    document start t0 the state of the last document run alone (the scan restarts)."""
    torch.manual_seed(3)
    b, T, H, d, n = 2, 24, 4, 3, 5
    x = torch.randn(b, T, H, d, dtype=torch.float64)
    e = torch.rand(b, T, H, dtype=torch.float64) * 0.3
    A = -torch.rand(H, dtype=torch.float64) - 0.2
    B = torch.randn(b, T, G, n, dtype=torch.float64)
    C = torch.randn(b, T, G, n, dtype=torch.float64)
    cum = torch.cumsum(A[None, None, :] * e, dim=1)
    _, h_ref = sp.ssd_reference(x, e, A, B, C)
    assert (sp.chunk_state(x, B, e, cum) - h_ref).abs().max().item() < 1e-12
    t0 = torch.tensor([7, 0])
    got = sp.chunk_state(x, B, e, cum, t0)
    for r in range(b):
        lo = int(t0[r])
        _, h = sp.ssd_reference(x[r:r + 1, lo:], e[r:r + 1, lo:], A, B[r:r + 1, lo:],
                                C[r:r + 1, lo:])
        assert (got[r] - h[0]).abs().max().item() < 1e-12


def test_chunk_state_gradients_equal_recurrence_gradients():
    """Gradients of the closed form (through cum_A = cumsum(A e), e = softplus(dt + bias))
    equal autograd through the SSD recurrence w.r.t. x, B, dt, A and dt_bias."""
    torch.manual_seed(4)
    b, T, H, d, G, n = 1, 12, 2, 3, 1, 4
    x = torch.randn(b, T, H, d, dtype=torch.float64, requires_grad=True)
    B = torch.randn(b, T, G, n, dtype=torch.float64, requires_grad=True)
    C = torch.randn(b, T, G, n, dtype=torch.float64)
    dt = (torch.randn(b, T, H, dtype=torch.float64) - 1.5).requires_grad_(True)
    bias = (torch.randn(H, dtype=torch.float64) * 0.1).requires_grad_(True)
    A = (-torch.rand(H, dtype=torch.float64) - 0.2).requires_grad_(True)
    cum, _ = sp.chunk_decay(dt, A, bias, True)
    e = torch.nn.functional.softplus(dt + bias)
    S = sp.chunk_state(x, B, e, cum)
    _, h_ref = sp.ssd_reference(x, e, A, B, C)
    gw = torch.randn_like(S)
    gs = torch.autograd.grad((S * gw).sum(), (x, B, dt, A, bias), retain_graph=True)
    rs = torch.autograd.grad((h_ref * gw).sum(), (x, B, dt, A, bias))
    for g, r in zip(gs, rs):
        assert (g - r).abs().max().item() < 1e-10


def test_rank_linear_scan_is_the_recurrence_from_h_in():
    """One rank's scan given h_in equals the recurrence started at h_in (fp64), its
    h_in gradient is a_0 g_0, and the ranks stitched with the folded prefix equal the
    global scan from zero (strategies/state_passing.py:29-59)."""
    g = torch.Generator().manual_seed(21)
    bsz, L, d, world = 2, 24, 5, 4
    a = (torch.rand(bsz, L, d, generator=g, dtype=torch.float64) * 0.9 + 0.05)
    b = torch.randn(bsz, L, d, generator=g, dtype=torch.float64)
    h_in = torch.randn(bsz, d, generator=g, dtype=torch.float64).requires_grad_(True)
    h = h_in
    direct = []
    for t in range(L):
        h = a[:, t] * h + b[:, t]
        direct.append(h)
    got = sp.rank_linear_scan(a, b, h_in)
    assert torch.allclose(got, torch.stack(direct, 1), atol=1e-12, rtol=1e-12)
    dh = torch.randn(bsz, L, d, generator=g, dtype=torch.float64)
    (gin,) = torch.autograd.grad(got, h_in, dh)
    adj = torch.zeros_like(b[:, 0])
    for t in reversed(range(L)):  # g_t = dh_t + a_{t+1} g_{t+1}
        adj = dh[:, t] + (a[:, t + 1] * adj if t + 1 < L else 0)
    assert torch.allclose(gin, a[:, 0] * adj, atol=1e-12, rtol=1e-12)
    pre = sp.scan_prefix(a, b, world)
    n = L // world
    stitched = torch.cat([sp.rank_linear_scan(a[:, r * n:(r + 1) * n], b[:, r * n:(r + 1) * n],
                                              pre[r]) for r in range(world)], 1)
    assert torch.allclose(stitched, sp.local_linear_scan(a, b), atol=1e-12, rtol=1e-12)
    assert torch.allclose(stitched, sp.cp_linear_scan_emulated(a, b, world), atol=1e-12)


@pytest.mark.parametrize("with_h_in", [False, True])
def test_linear_scan_grads_is_autograd_of_the_scan(with_h_in):
    """The explicit adjoint scan (values, da, db, dh_in) against torch autograd through
    the per-token recurrence of local_linear_scan / rank_linear_scan (fp64), also at L = 1."""
    g = torch.Generator().manual_seed(5)
    for bsz, L, d in ((2, 37, 6), (1, 1, 3)):
        a = (torch.rand(bsz, L, d, generator=g, dtype=torch.float64) * 1.2 - 0.1).requires_grad_(True)
        b = torch.randn(bsz, L, d, generator=g, dtype=torch.float64).requires_grad_(True)
        dh = torch.randn(bsz, L, d, generator=g, dtype=torch.float64)
        h_in = torch.randn(bsz, d, generator=g, dtype=torch.float64).requires_grad_(True)
        ref = sp.rank_linear_scan(a, b, h_in) if with_h_in else sp.local_linear_scan(a, b)
        wrt = (a, b, h_in) if with_h_in else (a, b)
        grads = torch.autograd.grad(ref, wrt, dh)
        h, da, db, dhin = sp.linear_scan_grads(a.detach(), b.detach(), dh,
                                               h_in.detach() if with_h_in else None)
        assert torch.allclose(h, ref, atol=1e-12, rtol=1e-12)
        assert torch.allclose(da, grads[0], atol=1e-12, rtol=1e-12)
        assert torch.allclose(db, grads[1], atol=1e-12, rtol=1e-12)
        if with_h_in:
            assert torch.allclose(dhin, grads[2], atol=1e-12, rtol=1e-12)


def test_effective_dt_rules():
    """The shard scan's step (mamba.py:143-148) against values fixed by the reference's
    text: the bias is added with or without softplus, negative steps clamp to the default
    dt_limit (0, inf), softplus(0) = ln 2, and a finite dt_limit clamps both ends. The CP
    wrapper's chunk decay (strategies/mamba.py:276-281) instead keeps dt as it is when
    softplus is off, bias or not."""
    t = torch.tensor
    assert sp.effective_dt(t([-1.0, 0.5])).tolist() == [0.0, 0.5]
    assert sp.effective_dt(t([-1.0]), t([3.0])).tolist() == [2.0]
    assert torch.allclose(sp.effective_dt(t([-0.5]), t([0.5]), True), t([math.log(2.0)]))
    assert torch.allclose(sp.effective_dt(t([5.0, -5.0]), None, False, (0.1, 1.0)), t([1.0, 0.1]))
    dt = t([[[-1.0]]])
    cum, decay = sp.chunk_decay(dt, t([2.0]), t([3.0]), False)
    assert cum.item() == -2.0 and torch.allclose(decay, torch.exp(t([[-2.0]])))
