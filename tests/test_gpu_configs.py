"""The BASELINE.json configs on the GPU.

* configs[0] (P=2 zigzag, S=4096, H=8, D=64, seeds 1-4): the emulated ring against the
  oracle ring (ring/zigzag.py:70-254) in values and gradients.
* configs[3] at reduced size (P=4, GQA 4:1, seed-5 lognormal documents scaled down)
  against the oracle ring; at full size (S=65536, Hq=32, Hkv=8) a row spot check against
  per-document causal attention in fp64.
* configs[2] at full size (P=8, S=131072, H=16, D=128): out and lse of sampled rows of
  every rank (both chunks, tile edges, the chunk boundaries) against fp64 attention on the
  CPU, and every row's out, dq, dk, dv of one head against a chunked fp32 reference on
  the GPU. Only these sizes reach the 16384-row slices, 64+ query tiles per head, the
  workgroup map over 4096+ workgroups and the causal diagonal at 16384^2.
* configs[1] at full size (one non-causal 16384^2 step, Hq=32, Hkv=8, merged into a
  running (out, lse) from a prior step): sampled rows against fp64 attention over both
  steps' keys, and one KV group's gradients against a chunked fp32 reference.

Tolerances: the north-star bar (max-abs 2e-2 and rel-L2 1e-2 against fp32; fp32 lse
1e-4 relative), checked on the fp32 values the kernels produce before the final bf16
rounding (out32, the fp32 gradient accumulators): gradients folded over a GQA group reach
|dv| ~ 8, where one bf16 half-ulp is already 1.6e-2.
"""

import math

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import assert_bf16_close, assert_f32_rel, bf16_pair

pytestmark = pytest.mark.gpu


def _zigzag_rows(world, half):
    return [rm.zigzag_gidx(r, half, world) for r in range(world)]


def _ring_vs_oracle(world, half, hq, hkv, d, cu=None, seed=0):
    """The emulated ring against the oracle ring. The bar is checked on the ring's fp32
    results (out before its bf16 rounding, lse, the fp32 gradient accumulators): with
    GQA folding |dv| reaches ~8, where the bf16 format's own half-ulp (2^-5) exceeds the
    2e-2 bar. The autograd entry point's bf16 outputs are then checked to be exactly the
    bf16 rounding of those fp32 results."""
    from ringmaster_amd.ring.zigzag import (doc_for, ring_backward, ring_forward,
                                            zigzag_ring_attention)

    S = 2 * world * half
    scale = 1.0 / math.sqrt(d)
    full = [bf16_pair((1, S, h, d), seed + i + 1)[0] for i, h in enumerate((hq, hkv, hkv, hq))]
    idx = _zigzag_rows(world, half)
    per = [[t[:, i].transpose(1, 2).contiguous() for i in idx] for t in full[:3]]
    dos = [full[3][:, i] for i in idx]
    dev = [torch.stack(p).to(torch.bfloat16).cuda() for p in per]
    dout = torch.stack(dos).to(torch.bfloat16).cuda()
    cu_dev = None if cu is None else cu.cuda()
    doc = doc_for(cu_dev, dev[0])
    out, lse, out32 = ring_forward(*dev, scale, doc)
    dq, dk, dv = ring_backward(dout, *dev, out32, lse, scale, doc)
    leaves = [t.clone().requires_grad_(True) for t in dev]
    o = zigzag_ring_attention(*leaves, cu_seqlens=cu_dev)
    o.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(o, out) and torch.equal(out, out32.to(torch.bfloat16))
    for g, leaf in zip((dq, dk, dv), leaves):
        assert torch.equal(leaf.grad, g.to(torch.bfloat16).transpose(2, 3))
    ref_out, ref_lse = rm.zigzag_ring_forward(*per, cu_seqlens=cu)
    rdq, rdk, rdv = rm.zigzag_ring_backward(dos, *per, ref_out, ref_lse, cu_seqlens=cu)
    for r in range(world):
        assert_bf16_close(out32[r], ref_out[r], f"out rank {r}")
        assert_f32_rel(lse[r], ref_lse[r], f"lse rank {r}")
        assert_bf16_close(dq[r].transpose(1, 2), rdq[r], f"dq rank {r}")
        assert_bf16_close(dk[r].transpose(1, 2), rdk[r], f"dk rank {r}")
        assert_bf16_close(dv[r].transpose(1, 2), rdv[r], f"dv rank {r}")


def test_configs0_zigzag_ring():
    """P=2, S=4096 (two 1024-token chunks per rank), H=8 MHA, D=64, seeds 1-4."""
    print("case configs[0] P=2 S=4096 H=8 D=64", flush=True)
    _ring_vs_oracle(world=2, half=1024, hq=8, hkv=8, d=64, seed=0)


def _lognormal_docs(total, median, lo, hi, seed=5):
    from bench import varlen_docs

    lens = varlen_docs(total, seed=seed, median=median, lo=lo, hi=hi)
    return torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)


def test_configs3_reduced_gqa_lognormal():
    """configs[3]'s combination at 1/8 of the length: P=4, Hq:Hkv = 4:1, D=128, documents
    drawn like configs[3] (seed 5, sigma 1) with median 256 clipped to [16, 2048]."""
    S = 8192
    cu = _lognormal_docs(S, median=256, lo=16, hi=2048)
    print(f"case configs[3] reduced: {cu.numel() - 1} documents", flush=True)
    assert cu.numel() > 8
    _ring_vs_oracle(world=4, half=S // 8, hq=8, hkv=2, d=128, cu=cu, seed=10)


# ---------------------------------------------------------------- full-size helpers
def _gen(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    return (x * scale).to(torch.bfloat16)


def _reference_head(Q, K, V, dO, scale, *, causal, chunk=4096, doc=None):
    """fp32 attention of one head (Q [S, d], K/V [Sk, d], dO [S, d]) and its gradients,
    chunked over queries on the GPU; causal is bottom-right aligned (Sk == S here)."""
    S, Sk = Q.shape[0], K.shape[0]
    out = torch.empty_like(Q)
    lse = torch.empty(S, device=Q.device)
    dQ, dK, dV = torch.zeros_like(Q), torch.zeros_like(K), torch.zeros_like(V)
    for i0 in range(0, S, chunk):
        i1 = min(i0 + chunk, S)
        kend = i1 if causal else Sk
        s = (Q[i0:i1] @ K[:kend].T) * scale
        if causal:
            qi = torch.arange(i0, i1, device=Q.device)[:, None]
            s.masked_fill_(torch.arange(kend, device=Q.device)[None, :] > qi, float("-inf"))
        ls = torch.logsumexp(s, dim=1)
        p = torch.exp(s - ls[:, None])
        del s
        o = p @ V[:kend]
        out[i0:i1], lse[i0:i1] = o, ls
        delta = (dO[i0:i1] * o).sum(1)
        dp = dO[i0:i1] @ V[:kend].T
        ds = p * (dp - delta[:, None])
        del dp
        dV[:kend] += p.T @ dO[i0:i1]
        dQ[i0:i1] = (ds @ K[:kend]) * scale
        dK[:kend] += (ds.T @ Q[i0:i1]) * scale
        del p, ds
    return out, lse, dQ, dK, dV


def test_configs2_full_size():
    """P=8, S=131072, H=16, D=128. Rows of every rank in fp64; one head whole."""
    from ringmaster_amd.ring.zigzag import ring_backward, ring_forward

    P, S, H, D = 8, 131072, 16, 128
    L, half = S // P, S // (2 * P)
    scale = 1.0 / math.sqrt(D)
    print("case configs[2] full size", flush=True)
    qg, kg, vg, dog = (_gen((1, S, H, D), s) for s in (1, 2, 3, 4))
    idx = _zigzag_rows(P, half)
    rows_dev = torch.stack(idx).cuda()
    # per-rank interface tensors [P, 1, H, L, D] (the ring's input layout)
    shard = lambda t: t[0][rows_dev].unsqueeze(1).transpose(2, 3).contiguous()  # noqa: E731
    q, k, v = shard(qg), shard(kg), shard(vg)
    dout = dog[0][rows_dev].unsqueeze(1).contiguous()                       # [P, 1, L, H, D]
    out, lse, out32 = ring_forward(q, k, v, scale)
    dq, dk, dv = ring_backward(dout, q, k, v, out32, lse, scale)
    torch.cuda.synchronize()

    # (1) sampled rows of every rank, two heads, fp64 on the CPU
    heads = [0, 11]
    kc = kg[0][:, heads].double().cpu().unsqueeze(0)
    vc = vg[0][:, heads].double().cpu().unsqueeze(0)
    local = torch.tensor([0, 1, 63, 64, 255, 256, 4095, half - 1, half, half + 1, half + 255,
                          L - 257, L - 1])
    for r in range(P):
        pos = idx[r][local]
        q_rows = qg[0][pos.cuda()][:, heads].double().cpu().unsqueeze(0)
        ro, rl = rm.attention_rows(q_rows, kc, vc, pos, scaling=scale, causal=True)
        assert_bf16_close(out[r][0][local.cuda()][:, heads], ro[0], f"out rows rank {r}")
        assert_f32_rel(lse[r][0][heads][:, local.cuda()], rl[0], f"lse rows rank {r}")

    # (2) one head, every row: out and the gradients against chunked fp32 on the GPU
    h = 5
    Q, K, V, dO = (t[0, :, h].float() for t in (qg, kg, vg, dog))
    ro, rl, rdq, rdk, rdv = _reference_head(Q, K, V, dO, scale, causal=True)
    flat = rows_dev.reshape(-1)
    got_out = torch.empty(S, D, device="cuda")
    got_out[flat] = out[:, 0, :, h].reshape(-1, D).float()
    got_lse = torch.empty(S, device="cuda")
    got_lse[flat] = lse[:, 0, h].reshape(-1)
    got_out[flat] = out32[:, 0, :, h].reshape(-1, D)     # the fp32 out before its rounding
    grads = []
    for g in (dq, dk, dv):
        t = torch.empty(S, D, device="cuda")
        t[flat] = g[:, 0, :, h].reshape(-1, D)
        grads.append(t)
    torch.cuda.synchronize()
    assert_bf16_close(got_out, ro, "out head 5")
    assert_f32_rel(got_lse, rl, "lse head 5")
    for name, got, ref in zip(("dq", "dk", "dv"), grads, (rdq, rdk, rdv)):
        assert_bf16_close(got, ref, f"{name} head 5")


def test_configs1_full_size():
    """one non-causal step, Hq=32, Hkv=8, 16384^2, D=128, q/k/v ~ N(0,1)/sqrt(D),
    merged (ACC_FINAL) into the running (out, lse) of a prior step over other keys (seeds
    6, 7); the backward of both steps with the merged lse."""
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops

    S, Hq, Hkv, D = 16384, 32, 8, 128
    sc = 1.0 / math.sqrt(D)
    print("case configs[1] full size", flush=True)
    q, k, v = _gen((1, S, Hq, D), 1, sc), _gen((1, S, Hkv, D), 2, sc), _gen((1, S, Hkv, D), 3, sc)
    kp, vp = _gen((1, S, Hkv, D), 6, sc), _gen((1, S, Hkv, D), 7, sc)
    dout = _gen((1, S, Hq, D), 4)
    acc = torch.empty((1, S, Hq, D), device="cuda")
    acc_lse = torch.empty((1, Hq, S), device="cuda")
    out = torch.empty((1, S, Hq, D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((1, Hq, S), device="cuda")
    ops.attn_fwd([ops.FwdJob(q=q, k=kp, v=vp, mode=abi.FWD_ACC_INIT, acc_out=acc,
                             acc_lse=acc_lse)], scale=sc, mask=abi.MASK_FULL)
    ops.attn_fwd([ops.FwdJob(q=q, k=k, v=v, mode=abi.FWD_ACC_FINAL, out=out, lse=lse,
                             acc_out=acc, acc_lse=acc_lse)], scale=sc, mask=abi.MASK_FULL)
    delta, nlse = torch.empty_like(lse), torch.empty_like(lse)
    ops.attn_bwd_delta(acc, dout, delta, Hkv, lse=lse, nlse=nlse)
    dq = torch.empty((1, S, Hq, D), device="cuda")
    dks = [torch.empty((1, S, Hkv, D), device="cuda") for _ in range(4)]
    for i, (kk, vv) in enumerate(((kp, vp), (k, v))):
        ops.attn_bwd([ops.BwdJob(q=q, k=kk, v=vv, dout=dout, lse=lse, delta=delta, nlse=nlse,
                                 dq_mode=abi.GRAD_WRITE_F32 if i == 0 else abi.GRAD_ACC_F32,
                                 dkv_mode=abi.GRAD_WRITE_F32, dq_acc=dq, dk_acc=dks[2 * i],
                                 dv_acc=dks[2 * i + 1])], scale=sc, mask=abi.MASK_FULL)
    torch.cuda.synchronize()

    # rows in fp64 against attention over both steps' keys
    heads = [0, 3, 4, 31]                       # kv heads 0, 0, 1, 7
    kv_of = [h // (Hq // Hkv) for h in heads]
    kall = torch.cat([kp, k], 1)[0][:, kv_of].double().cpu().unsqueeze(0)
    vall = torch.cat([vp, v], 1)[0][:, kv_of].double().cpu().unsqueeze(0)
    rows = torch.tensor([0, 1, 255, 256, 8191, 8192, 16383])
    q_rows = q[0][rows.cuda()][:, heads].double().cpu().unsqueeze(0)
    ro, rl = rm.attention_rows(q_rows, kall, vall, rows, scaling=sc, causal=False)
    assert_bf16_close(out[0][rows.cuda()][:, heads], ro[0], "out rows")
    assert_f32_rel(lse[0][heads][:, rows.cuda()], rl[0], "lse rows")

    # kv group 1 (q heads 4..7): gradients against chunked fp32 over both steps' keys
    g = 1
    K = torch.cat([kp, k], 1)[0, :, g].float()
    V = torch.cat([vp, v], 1)[0, :, g].float()
    dK = torch.zeros(2 * S, D, device="cuda")
    dV = torch.zeros(2 * S, D, device="cuda")
    for h in range(4 * g, 4 * g + 4):
        ro, rl, rdq, rdk, rdv = _reference_head(q[0, :, h].float(), K, V, dout[0, :, h].float(),
                                                sc, causal=False)
        assert_bf16_close(dq[0, :, h], rdq, f"dq head {h}")
        dK += rdk
        dV += rdv
    for i, name in enumerate(("prior", "step")):
        sl = slice(i * S, (i + 1) * S)
        assert_bf16_close(dks[2 * i][0, :, g], dK[sl], f"dk {name}")
        assert_bf16_close(dks[2 * i + 1][0, :, g], dV[sl], f"dv {name}")


def test_configs3_full_size_rows():
    """configs[3] at full size (P=4, S=65536, Hq=32, Hkv=8, seed-5 lognormal documents):
    sampled rows of every rank against per-document causal attention in fp64."""
    from ringmaster_amd.ring.zigzag import doc_ids_from_cu, ring_forward

    P, S, Hq, Hkv, D = 4, 65536, 32, 8, 128
    L, half = S // P, S // (2 * P)
    scale = 1.0 / math.sqrt(D)
    cu = _lognormal_docs(S, median=2048, lo=128, hi=16384)
    print(f"case configs[3] full size: {cu.numel() - 1} documents", flush=True)
    qg, kg, vg = _gen((1, S, Hq, D), 1), _gen((1, S, Hkv, D), 2), _gen((1, S, Hkv, D), 3)
    idx = _zigzag_rows(P, half)
    rows_dev = torch.stack(idx).cuda()
    shard = lambda t: t[0][rows_dev].unsqueeze(1).transpose(2, 3).contiguous()  # noqa: E731
    doc = doc_ids_from_cu(cu.cuda(), "cuda", S)
    out, lse, _ = ring_forward(shard(qg), shard(kg), shard(vg), scale, doc)
    torch.cuda.synchronize()
    heads = [2, 29]
    kv_of = [h // (Hq // Hkv) for h in heads]
    kc = kg[0][:, kv_of].double().cpu()
    vc = vg[0][:, kv_of].double().cpu()
    starts = cu[:-1].tolist()
    local = torch.tensor([0, 1, 255, 256, half - 1, half, half + 1, L - 1, 1000, 12345])
    for r in range(P):
        pos = idx[r][local]
        qr = qg[0][pos.cuda()][:, heads].double().cpu()                  # [n, 2, D]
        ref_o = torch.empty(len(pos), len(heads), D, dtype=torch.float64)
        ref_l = torch.empty(len(heads), len(pos), dtype=torch.float64)
        for i, p in enumerate(pos.tolist()):
            s0 = max(st for st in starts if st <= p)                       # the row's document
            sc_ = torch.einsum("hd,khd->hk", qr[i], kc[s0:p + 1]) * scale
            ref_l[:, i] = torch.logsumexp(sc_, dim=1)
            ref_o[i] = torch.einsum("hk,khd->hd", torch.softmax(sc_, dim=1), vc[s0:p + 1])
        assert_bf16_close(out[r][0][local.cuda()][:, heads], ref_o, f"out rows rank {r}")
        assert_f32_rel(lse[r][0][heads][:, local.cuda()], ref_l, f"lse rows rank {r}")


def test_configs3_full_size_group():
    """configs[3] at full size (P=4, S=65536, Hq=32, Hkv=8, the 25 seed-5 lognormal
    documents), forward and reverse-ring backward: every row of KV group 5 (q heads 20-23)
    against per-document causal attention in fp32 on the GPU (ring/zigzag.py:86-120,170-209,
    ring/varlen_blocks.py:176-200): out and dq of the four heads, and the GQA-folded dk, dv."""
    from ringmaster_amd.ring.zigzag import doc_ids_from_cu, ring_backward, ring_forward

    P, S, Hq, Hkv, D = 4, 65536, 32, 8, 128
    L, half, G = S // P, S // (2 * P), Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    cu = _lognormal_docs(S, median=2048, lo=128, hi=16384)
    print(f"case configs[3] full size fwd+bwd: {cu.numel() - 1} documents", flush=True)
    qg, kg, vg = _gen((1, S, Hq, D), 1), _gen((1, S, Hkv, D), 2), _gen((1, S, Hkv, D), 3)
    dog = _gen((1, S, Hq, D), 4)
    idx = _zigzag_rows(P, half)
    rows_dev = torch.stack(idx).cuda()
    shard = lambda t: t[0][rows_dev].unsqueeze(1).transpose(2, 3).contiguous()  # noqa: E731
    q, k, v = shard(qg), shard(kg), shard(vg)
    dout = dog[0][rows_dev].unsqueeze(1).contiguous()                       # [P, 1, L, Hq, D]
    doc = doc_ids_from_cu(cu.cuda(), "cuda", S)
    out, lse, out32 = ring_forward(q, k, v, scale, doc)
    dq, dk, dv = ring_backward(dout, q, k, v, out32, lse, scale, doc)
    torch.cuda.synchronize()
    del q, k, v, dout

    flat = rows_dev.reshape(-1)

    def unshard(t, h):
        full = torch.empty(S, D, device="cuda")
        full[flat] = t[:, 0, :, h].reshape(-1, D).float()
        return full

    g = 5
    K, V = kg[0, :, g].float(), vg[0, :, g].float()
    rdK, rdV = torch.zeros(S, D, device="cuda"), torch.zeros(S, D, device="cuda")
    bounds = cu.tolist()
    for h in range(G * g, G * g + G):
        Q, dO = qg[0, :, h].float(), dog[0, :, h].float()
        ro, rdq = torch.empty(S, D, device="cuda"), torch.empty(S, D, device="cuda")
        for a, b in zip(bounds[:-1], bounds[1:]):
            o, _, dqd, dkd, dvd = _reference_head(Q[a:b], K[a:b], V[a:b], dO[a:b], scale,
                                                  causal=True)
            ro[a:b], rdq[a:b] = o, dqd
            rdK[a:b] += dkd
            rdV[a:b] += dvd
        assert_bf16_close(unshard(out32, h), ro, f"out head {h}")
        assert_bf16_close(unshard(dq, h), rdq, f"dq head {h}")
    assert_bf16_close(unshard(dk, g), rdK, f"dk kv head {g}")
    assert_bf16_close(unshard(dv, g), rdV, f"dv kv head {g}")
