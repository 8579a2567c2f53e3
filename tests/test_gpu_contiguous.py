"""Emulated contiguous rings on the MI355X (p2p / allgather ``ring_attention``,
``ring_p2p_attention``, DistFlash, packed ``varlen_ring_attention``) vs the CPU oracle
rings (fp32), values and gradients."""

import math

import pytest
import torch

from oracle import ring_math as rm
from tests.gpu_util import BF16_MAX_ABS, BF16_REL_L2, assert_bf16_close, bf16_pair, rel_l2

pytestmark = pytest.mark.gpu


def _inputs(world, L, hq, hkv, d=128, seed=0):
    S = world * L
    full = [bf16_pair((1, S, h, d), seed + i)[0] for i, h in enumerate((hq, hkv, hkv, hq), 1)]
    idx = [rm.contiguous_gidx(r, L) for r in range(world)]
    per = [[t[:, i].transpose(1, 2).contiguous() for i in idx] for t in full[:3]]
    dev = [torch.stack(p).to(torch.bfloat16).cuda().requires_grad_(True) for p in per]
    dos = [full[3][:, i] for i in idx]
    dod = torch.stack(dos).to(torch.bfloat16).cuda()
    return per, dev, dos, dod


def _check(fn, ref_fwd, ref_bwd, world, L, hq=2, hkv=2, cu=None, seed=0):
    per, (qd, kd, vd), dos, dod = _inputs(world, L, hq, hkv, seed=seed)
    print(f"case world={world} L={L} hq={hq} hkv={hkv} docs={cu}", flush=True)
    out = fn(qd, kd, vd)
    out.backward(dod)
    torch.cuda.synchronize()
    ref_out, ref_lse = ref_fwd(*per, cu_seqlens=cu)
    rdq, rdk, rdv = ref_bwd(dos, *per, ref_out, ref_lse, cu_seqlens=cu)
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        assert_bf16_close(qd.grad[r], rdq[r], f"dq rank {r}")
        assert_bf16_close(kd.grad[r], rdk[r], f"dk rank {r}")
        assert_bf16_close(vd.grad[r], rdv[r], f"dv rank {r}")


def _contig(causal):
    return (lambda *a, **kw: rm.contiguous_ring_forward(*a, causal=causal, **kw),
            lambda *a, **kw: rm.contiguous_ring_backward(*a, causal=causal, **kw))


@pytest.mark.parametrize("world", [1, 2, 4, 8])
@pytest.mark.parametrize("causal", [True, False])
def test_p2p_ring(world, causal):
    from ringmaster_amd.ring import ring_p2p_attention

    _check(lambda q, k, v: ring_p2p_attention(q, k, v, causal=causal, scaling=None),
           *_contig(causal), world, 128)


@pytest.mark.parametrize("method", ["allgather", "alltoall"])
def test_ring_attention_methods_gqa_ragged(method):
    from ringmaster_amd.ring import ring_attention

    _check(lambda q, k, v: ring_attention(q, k, v, causal=True, rotate_method=method,
                                          attn_implementation="math"),
           *_contig(True), 4, 100, hq=4, hkv=2)


def test_ring_attention_single_rank_is_one_block():
    from ringmaster_amd.ring import ring_attention

    _check(lambda q, k, v: ring_attention(q, k, v, causal=True), *_contig(True), 1, 192)


@pytest.mark.parametrize("world", [2, 4, 8])
def test_distflash(world):
    from ringmaster_amd.ring import distflash_attention

    # MHA: with GQA the first rank's dV sums two heads over every rank and reaches |dV| ~ 4,
    # where one bf16 rounding of the output (half an ulp, 2^-7 * 4) nearly fills the 2e-2
    # bound by itself; the GQA fold is covered by the ring_attention and varlen cases
    _check(lambda q, k, v: distflash_attention(q, k, v, scaling=None),
           rm.distflash_forward, rm.distflash_backward, world, 96, hq=2, hkv=2)


@pytest.mark.parametrize("docs", [[300, 212], [100, 50, 250, 112]])
def test_distflash_varlen(docs):
    from ringmaster_amd.ring import distflash_attention

    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()], dtype=torch.int32)
    world = 4
    _check(lambda q, k, v: distflash_attention(q, k, v, scaling=None, cu_seqlens=cu.cuda()),
           rm.distflash_forward, rm.distflash_backward, world, 128, hq=2, hkv=1, cu=cu)


def test_varlen_ring_attention():
    from ringmaster_amd.ring import varlen_ring_attention

    cu = torch.tensor([0, 37, 200, 201, 390, 512], dtype=torch.int32)
    _check(lambda q, k, v: varlen_ring_attention(q, k, v, scaling=None, cu_seqlens=cu.cuda()),
           *_contig(True), 4, 128, cu=cu)


def test_p2p_preconditions():
    from ringmaster_amd.ring import ring_attention

    q = torch.zeros(2, 1, 2, 64, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="P2P Ring requires"):
        ring_attention(q, q, q, causal=True, dropout=0.1)
    with pytest.raises(ValueError, match="P2P Ring requires"):
        ring_attention(q, q, q, causal=True, attn_implementation="sdpa")
    with pytest.raises(ValueError, match="P2P Ring requires"):
        ring_attention(q, q, q, causal=True, window=(4, 0))
    with pytest.raises(ValueError, match="dropout"):
        ring_attention(q, q, q, causal=True, rotate_method="allgather", dropout=1.0)
    from ringmaster_amd.ring import varlen_ring_attention

    cu = torch.tensor([0, 64, 128], dtype=torch.int32, device="cuda")
    with pytest.raises(NotImplementedError, match="non-causal"):
        varlen_ring_attention(q, q, q, scaling=None, cu_seqlens=cu, causal=False, window=(8, 0))
    with pytest.raises(ValueError, match="cu_seqlens"):  # a host cu_seqlens must cover b S
        varlen_ring_attention(torch.zeros(2, 2, 2, 64, 128, dtype=torch.bfloat16, device="cuda"),
                              *[torch.zeros(2, 2, 2, 64, 128, dtype=torch.bfloat16,
                                            device="cuda")] * 2,
                              scaling=None, cu_seqlens=torch.tensor([0, 64, 128]))


# per-row documents of the packed ring (ring/loop.py:178): row 0 packs 7 documents, row 1 three,
# over b S = 2 * 4 * 128 tokens; a document boundary at the row boundary
_ROW_CU = [0, 37, 200, 201, 390, 420, 480, 512, 700, 703, 1024]


def _row_inputs(world, L, b, hq, hkv, d=128, seed=40):
    per = []
    for i, h in enumerate((hq, hkv, hkv)):
        per.append([bf16_pair((b, h, L, d), seed + 10 * i + r)[0] for r in range(world)])
    dev = [torch.stack(ts).to(torch.bfloat16).cuda().requires_grad_(True) for ts in per]
    dos = [bf16_pair((b, L, hq, d), seed + 50 + r)[0] for r in range(world)]
    return per, dev, dos, torch.stack(dos).to(torch.bfloat16).cuda()


def _check_rows(world, L, b, hq, hkv, cu, causal, dropout=0.0, gseed=0):
    from ringmaster_amd.ring import varlen_ring_attention
    from ringmaster_amd.ring.kernels import new_dropout_seed

    per, (qd, kd, vd), dos, dod = _row_inputs(world, L, b, hq, hkv)
    print(f"case varlen rows world={world} L={L} b={b} causal={causal} dropout={dropout}",
          flush=True)
    torch.manual_seed(gseed)
    out = varlen_ring_attention(qd, kd, vd, scaling=None, cu_seqlens=cu.cuda(), causal=causal,
                                dropout=dropout)
    out.backward(dod)
    torch.cuda.synchronize()
    torch.manual_seed(gseed)
    seed = new_dropout_seed() if dropout else None
    refs = [[t.clone().requires_grad_(True) for t in ts] for ts in per]
    ref_out, _ = rm.varlen_ring_forward(*refs, cu, causal=causal, dropout=dropout, drop_seed=seed)
    sum((o * g).sum() for o, g in zip(ref_out, dos)).backward()
    extra = _delta_rounding_bound(per, dos, cu, causal, dropout, seed) if dropout else None
    # GQA-folded dK / dV (and kept probabilities scaled by 1 / (1 - p) with dropout) reach
    # values where one bf16 ulp of the output alone exceeds 2e-2: per-element ulp bars there
    for r in range(world):
        assert_bf16_close(out[r], ref_out[r], f"out rank {r}")
        if extra is None:
            assert_bf16_close(qd.grad[r], refs[0][r].grad, f"dq rank {r}")
            assert_bf16_close(kd.grad[r], refs[1][r].grad, f"dk rank {r}", ulp_floor=True)
        else:
            for what, got, ref, ex in (("dq", qd.grad[r], refs[0][r].grad, extra[0][r]),
                                       ("dk", kd.grad[r], refs[1][r].grad, extra[1][r])):
                # the element bar (2e-2, or one bf16 ulp of the value) plus the delta term
                got = got.float().cpu()
                bar = torch.clamp(ref.abs() * 2.0 ** -7, min=BF16_MAX_ABS) + ex
                over = ((got - ref).abs() / bar).max().item()
                assert over < 1 and rel_l2(got, ref) < BF16_REL_L2, \
                    f"{what} rank {r}: {over:.2f} of the bar, rel-L2 {rel_l2(got, ref):.2e}"
        assert_bf16_close(vd.grad[r], refs[2][r].grad, f"dv rank {r}", ulp_floor=True)


def _delta_rounding_bound(per, dos, cu, causal, p, seed):
    """Per element of dq [b, Hq, L, d] and of dk [b, Hkv, L, d], per rank: the part of its
    error that the forward's 16-bit P leaves in delta. The forward multiplies V by P m
    rounded to bf16 (relative error at most 2^-8, m the dropout keep scale), delta =
    rowsum(dO * O) inherits that rounding, and the backward's dS = P (m dP - delta)
    recomputes P in fp32, so dS_qk moves by P_qk d_q with |d_q| <= 2^-8 sum_j P_qj m_qj
    |dP_qj|: |d dq_q| <= scale |d_q| |sum_k P_qk K_k| and |d dk_k| <= scale sum_q P_qk |d_q|
    |Q_q| (summed over the q heads of the kv head). Each row's dS sums to zero exactly
    (m sum P dP - delta = 0 when nothing is dropped), so on rows of one or two keys (the
    first tokens of a document) this term is all there is: e.g. a row of two keys with
    |m dP| = 41 misses 0.025 of a dq of 1.77 after a 0.4% rounding of delta."""
    world, b, hq, L, d = len(per[0]), *per[0][0].shape
    hkv = per[1][0].shape[1]
    S = world * L
    doc = rm.doc_ids_from_cu(cu).reshape(b, S)
    kf = torch.cat([t for t in per[1]], 2).double().repeat_interleave(hq // hkv, 1)  # [b,hq,S,d]
    vf = torch.cat([t for t in per[2]], 2).double().repeat_interleave(hq // hkv, 1)
    scale = 1.0 / math.sqrt(d)
    kidx = torch.arange(S)
    dq_b, dk_b = [], torch.zeros(b, hq, S, d, dtype=torch.float64)
    for r in range(world):
        qidx = torch.arange(r * L, r * L + L)
        allow = doc[:, qidx, None] == doc[:, None, :]
        if causal:
            allow &= (kidx[None, :] <= qidx[:, None])[None]
        q = per[0][r].double()
        s = (q @ kf.transpose(-1, -2)) * scale
        s = s.masked_fill(~allow[:, None], float("-inf"))
        pr = torch.softmax(s, -1)
        m = rm.dropout_scale_mask(seed, b, hq, L, S, p, q0=r * L).double()
        dp = dos[r].double().transpose(1, 2) @ vf.transpose(-1, -2)
        dlt = 2.0 ** -8 * (pr * m * dp.abs()).sum(-1, keepdim=True)  # [b, hq, L, 1]
        dq_b.append((scale * dlt * (pr @ kf).abs()).float())
        dk_b += scale * (pr * dlt).transpose(-1, -2) @ q.abs()
    dk_b = dk_b.unflatten(1, (hkv, hq // hkv)).sum(2).float()
    return dq_b, [dk_b[:, :, r * L:(r + 1) * L] for r in range(world)]
