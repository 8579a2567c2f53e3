"""The backward's gradient modes on the MI355X against each other (one rounding apart at most).

`rmx_attn_bwd` writes dq and dk/dv in one of four modes (include/ringmaster_amd.h,
RMX_GRAD_*): WRITE_F32 (acc := g), ACC_F32 (acc += g), ACC_FINAL (16-bit := acc + g)
and WRITE_BF16 (16-bit := g). The reverse ring accumulates its steps with ACC_F32 and a
caller finishing a ring in 16 bits uses ACC_FINAL (ring/zigzag.py:165-168,221-243 keep
the running gradients). With the same inputs the kernels compute the same fp32 g in every
mode. WRITE_BF16 is that g rounded to nearest even, exactly. The accumulating modes add g
onto the prior values; the compiler may fuse g's final scale into that add (one rounding
instead of two, which can differ from rounding g first by up to an ulp of g), so ACC_F32
is checked to one fp32 ulp of g plus one of prior + g, and ACC_FINAL to that plus one
16-bit ulp of the sum."""

import pytest
import torch

from tests.gpu_util import bf16_pair, f16_pair

pytestmark = pytest.mark.gpu


# head dims 96 and 200 leave the last 16-byte column chunks of the 128- and 256-wide kernels
# past the head dim, which the row-staged dQ epilogue must not store in any mode
@pytest.mark.parametrize("d,causal,half", [(64, True, torch.bfloat16), (128, False, torch.bfloat16),
                                           (128, True, torch.float16), (256, True, torch.bfloat16),
                                           (96, False, torch.bfloat16), (200, True, torch.bfloat16)])
def test_accumulating_gradient_modes_are_one_add(d, causal, half):
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops
    from ringmaster_amd.ring.kernels import block_forward

    b, sq, sk, hq, hkv = 2, 333, 300, 4, 2
    print(f"case grad modes d={d} causal={causal} dtype={half}", flush=True)
    pair = f16_pair if half == torch.float16 else bf16_pair
    _, q = pair((b, sq, hq, d), 31)
    _, k = pair((b, sk, hkv, d), 32)
    _, v = pair((b, sk, hkv, d), 33)
    _, do = pair((b, sq, hq, d), 34)
    sc = d ** -0.5
    mask = abi.MASK_CAUSAL if causal else abi.MASK_FULL
    out, lse, out32 = block_forward(q, k, v, sc, causal, keep_f32=True)
    delta = torch.empty((b, hq, sq), device="cuda")
    nlse = torch.empty_like(delta)
    ops.attn_bwd_delta(out32, do, delta, hkv, lse=lse, nlse=nlse)
    common = dict(q=q, k=k, v=v, dout=do, lse=lse, delta=delta, nlse=nlse)
    g = torch.Generator(device="cuda").manual_seed(35)
    prior = [torch.randn(t.shape, generator=g, device="cuda") for t in (q, k, v)]

    def run(mode, accs=None):
        dq_acc, dk_acc, dv_acc = accs if accs is not None else (None, None, None)
        half_out = [torch.empty_like(t) for t in (q, k, v)]
        ops.attn_bwd([ops.BwdJob(dq_mode=mode, dkv_mode=abi.GRAD_NONE, dq_acc=dq_acc,
                                 dq=half_out[0], **common)], scale=sc, mask=mask)
        ops.attn_bwd([ops.BwdJob(dq_mode=abi.GRAD_NONE, dkv_mode=mode, dk_acc=dk_acc,
                                 dv_acc=dv_acc, dk=half_out[1], dv=half_out[2], **common)],
                     scale=sc, mask=mask)
        torch.cuda.synchronize()
        return half_out

    grads = [torch.zeros(t.shape, device="cuda") for t in (q, k, v)]
    run(abi.GRAD_WRITE_F32, grads)
    acc = [p.clone() for p in prior]
    run(abi.GRAD_ACC_F32, acc)
    fin = run(abi.GRAD_ACC_FINAL, [p.clone() for p in prior])
    wbf = run(abi.GRAD_WRITE_BF16)
    mant = 10 if half == torch.float16 else 7  # explicit mantissa bits of the 16-bit type
    for name, gr, p, a, f, w in zip(("dq", "dk", "dv"), grads, prior, acc, fin, wbf):
        assert gr.abs().sum() > 0, name
        e = p + gr
        inf = torch.full_like(e, float("inf"))
        bar = (torch.nextafter(gr.abs(), inf) - gr.abs()) + (torch.nextafter(e.abs(), inf) - e.abs())
        err = (a - e).abs()
        i = int((err / bar).argmax())
        assert (err <= bar).all(), (f"{name}: ACC_F32 off prior + WRITE_F32 by {err.view(-1)[i]:.3e} "
                                    f"at g {gr.view(-1)[i]:.6e}, prior {p.view(-1)[i]:.6e}")
        ulp16 = torch.exp2(torch.floor(torch.log2(e.abs().clamp_min(1e-30))) - mant)
        if half == torch.float16:
            ulp16 = ulp16.clamp_min(2.0 ** -24)  # fp16 subnormal spacing below 2^-14
        assert ((f.float() - e).abs() <= ulp16 + bar).all(), f"{name}: ACC_FINAL off the sum by > 1 ulp"
        assert torch.equal(w, gr.to(half)), f"{name}: WRITE_BF16 differs from the rounded gradient"


@pytest.mark.parametrize("d", [96, 200])
def test_row_stores_stay_inside_the_head_dim(d):
    """The forward and dQ epilogues stage their rows through LDS and store 16-byte chunks of
    whole rows; at d = 96 and 200 (the 128- and 256-wide kernels) the last chunks lie past
    the head dim and are not stored. Every forward mode (WRITE, ACC_INIT, ACC_MERGE,
    ACC_FINAL) and every dQ mode writes into views of buffers padded past d with a sentinel:
    the padding keeps the sentinel, and the values equal those of contiguous outputs bit
    for bit."""
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops

    b, sq, sk, hq, hkv, pad, sentinel = 2, 333, 300, 4, 2, 40, 1024.0
    print(f"case padded rows d={d}", flush=True)
    _, q = bf16_pair((b, sq, hq, d), 41)
    _, k = bf16_pair((b, sk, hkv, d), 42)
    _, v = bf16_pair((b, sk, hkv, d), 43)
    _, do = bf16_pair((b, sq, hq, d), 44)
    sc = d ** -0.5
    mask = abi.MASK_FULL
    bufs = []

    def out_like(dtype, padded, fill=None):
        shape = (b, sq, hq, d + (pad if padded else 0))
        buf = torch.full(shape, sentinel, dtype=dtype, device="cuda")
        view = buf[..., :d]
        if fill is not None:
            view.copy_(fill)
        if padded:
            bufs.append(buf)
        return view

    def lse_like(fill=None):
        t = torch.empty((b, hq, sq), device="cuda")
        if fill is not None:
            t.copy_(fill)
        return t

    def forward_modes(padded):
        res = []
        out, acc = out_like(torch.bfloat16, padded), out_like(torch.float32, padded)
        lse = lse_like()
        ops.attn_fwd([ops.FwdJob(q=q, k=k, v=v, mode=abi.FWD_WRITE, out=out, lse=lse, acc_out=acc)],
                     scale=sc, mask=mask)
        res += [out.clone(), acc.clone(), lse.clone()]
        acc, acc_lse = out_like(torch.float32, padded), lse_like()
        ops.attn_fwd([ops.FwdJob(q=q, k=k, v=v, mode=abi.FWD_ACC_INIT, acc_out=acc, acc_lse=acc_lse)],
                     scale=sc, mask=mask)
        res += [acc.clone(), acc_lse.clone()]
        ops.attn_fwd([ops.FwdJob(q=q, k=torch.flip(k, dims=[1]), v=v, mode=abi.FWD_ACC_MERGE, acc_out=acc,
                                 acc_lse=acc_lse)], scale=sc, mask=mask)
        res += [acc.clone(), acc_lse.clone()]
        out = out_like(torch.bfloat16, padded)
        ops.attn_fwd([ops.FwdJob(q=q, k=k, v=torch.flip(v, dims=[1]), mode=abi.FWD_ACC_FINAL, out=out,
                                 acc_out=acc, acc_lse=acc_lse)], scale=sc, mask=mask)
        res += [out.clone(), acc.clone()]
        torch.cuda.synchronize()
        return res, lse

    ref, lse = forward_modes(False)
    got, _ = forward_modes(True)
    for i, (a, g) in enumerate(zip(ref, got)):
        assert torch.equal(a, g), f"forward result {i} differs with padded outputs"

    out32 = ref[1]
    delta, nlse = lse_like(), lse_like()
    ops.attn_bwd_delta(out32, do, delta, hkv, lse=lse, nlse=nlse)
    g = torch.Generator(device="cuda").manual_seed(45)
    prior = torch.randn((b, sq, hq, d), generator=g, device="cuda")

    def dq_modes(padded):
        dout = out_like(torch.bfloat16, padded, do)
        common = dict(q=q, k=k, v=v, dout=dout, lse=lse, delta=delta, nlse=nlse, dkv_mode=abi.GRAD_NONE)
        res = []
        for mode in (abi.GRAD_WRITE_F32, abi.GRAD_ACC_F32, abi.GRAD_ACC_FINAL, abi.GRAD_WRITE_BF16):
            acc = out_like(torch.float32, padded, prior) if mode != abi.GRAD_WRITE_BF16 else None
            dq = out_like(torch.bfloat16, padded)
            ops.attn_bwd([ops.BwdJob(dq_mode=mode, dq_acc=acc, dq=dq, **common)], scale=sc, mask=mask)
            torch.cuda.synchronize()
            res += [dq.clone()] + ([acc.clone()] if acc is not None else [])
        return res

    ref = dq_modes(False)
    got = dq_modes(True)
    for i, (a, g) in enumerate(zip(ref, got)):
        assert torch.equal(a, g), f"dq result {i} differs with padded outputs"
    for buf in bufs:
        assert (buf[..., d:] == sentinel).all(), "a store reached the padding past the head dim"
