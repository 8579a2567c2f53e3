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


@pytest.mark.parametrize("d,causal,half", [(64, True, torch.bfloat16), (128, False, torch.bfloat16),
                                           (128, True, torch.float16), (256, True, torch.bfloat16)])
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
