"""The Mamba2 shard final state on the GPU (rmx_mamba2_chunk_state and its backward,
mamba2_chunk_state): the final_states of each shard's zero-state scan that the
reference's CP wrapper gathers (mamba.py:113-141,160-172), against the oracle
closed form (pinned to the SSD recurrence on the CPU) and autograd through it."""

import pytest
import torch

from oracle import state_passing as sp
from tests.gpu_util import BF16_REL_L2, rel_l2, seeded

pytestmark = pytest.mark.gpu

# (rows, T, H, D, G, N): ragged T, both state and head sizes, one or two groups, the
# two-workgroup split (T >= 1024 with few rows), a single token
# the forward runs two heads per workgroup when a group has an even number of heads
# (D * N <= 64 * 128), one otherwise: (6 heads, 2 groups) takes the one-head path
CASES = [(2, 200, 8, 64, 2, 128), (1, 2048, 4, 64, 1, 64), (2, 130, 4, 128, 2, 64),
         (1, 300, 2, 128, 1, 128), (1, 1, 2, 64, 1, 64), (1, 333, 6, 64, 2, 128)]


def _weights(R, T, H, seed):
    """Effective dt e (softplus of a bias-shifted dt) and cum_A = cumsum(A e), fp32."""
    dt = seeded((R, T, H), seed) - 1.0
    bias = seeded((H,), seed + 1) * 0.5
    A = -0.02 * torch.exp(seeded((H,), seed + 2) * 0.3)
    e = torch.nn.functional.softplus(dt + bias)
    cum = torch.cumsum(A.double()[None, None, :] * e.double(), dim=1).float()
    return e, cum


def _t0_of(R, T, docs):
    """Row 0 starts its last document at docs[0]; the other rows hold one document."""
    return torch.tensor([docs[0] if docs and r == 0 else 0 for r in range(R)], dtype=torch.int32)


def _raw_forward(x, B, e, cum, t0):
    from ringmaster_amd import abi

    R, T, H, D = x.shape
    G, N = B.shape[2:]
    state = torch.full((R, H, D, N), float("nan"), dtype=torch.float32, device="cuda")
    abi.check(abi.lib().rmx_mamba2_chunk_state(
        x.data_ptr(), B.data_ptr(), e.data_ptr(), cum.data_ptr(), abi.ptr(t0), state.data_ptr(),
        R, T, H, D, G, N, abi.stream_of(x)))
    return state


def _kernel_rounding_ref(x, B, e, cum, t0):
    """The closed form with the weighted x rounded to bf16 as the kernel does, summed
    in fp64."""
    R, T, H, _ = x.shape
    G = B.shape[2]
    w = e * torch.exp(cum[:, -1:, :] - cum)
    keep = torch.arange(T)[None, :] >= t0[:, None]
    w = torch.where(keep[:, :, None], w, torch.zeros_like(w))
    xs = (x.float() * w[..., None]).to(torch.bfloat16).double()
    Bx = B.double().repeat_interleave(H // G, dim=2)
    return torch.einsum("bthd,bthn->bhdn", xs, Bx)


@pytest.mark.parametrize("docs", [None, (7,)])
@pytest.mark.parametrize("R,T,H,D,G,N", CASES)
def test_chunk_state_forward(R, T, H, D, G, N, docs):
    print(f"case fwd R={R} T={T} H={H} D={D} G={G} N={N} docs={docs}", flush=True)
    if docs and T <= docs[0]:
        pytest.skip("document start past the shard")
    x = seeded((R, T, H, D), 1).to(torch.bfloat16)
    B = seeded((R, T, G, N), 2).to(torch.bfloat16)
    e, cum = _weights(R, T, H, 3)
    t0 = _t0_of(R, T, docs)
    dev = [t.cuda() for t in (x, B, e, cum)] + [t0.cuda() if docs else None]
    got = _raw_forward(*dev)
    torch.cuda.synchronize()
    got = got.cpu().double()
    assert torch.isfinite(got).all()
    emu = _kernel_rounding_ref(x, B, e, cum, t0)
    exact = sp.chunk_state(x.double(), B.double(), e.double(), cum.double(), t0)
    assert rel_l2(got, emu) < 2e-4, rel_l2(got, emu)
    assert rel_l2(got, exact) < BF16_REL_L2, rel_l2(got, exact)


# backward extras: groups of 12 heads (32-byte g_e / g_cum_A rows at aligned head
# offsets, then a partial group), 10 heads (the second group starts unaligned), and
# the configs[4] layout (64 heads in one group) on a shorter shard
# groups of 12 and 10 heads: 8-head strips ending part-way; (1, 300, 3, 64, 1, 128): an
# odd head count (the second head slot idles in the last step, no 8-head tables)
# (2, 512, 64, ...) and (1, 384, 32, ...): 8 and 2 groups of 8 heads per C group, so
# both backward forms start their workgroups at rotated head groups; (1, 600, 16, 128,
# ...): the same in the one-head form at head_dim 128 (three token blocks)
BWD_CASES = CASES[:4] + [(1, 256, 24, 64, 2, 128), (1, 160, 20, 64, 2, 64),
                         (2, 512, 64, 64, 1, 128), (1, 300, 3, 64, 1, 128),
                         (1, 384, 32, 64, 2, 128), (1, 600, 16, 128, 1, 64)]


@pytest.mark.parametrize("two_heads", [True, False])
@pytest.mark.parametrize("docs", [None, (100,)])
@pytest.mark.parametrize("R,T,H,D,G,N", BWD_CASES)
def test_chunk_state_backward_raw(R, T, H, D, G, N, docs, two_heads):
    """Both forms of the backward: with the bf16 workspace (two heads per step, G by LDS
    DMA; where D * N <= 64 * 128) and without it (one head per step)."""
    from ringmaster_amd import abi

    print(f"case bwd R={R} T={T} H={H} D={D} G={G} N={N} docs={docs} two_heads={two_heads}",
          flush=True)
    x = seeded((R, T, H, D), 11).to(torch.bfloat16)
    B = seeded((R, T, G, N), 12).to(torch.bfloat16)
    e, cum = _weights(R, T, H, 13)
    t0 = _t0_of(R, T, docs)
    gs = seeded((R, H, D, N), 14)
    leaves = [t.double().requires_grad_(True) for t in (x.float(), B.float(), e, cum)]
    S = sp.chunk_state(*leaves, t0)
    (S * gs.double()).sum().backward()

    # every device buffer stays referenced until the kernel has run
    xd, Bd, ed, cd, gsd = x.cuda(), B.cuda(), e.cuda(), cum.cuda(), gs.cuda()
    t0d = t0.cuda() if docs else None
    g_x, g_B = torch.empty_like(xd), torch.empty_like(Bd)
    g_e = torch.empty_like(ed)
    g_cum = torch.empty_like(ed)
    lib = abi.lib()
    ws_bytes = lib.rmx_mamba2_chunk_state_bwd_workspace(R, H, D, N) if two_heads else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if ws_bytes else None
    abi.check(lib.rmx_mamba2_chunk_state_bwd(
        xd.data_ptr(), Bd.data_ptr(), ed.data_ptr(), cd.data_ptr(), abi.ptr(t0d),
        gsd.data_ptr(), g_x.data_ptr(), g_B.data_ptr(), g_e.data_ptr(), g_cum.data_ptr(),
        R, T, H, D, G, N, abi.ptr(ws), ws_bytes, abi.stream_of(xd)))
    g_cum[:, T - 1] = -g_cum[:, :T - 1].sum(1)
    torch.cuda.synchronize()
    for name, got, ref in zip(("g_x", "g_B", "g_e", "g_cum_A"), (g_x, g_B, g_e, g_cum),
                              (leaf.grad for leaf in leaves)):
        got = got.cpu().double()
        assert torch.isfinite(got).all(), name
        assert rel_l2(got, ref) < BF16_REL_L2, (name, rel_l2(got, ref))
    if docs:  # tokens before the last document carry no gradient
        assert g_x[0, :docs[0]].abs().max().item() == 0.0
        assert g_e[0, :docs[0]].abs().max().item() == 0.0


@pytest.mark.parametrize("softplus,dt_f32,with_bias,limit", [
    (True, False, True, None), (False, True, False, None),
    (False, True, True, None),          # bias without softplus: added, then clamped at 0
    (True, True, True, (0.05, 0.8)),    # a dt_limit that clamps both ends
])
@pytest.mark.parametrize("packed", [False, True])
def test_chunk_state_chain_values_and_grads(softplus, dt_f32, with_bias, limit, packed):
    """mamba2_chunk_state from raw dt (dt kernel with its effective-dt output + state)
    against the oracle chain (effective_dt of mamba.py:143-148, cumsum, chunk_state) in
    fp64: values and gradients w.r.t. x, B, dt, A and dt_bias."""
    from ringmaster_amd.strategies.mamba import mamba2_chunk_state

    print(f"case chain softplus={softplus} dt_f32={dt_f32} bias={with_bias} limit={limit} "
          f"packed={packed}", flush=True)
    P, Bsz, T, H, D, G, N = 2, 2, 384, 8, 64, 2, 128
    x = seeded((P, Bsz, T, H, D), 21).to(torch.bfloat16)
    B = seeded((P, Bsz, T, G, N), 22).to(torch.bfloat16)
    raw = seeded((P, Bsz, T, H), 23) - 1.0
    if not softplus and not with_bias:
        raw = torch.nn.functional.softplus(raw)  # positive steps
    dt = raw.to(torch.float32 if dt_f32 else torch.bfloat16)
    lim = limit or (0.0, float("inf"))
    A = -0.02 * torch.exp(seeded((H,), 24) * 0.3)
    bias = seeded((H,), 25) * 0.5
    seq = None
    if packed:
        seq = torch.zeros(P, Bsz, T, dtype=torch.int32)
        seq[0, 0, 150:] = 1
        seq[1, 1, 40:] = 1
        seq[1, 1, 300:] = 2
    gs = seeded((P, Bsz, H, D, N), 26)

    xr, Br, dtr, Ar, br = (t.double().requires_grad_(True)
                           for t in (x.float(), B.float(), dt.float(), A, bias))
    rows = P * Bsz
    e_r = sp.effective_dt(dtr, br if with_bias else None, softplus, lim)
    cum_r = torch.cumsum(Ar[None, None, :] * e_r.reshape(rows, T, H), dim=1)
    t0 = None
    if packed:
        s = seq.reshape(rows, T)
        t0 = torch.tensor([max([t + 1 for t in range(T) if s[r, t] != s[r, -1]], default=0)
                           for r in range(rows)])
    S_r = sp.chunk_state(xr.reshape(rows, T, H, D), Br.reshape(rows, T, G, N),
                         e_r.reshape(rows, T, H), cum_r, t0).reshape(P, Bsz, H, D, N)
    (S_r * gs.double()).sum().backward()

    xd, Bd, dtd, Ad, bd = (t.cuda().requires_grad_(True) for t in (x, B, dt, A, bias))
    S = mamba2_chunk_state(xd, dtd, Ad, Bd, dt_bias=bd if with_bias else None,
                           dt_softplus=softplus, dt_limit=lim,
                           seq_idx=seq.cuda() if packed else None)
    S.backward(gs.cuda())
    torch.cuda.synchronize()
    assert rel_l2(S.detach().cpu(), S_r) < BF16_REL_L2
    checks = [("x", xd, xr), ("B", Bd, Br), ("dt", dtd, dtr), ("A", Ad, Ar)]
    if with_bias:
        checks.append(("dt_bias", bd, br))
    for name, got, ref in checks:
        assert got.grad is not None, name
        err = rel_l2(got.grad.cpu(), ref.grad)
        assert err < 2e-2, (name, err)


def test_host_tensors_next_to_device_ones_are_refused():
    """A dt_bias or seq_idx left on the host raises instead of reaching a kernel."""
    from ringmaster_amd.strategies.mamba import mamba2_chunk_state

    x = torch.zeros(1, 64, 2, 64, dtype=torch.bfloat16, device="cuda")
    dt = torch.zeros(1, 64, 2, device="cuda")
    A = torch.zeros(2, device="cuda")
    B = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="ROCm device"):
        mamba2_chunk_state(x, dt, A, B, dt_bias=torch.zeros(2), dt_softplus=True)
    with pytest.raises(RuntimeError, match="ROCm device"):
        mamba2_chunk_state(x, dt, A, B, seq_idx=torch.zeros(1, 64, dtype=torch.int32))


def test_host_bias_next_to_device_tensors_is_refused():
    """Device x / weight / dt / A with a host bias or dt_bias: the check of that one
    tensor raises (the others alone would pass it)."""
    from ringmaster_amd.strategies.mamba import causal_conv1d_cp, mamba2_chunk_decay

    x = torch.zeros(1, 1, 8, 16, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 4, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="ROCm device"):
        causal_conv1d_cp(x, w, torch.zeros(8, dtype=torch.bfloat16))
    dt = torch.zeros(1, 64, 2, device="cuda")
    A = torch.zeros(2, device="cuda")
    with pytest.raises(RuntimeError, match="ROCm device"):
        mamba2_chunk_decay(dt, A, torch.zeros(2), dt_softplus=True)
    causal_conv1d_cp(x, w, torch.zeros(8, dtype=torch.bfloat16, device="cuda"))  # all on device
    mamba2_chunk_decay(dt, A, torch.zeros(2, device="cuda"), dt_softplus=True)
