"""The allocation-free Mamba2 correction backward (rmx_mamba2_cp_correction_bwd_noalloc)
against the workspace entry point (rmx_mamba2_cp_correction_bwd) on the same inputs,
both called through the C ABI. Two calls in a row, the second on a smaller shape, so the
second runs over the scratch contents the first left behind; then the configs[4] shape
(8 shards x 8192 tokens, 64 heads of 64 channels, d_state 128), whose 64 MiB workspace
is the largest the tests use. Both entry points run the same kernels, so the outputs
must agree bit for bit (dC bf16; dcumA, dh_prev fp32)."""

import pytest
import torch

from ringmaster_amd import abi
from tests.gpu_util import seeded

pytestmark = pytest.mark.gpu


def _inputs(Bsz, T, H, d, G, n, seed, seq_idx=False):
    g = torch.Generator().manual_seed(seed + 2)
    A = -torch.rand(H, generator=g)
    dt = torch.rand(Bsz, T, H, generator=g) * 0.1
    t = dict(
        gy=seeded((Bsz, T, H * d), seed).to(torch.bfloat16),
        ghf=seeded((Bsz, H, d, n), seed + 1),
        C=seeded((Bsz, T, G, n), seed + 3).to(torch.bfloat16),
        cum_A=torch.cumsum(A[None, None, :] * dt, dim=1).float(),
        h_prev=seeded((Bsz, H, d, n), seed + 4),
    )
    t = {k: v.cuda().contiguous() for k, v in t.items()}
    sid = None
    if seq_idx:
        sid = torch.zeros(Bsz, T, dtype=torch.int32)
        sid[0, T // 3:] = 1
        sid = sid.cuda()
    return t, sid


def _outputs(t):
    return (torch.empty_like(t["C"]), torch.empty_like(t["cum_A"]),
            torch.empty_like(t["h_prev"]))


_CACHE = {}


def _run(shape, seed, noalloc, seq_idx=False):
    Bsz, T, H, d, G, n = shape
    key = (shape, seed, seq_idx)
    if key not in _CACHE:
        _CACHE.clear()
        _CACHE[key] = _inputs(Bsz, T, H, d, G, n, seed, seq_idx)
    t, sid = _CACHE[key]
    gC, gA, gH = _outputs(t)
    lib = abi.lib()
    common = (t["gy"].data_ptr(), t["ghf"].data_ptr(), t["C"].data_ptr(), t["cum_A"].data_ptr(),
              t["h_prev"].data_ptr(), abi.ptr(sid), gC.data_ptr(), gA.data_ptr(), gH.data_ptr())
    stream = abi.stream_of(t["gy"])
    if noalloc:
        abi.check(lib.rmx_mamba2_cp_correction_bwd_noalloc(*common, Bsz, T, H, d, G, n, stream))
    else:
        nbytes = lib.rmx_mamba2_cp_correction_bwd_workspace(Bsz, T, H, d, G, n)
        assert nbytes > 0
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        abi.check(lib.rmx_mamba2_cp_correction_bwd(*common, ws.data_ptr(), nbytes, Bsz, T, H, d,
                                                   G, n, stream))
    torch.cuda.synchronize()
    return gC, gA, gH


def _same(got, ref, what):
    for name, a, b in zip(("dC", "dcumA", "dh_prev"), got, ref):
        assert torch.isfinite(a.float()).all(), f"{what}: {name} not finite"
        assert torch.equal(a, b), (f"{what}: {name} differs, max-abs "
                                   f"{(a.float() - b.float()).abs().max().item():.3e}")


@pytest.mark.parametrize("first,second", [
    ((4, 4500, 8, 64, 1, 128), (2, 300, 4, 128, 2, 64)),
    ((2, 2100, 8, 128, 2, 128), (1, 70, 4, 64, 1, 64)),
])
def test_noalloc_matches_workspace_entry(first, second):
    for i, shape in enumerate((first, second)):
        got = _run(shape, 40 + i, noalloc=True)
        ref = _run(shape, 40 + i, noalloc=False)
        _same(got, ref, f"call {i + 1} {shape}")


def test_noalloc_seq_idx_and_configs4_size():
    _same(_run((2, 160, 4, 64, 1, 64), 50, True, seq_idx=True),
          _run((2, 160, 4, 64, 1, 64), 50, False, seq_idx=True), "seq_idx")
    shape = (8, 8192, 64, 64, 1, 128)  # configs[4]: a 64 MiB workspace
    _same(_run(shape, 51, True), _run(shape, 51, False), "configs[4]")
    # and a smaller call after the largest one
    _same(_run((1, 33, 4, 128, 1, 128), 52, True), _run((1, 33, 4, 128, 1, 128), 52, False),
          "after configs[4]")


def test_noalloc_rejects_oversize_shape():
    lib = abi.lib()
    x = torch.zeros(16, dtype=torch.uint8, device="cuda")
    p = x.data_ptr()
    rc = lib.rmx_mamba2_cp_correction_bwd_noalloc(p, None, p, p, p, None, p, p, p, 8, 16384, 64,
                                                  64, 1, 128, abi.stream_of(x))
    assert rc == abi.RMX_EINVAL and b"scratch" in lib.rmx_last_error()
