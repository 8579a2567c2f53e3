"""The C-ABI library loads without a GPU, exports every symbol include/*.h declares, and
rejects bad arguments on the host (before any launch) with the reference's exception
classes."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from ringmaster_amd import abi

HEADER = Path(__file__).resolve().parents[1] / "include" / "ringmaster_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(rmx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"missing export {name}"
    assert set(names) == set(abi.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_error_string():
    lib = abi.lib()
    assert lib.rmx_abi_version() == abi.ABI_VERSION == 18
    assert isinstance(lib.rmx_last_error(), bytes)


def _layout(**kw):
    lay = abi.AttnLayout()
    lay.batch, lay.hq, lay.hkv, lay.head_dim = 1, 4, 2, 128
    lay.scale, lay.mask = 0.125, abi.MASK_FULL
    for k, v in kw.items():
        setattr(lay, k, v)
    return lay


def _fwd(lay, n=0):
    arr = (abi.FwdProblem * max(n, 1))()
    return abi.lib().rmx_attn_fwd(ctypes.byref(lay), arr, n, None)


def test_host_validation_gqa_divisibility():
    rc = _fwd(_layout(hq=3, hkv=2))
    assert rc == abi.RMX_EINVAL
    with pytest.raises(ValueError, match="divisible"):
        abi.check(rc)


def test_host_validation_head_dim_and_mask():
    assert _fwd(_layout(head_dim=264)) == abi.RMX_EUNSUPPORTED  # above 256
    assert _fwd(_layout(head_dim=136)) == abi.RMX_OK            # zero problems: no launch
    assert _fwd(_layout(head_dim=256)) == abi.RMX_OK
    assert _fwd(_layout(head_dim=100)) == abi.RMX_EUNSUPPORTED  # not a multiple of 8
    assert _fwd(_layout(head_dim=96)) == abi.RMX_OK             # zero problems: no launch
    with pytest.raises(NotImplementedError):
        abi.check(abi.RMX_EUNSUPPORTED)
    assert _fwd(_layout(mask=7)) == abi.RMX_EINVAL
    assert _fwd(_layout(scale=float("nan"))) == abi.RMX_EINVAL
    assert _fwd(_layout(q_ss=12)) == abi.RMX_EINVAL  # not a multiple of 8 elements


def test_host_validation_problem_fields():
    lay = _layout()
    arr = (abi.FwdProblem * 1)()
    arr[0].sq, arr[0].sk, arr[0].mode = 4, 4, abi.FWD_WRITE
    assert abi.lib().rmx_attn_fwd(ctypes.byref(lay), arr, 1, None) == abi.RMX_EINVAL  # q NULL
    assert b"NULL" in abi.lib().rmx_last_error()
    arr[0].q = arr[0].k = arr[0].v = arr[0].out = 16
    arr[0].mode = 9
    assert abi.lib().rmx_attn_fwd(ctypes.byref(lay), arr, 1, None) == abi.RMX_EINVAL
    assert b"mode" in abi.lib().rmx_last_error()


def test_host_validation_dtype_and_merge_type():
    assert _fwd(_layout(dtype=2)) == abi.RMX_EINVAL
    assert b"element type" in abi.lib().rmx_last_error()
    assert _fwd(_layout(dtype=abi.DTYPE_F16)) == abi.RMX_OK  # no problems: no launch
    st = abi.i64_array((0, 0, 0))
    assert abi.lib().rmx_lse_merge(16, 16, 16, 3, 16, 1, 1, 1, 8, st, st, st, st, 1, None) \
        == abi.RMX_EINVAL
    assert b"block type" in abi.lib().rmx_last_error()


def test_host_validation_dropout():
    assert _fwd(_layout(dropout_p=1.0)) == abi.RMX_EINVAL
    assert _fwd(_layout(dropout_p=-0.1)) == abi.RMX_EINVAL
    assert b"dropout_p" in abi.lib().rmx_last_error()
    assert _fwd(_layout(dropout_p=0.1, mask=abi.MASK_DOC)) == abi.RMX_OK  # no problems: no launch
    assert _fwd(_layout(dropout_p=0.1, drop_seed_lo=5, drop_seed_hi=7)) == abi.RMX_OK


def test_host_validation_window_flag():
    lay = _layout()
    arr = (abi.FwdProblem * 1)()
    arr[0].has_window, arr[0].window_left = 2, 10
    assert abi.lib().rmx_attn_fwd(ctypes.byref(lay), arr, 1, None) == abi.RMX_EINVAL
    assert b"has_window" in abi.lib().rmx_last_error()
    barr = (abi.BwdProblem * 1)()
    barr[0].has_window = -1
    assert abi.lib().rmx_attn_bwd(ctypes.byref(lay), barr, 1, None) == abi.RMX_EINVAL


def test_host_validation_window_right():
    """window_right (the shift of the causal diagonal) lies in [0, 2^28] and needs the
    causal mask kind; the checks run before any pointer is read."""
    lib = abi.lib()
    for mask, right, rc in ((abi.MASK_CAUSAL, -1, abi.RMX_EINVAL),
                            (abi.MASK_CAUSAL, (1 << 28) + 1, abi.RMX_EINVAL),
                            (abi.MASK_FULL, 5, abi.RMX_EINVAL),
                            (abi.MASK_DOC, 5, abi.RMX_EINVAL),
                            (abi.MASK_CAUSAL, 1 << 28, abi.RMX_OK),
                            (abi.MASK_CAUSAL, 0, abi.RMX_OK)):
        lay = _layout(mask=mask, m_sb=0)
        arr = (abi.FwdProblem * 1)()
        arr[0].window_right = right  # sq = sk = 0: validated, nothing launched
        assert lib.rmx_attn_fwd(ctypes.byref(lay), arr, 1, None) == rc, (mask, right)
        if rc:
            assert b"window_right" in lib.rmx_last_error()
        barr = (abi.BwdProblem * 1)()
        barr[0].window_right = right
        assert lib.rmx_attn_bwd(ctypes.byref(lay), barr, 1, None) == rc, (mask, right)


def test_problem_structs_match_the_header():
    """The ctypes mirrors have the C layout: the window and dropout fields sit at the end
    of each problem struct (a zero-filled problem has no window and no offsets)."""
    assert ctypes.sizeof(abi.FwdProblem) == 11 * 8 + 8 * 4
    assert ctypes.sizeof(abi.BwdProblem) == 17 * 8 + 9 * 4 + 4
    assert abi.FwdProblem.has_window.offset == 11 * 8 + 3 * 4
    assert abi.BwdProblem.has_window.offset == 17 * 8 + 4 * 4
    assert abi.FwdProblem.drop_k0.offset == 11 * 8 + 6 * 4
    assert abi.FwdProblem.window_right.offset == 11 * 8 + 7 * 4
    assert abi.BwdProblem.window_right.offset == 17 * 8 + 8 * 4
    assert abi.AttnLayout.q_sb.offset == 40  # after the dtype, dropout and seed words
    assert abi.AttnLayout.m_sb.offset == 40 + 23 * 8  # after the 23 tensor strides
    assert ctypes.sizeof(abi.AttnLayout) == 40 + 24 * 8


def test_host_validation_metadata_stride():
    assert _fwd(_layout(mask=abi.MASK_DOC, m_sb=-1)) == abi.RMX_EINVAL
    assert b"m_sb" in abi.lib().rmx_last_error()
    assert _fwd(_layout(mask=abi.MASK_DOC, m_sb=4096)) == abi.RMX_OK


def test_host_validation_backward_nlse():
    lay = _layout()
    arr = (abi.BwdProblem * 1)()
    p = arr[0]
    p.q = p.k = p.v = p.dout = p.lse = p.delta = 16
    p.dk_acc = p.dv_acc = 256
    p.sq, p.sk = 4, 4
    p.dq_mode, p.dkv_mode = abi.GRAD_NONE, abi.GRAD_WRITE_F32
    lib = abi.lib()
    assert lib.rmx_attn_bwd(ctypes.byref(lay), arr, 1, None) == abi.RMX_EINVAL
    assert b"nlse" in lib.rmx_last_error()
    # the delta pass writes nlse only from a given lse
    assert lib.rmx_attn_bwd_delta(ctypes.byref(lay), 16, 0, 16, 16, None, 16, 4, None) == abi.RMX_EINVAL
    assert b"lse" in lib.rmx_last_error()


def test_empty_calls_are_noops():
    assert _fwd(_layout(), 0) == abi.RMX_OK
    lib = abi.lib()
    assert lib.rmx_zigzag_gather(None, None, 0, 0, 2, -1, 16, 0, None, None) == abi.RMX_OK
    assert lib.rmx_linear_scan_fwd(None, None, None, None, None, 0, 8, 4, 4, 2, None, 0, None) \
        == abi.RMX_OK


def test_host_validation_shard_and_scan():
    lib = abi.lib()
    assert lib.rmx_zigzag_gather(16, 16, 1, 8, 0, -1, 16, 128, None, None) == abi.RMX_EINVAL
    assert lib.rmx_zigzag_gather(16, 16, 1, 8, 2, 2, 16, 128, None, None) == abi.RMX_EINVAL
    fwd = lambda *a: lib.rmx_linear_scan_fwd(*a, None, 0, None)  # noqa: E731
    assert fwd(16, 16, None, 16, None, 1, 9, 4, 4, 2) == abi.RMX_EINVAL
    assert fwd(16, 16, None, 16, None, 1, 8, 6, 4, 2) == abi.RMX_EINVAL
    assert fwd(16, 16, 8, 16, None, 1, 8, 4, 4, 2) == abi.RMX_EINVAL
    assert b"aligned" in lib.rmx_last_error()  # h_in not 16-byte aligned
    assert lib.rmx_linear_scan_bwd(16, 16, None, 16, 16, 16, 16, 1, 8, 4, 4, 1, None, 0, None) \
        == abi.RMX_EINVAL  # dh_in without h_in
    assert b"h_in" in lib.rmx_last_error()


def test_scan_workspace_plan_and_checks():
    """The L-parallel scan's workspace query and the checks of its entry points."""
    lib = abi.lib()
    tc = ctypes.c_int32(0)
    need = lib.rmx_linear_scan_workspace(1, 65536, 256, 8, ctypes.byref(tc))
    # 256 channels: one 64-lane x 4-channel token group per wave, 8 waves x 16 tokens
    assert tc.value == 128
    slots = 65536 // 128
    assert need >= 256 + slots * 4 + slots * 256 * 12
    assert lib.rmx_linear_scan_workspace(1, 0, 256, 8, None) == 0
    assert lib.rmx_linear_scan_workspace(1, 4096, 3, 2, None) == 0  # groups must divide d
    # d = 1: one channel per token group, 64 token groups per wave
    lib.rmx_linear_scan_workspace(2, 65536, 1, 1, ctypes.byref(tc))
    assert tc.value == 8 * 64 * 16
    # a workspace below the plan's size is refused before any launch
    assert lib.rmx_linear_scan_fwd(16, 16, None, 16, None, 1, 65536, 256, 8, 1, 16, need - 1,
                                   None) == abi.RMX_EINVAL
    assert b"workspace" in lib.rmx_last_error()
    assert lib.rmx_linear_scan_bwd(16, 16, None, 16, 16, 16, None, 1, 65536, 256, 8, 1, 16,
                                   need - 1, None) == abi.RMX_EINVAL
    # chunk states need shards aligned to the chunks
    assert lib.rmx_linear_scan_fwd(16, 16, None, 16, 16, 1, 65536 - 64 * 8 + 8 * 8, 256, 8, 8, 16,
                                   need, None) == abi.RMX_EINVAL
    assert b"chunk" in lib.rmx_last_error()


def test_scan_algo_selection():
    from ringmaster_amd.strategies import state_passing as sp

    ws = sp._workspace("auto", 1, 65536, 256, 8, 1, False, "cpu")
    assert ws is not None and ws.dtype.itemsize == 1          # long L, few channels: chunked
    assert sp._workspace("auto", 1, 256, 524288, 64, 8, True, "cpu") is None  # configs[4]
    assert sp._workspace("per_channel", 1, 65536, 256, 8, 1, False, "cpu") is None
    assert sp._workspace("auto", 1, 65536 - 8, 256, 8, 8, True, "cpu") is None
    with pytest.raises(ValueError, match="chunk"):
        sp._workspace("chunked", 1, 65536 - 8, 256, 8, 8, True, "cpu")
    with pytest.raises(ValueError, match="algo"):
        sp._workspace("serial", 1, 65536, 256, 8, 1, False, "cpu")


def test_product_refuses_cpu_tensors():
    import torch

    from ringmaster_amd.ring.kernels import mi355x_hip_block
    from ringmaster_amd.ring.zigzag import zigzag_ring_attention

    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        mi355x_hip_block(q, q, q, causal=True, scaling=None)
    with pytest.raises(RuntimeError, match="ROCm device"):
        zigzag_ring_attention(q[None].transpose(2, 3), q[None].transpose(2, 3),
                              q[None].transpose(2, 3))


def test_host_validation_chunk_state():
    lib = abi.lib()
    p = 16  # any 16-byte aligned non-null value: validation fails before a launch
    # head_dim / d_state outside {64, 128}, heads not a multiple of groups, bad rows
    assert lib.rmx_mamba2_chunk_state(p, p, p, p, None, p, 1, 8, 4, 32, 1, 64, None) \
        == abi.RMX_EUNSUPPORTED
    assert lib.rmx_mamba2_chunk_state(p, p, p, p, None, p, 1, 8, 4, 64, 1, 96, None) \
        == abi.RMX_EUNSUPPORTED
    assert lib.rmx_mamba2_chunk_state(p, p, p, p, None, p, 1, 8, 6, 64, 4, 64, None) \
        == abi.RMX_EINVAL
    assert lib.rmx_mamba2_chunk_state(p, p, p, p, None, p, -1, 8, 4, 64, 1, 64, None) \
        == abi.RMX_EINVAL
    assert lib.rmx_mamba2_chunk_state(8, p, p, p, None, p, 1, 8, 4, 64, 1, 64, None) \
        == abi.RMX_EINVAL  # x not 16-byte aligned
    assert lib.rmx_mamba2_chunk_state_bwd(p, p, p, p, None, None, p, p, p, p, 1, 8, 4, 64, 1, 64,
                                          None, 0, None) == abi.RMX_EINVAL  # no g_state
    # the two-head form's workspace: bf16 G, where its LDS fits (head_dim 64)
    assert lib.rmx_mamba2_chunk_state_bwd_workspace(8, 64, 64, 128) == 8 * 64 * 64 * 128 * 2
    assert lib.rmx_mamba2_chunk_state_bwd_workspace(8, 64, 128, 128) == 0
    assert lib.rmx_mamba2_chunk_state_bwd_workspace(8, 64, 32, 128) == 0
    assert lib.rmx_mamba2_chunk_state_bwd(p, p, p, p, None, p, p, p, p, p, 1, 8, 4, 64, 1, 64,
                                          p, 100, None) == abi.RMX_EINVAL  # workspace too small
    assert b"workspace" in lib.rmx_last_error()
    # empty problems are no-ops
    assert lib.rmx_mamba2_chunk_state(None, None, None, None, None, None, 0, 8, 4, 64, 1, 64,
                                      None) == abi.RMX_OK
    assert lib.rmx_mamba2_chunk_state_bwd(None, None, None, None, None, None, None, None, None,
                                          None, 2, 0, 4, 64, 1, 64, None, 0, None) == abi.RMX_OK


def test_host_validation_correction_bwd_noalloc():
    """The allocation-free correction backward checks its arguments, and rejects shapes
    whose workspace exceeds its fixed scratch array, before touching the device."""
    lib = abi.lib()
    p = 16  # any 16-byte aligned non-null value: validation fails before a launch
    need = lib.rmx_mamba2_cp_correction_bwd_workspace(8, 16384, 64, 64, 1, 128)
    assert need > (96 << 20)
    assert lib.rmx_mamba2_cp_correction_bwd_noalloc(p, None, p, p, p, None, p, p, p, 8, 16384, 64,
                                                    64, 1, 128, None) == abi.RMX_EINVAL
    assert b"scratch" in lib.rmx_last_error()
    # configs[4] (8 shards x 8192 tokens, 64 heads of 64, d_state 128) fits the array
    assert lib.rmx_mamba2_cp_correction_bwd_workspace(8, 8192, 64, 64, 1, 128) <= (96 << 20)
    assert lib.rmx_mamba2_cp_correction_bwd_noalloc(p, None, None, p, p, None, p, p, p, 2, 64, 4,
                                                    64, 1, 64, None) == abi.RMX_EINVAL  # C NULL
    assert b"NULL" in lib.rmx_last_error()
    assert lib.rmx_mamba2_cp_correction_bwd_noalloc(p, None, p, p, p, None, p, p, p, 2, 64, 4, 64,
                                                    1, 32, None) == abi.RMX_EUNSUPPORTED
    assert lib.rmx_mamba2_cp_correction_bwd_noalloc(None, None, None, None, None, None, None, None,
                                                    None, 0, 64, 4, 64, 1, 64, None) == abi.RMX_OK


def test_mamba_entry_points_refuse_cpu_tensors():
    import torch

    from ringmaster_amd.strategies.mamba import (causal_conv1d_cp, mamba2_chunk_decay,
                                                 mamba2_chunk_state)

    x = torch.zeros(1, 64, 2, 64, dtype=torch.bfloat16)
    dt = torch.zeros(1, 64, 2)
    A = torch.zeros(2)
    B = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        mamba2_chunk_state(x, dt, A, B)
    with pytest.raises(RuntimeError, match="ROCm device"):
        mamba2_chunk_decay(dt, A, torch.zeros(2), dt_softplus=True)
    with pytest.raises(RuntimeError, match="ROCm device"):
        causal_conv1d_cp(torch.zeros(1, 1, 8, 16, dtype=torch.bfloat16),
                         torch.zeros(8, 4, dtype=torch.bfloat16))


def test_cp_linear_scan_group_argument():
    """cp_linear_scan(a, b, group) takes the reference's process group as its third
    argument; an integer there (a world size) is refused with a pointer to world=."""
    import torch

    from ringmaster_amd.strategies.state_passing import cp_linear_scan

    a = torch.ones(1, 4, 2)
    with pytest.raises(TypeError, match="world="):
        cp_linear_scan(a, a, 2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        cp_linear_scan(a, a, None)
    with pytest.raises(ValueError, match="world=1"):
        cp_linear_scan(a, a, world=2, h_in=torch.zeros(1, 2))


def test_cp_state_prefix_arguments():
    """cp_state_prefix(ssm_state, chunk_decay, group, *, single_hop) as in the reference
    (strategies/mamba.py:68): an integer group is refused, the tensors must live on the
    GPU, and the gathered form checks the rank against the gathered ranks."""
    import torch

    from ringmaster_amd.strategies.mamba import cp_state_prefix, cp_state_prefix_gathered

    st, dc = torch.zeros(1, 2, 4, 8), torch.ones(1, 2)
    with pytest.raises(TypeError, match="cp_state_prefix_all"):
        cp_state_prefix(st, dc, 2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        cp_state_prefix(st, dc, None, single_hop=True)
    with pytest.raises(ValueError, match="rank"):
        cp_state_prefix_gathered(st[None].expand(3, -1, -1, -1, -1), dc[None].expand(3, -1, -1), 3)


def test_zigzag_ring_attention_group_keyword():
    """zigzag_ring_attention accepts the reference's ``group`` keyword (ring/zigzag.py:257);
    the emulated ring takes its ranks on the leading axis, so only None is valid."""
    import torch

    from ringmaster_amd.ring.zigzag import zigzag_ring_attention

    q = torch.zeros(2, 1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="leading axis"):
        zigzag_ring_attention(q, q, q, group=object())
    with pytest.raises(RuntimeError, match="ROCm device"):
        zigzag_ring_attention(q, q, q, group=None)


def test_linear_scan_status_host_checks():
    """No workspace: nothing to report; a workspace smaller than its header is refused
    before any device access."""
    lib = abi.lib()
    assert lib.rmx_linear_scan_status(None, 0, None) == abi.RMX_OK
    assert lib.rmx_linear_scan_status(16, 8, None) == abi.RMX_EINVAL
    assert b"too small" in lib.rmx_last_error()


def _band(sq, sk, causal, left, right):
    """The kept (q, k) pairs of a block under a causal flag and bounds (None: unbounded)
    on pos_q - pos_k and pos_k - pos_q, bottom-right aligned positions."""
    iq = torch.arange(sq)[:, None] + (sk - sq)
    ik = torch.arange(sk)[None, :]
    keep = torch.ones(sq, sk, dtype=torch.bool)
    if causal:
        keep &= ik <= iq
    if left is not None:
        keep &= iq - ik <= left
    if right is not None:
        keep &= ik - iq <= right
    return keep


def test_window_bounds_keep_the_flash_pairs():
    """The provider's window resolution (host logic that picks the kernels' mask kind and
    bounds) keeps exactly the pairs of the oracle's flash-attention window rules, over a
    grid of block shapes and windows; the gather ring's form (no sk) agrees wherever
    sq <= sk."""
    from oracle import ring_math as rm
    from ringmaster_amd.ring.kernels import _mask_of, window_bounds

    for sq, sk in ((5, 5), (3, 8), (8, 3), (9, 4), (1, 6), (6, 1), (7, 6)):
        for causal in (False, True):
            for w in ((-1, -1), (0, 0), (2, -1), (-1, 2), (1, 3), (3, 1), (sk, 0), (0, sk),
                      (sk + 2, sk + 2), (-5, 4), (7, -3)):
                left, right = window_bounds(w, causal, sk)
                mask, shift = _mask_of(causal, right)
                # the causal mask kind keeps k <= q + (sk - sq) + shift
                got = _band(sq, sk, False, left, shift if mask == abi.MASK_CAUSAL else None)
                ref = _band(sq, sk, causal, *rm.flash_window(w, causal, sk))
                assert torch.equal(got, ref), (sq, sk, causal, w)
                if sq <= sk:
                    left2, right2 = window_bounds(w, causal)
                    mask2, shift2 = _mask_of(causal, right2)
                    got2 = _band(sq, sk, False, left2, shift2 if mask2 == abi.MASK_CAUSAL else None)
                    assert torch.equal(got2, ref), (sq, sk, causal, w)
