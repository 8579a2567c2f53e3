"""Mamba2 CP causal conv1d on the MI355X (rmx_causal_conv1d_cp and its backward) vs the
CPU restatement of the reference's halo algorithm (oracle/conv.py) and autograd
through it: bf16 outputs / dx within the bf16 bounds, fp32 dweight / dbias within 1e-4."""

import pytest
import torch

from oracle import conv as oc
from tests.gpu_util import assert_bf16_close, assert_f32_rel, bf16_pair

pytestmark = pytest.mark.gpu


def _run(world, B, C, L, W, act, with_bias, cu=None, seed=0, elementwise=False):
    """``elementwise``: check y and dx per element to one bf16 rounding of
    max(|ref|, 1) instead of the absolute bf16 bound (long rows reach |y| > 8, where
    one rounding exceeds it)."""
    from ringmaster_amd.strategies.mamba import causal_conv1d_cp

    print(f"case world={world} B={B} C={C} L={L} W={W} act={act} bias={with_bias} docs={cu}",
          flush=True)
    xf, xd = bf16_pair((world, B, C, L), seed + 1)
    wf, wd = bf16_pair((C, W), seed + 2, scale=0.5)
    bf_, bd = bf16_pair((C,), seed + 3) if with_bias else (None, None)
    gf, gd = bf16_pair((world, B, C, L), seed + 4)
    xd, wd = xd.requires_grad_(True), wd.requires_grad_(True)
    if bd is not None:
        bd.requires_grad_(True)
    y = causal_conv1d_cp(xd, wd, bd, act, cu_seqlens=None if cu is None else cu.cuda())
    y.backward(gd)
    torch.cuda.synchronize()
    xr = xf.double().requires_grad_(True)
    wr = wf.double().requires_grad_(True)
    br = None if bf_ is None else bf_.double().requires_grad_(True)
    ref = torch.stack(oc.cp_conv(list(xr.unbind(0)), wr, br, act, cu_seqlens=cu))
    ref.backward(gf.double())
    if elementwise:
        assert_f32_rel(y.float(), ref, "y", tol=2.0 ** -8)
        assert_f32_rel(xd.grad.float(), xr.grad, "dx", tol=2.0 ** -8)
    else:
        assert_bf16_close(y, ref, "y")
        assert_bf16_close(xd.grad, xr.grad, "dx")
    # the kernel's fp32 dweight / dbias (the C ABI output) against the fp64 reference;
    # autograd hands back those sums rounded to the parameters' bf16 (the sums are
    # fp32 atomics, so two runs may differ in the last fp32 bits: compare at bf16
    # resolution, one rounding = 2^-9 relative)
    dw32, db32 = _raw_bwd(xd.detach(), wd.detach(), None if bd is None else bd.detach(), gd,
                          act, cu)
    assert_f32_rel(dw32, wr.grad, "dweight")
    assert_f32_rel(wd.grad.float(), dw32, "autograd dweight", tol=2.0 ** -8)
    if br is not None:
        assert_f32_rel(db32, br.grad, "dbias")
        assert_f32_rel(bd.grad.float(), db32, "autograd dbias", tol=2.0 ** -8)
    return y


def _raw_bwd(x, w, b, dy, act, cu):
    from ringmaster_amd import abi
    from ringmaster_amd.ring.zigzag import doc_ids_from_cu

    P, B, C, L = x.shape
    doc = None
    if cu is not None:
        doc = doc_ids_from_cu(cu.cuda(), x.device)
        doc = (doc.reshape(B, P * L) if doc.numel() == B * P * L
               else doc.reshape(1, P * L).expand(B, P * L)).contiguous()
    dx = torch.empty_like(x)
    dw = torch.zeros(w.shape, dtype=torch.float32, device=x.device)
    db = torch.zeros(C, dtype=torch.float32, device=x.device) if b is not None else None
    abi.check(abi.lib().rmx_causal_conv1d_cp_bwd(
        x.data_ptr(), w.data_ptr(), abi.ptr(b), abi.ptr(doc), dy.data_ptr(), dx.data_ptr(),
        dw.data_ptr(), abi.ptr(db), P, B, C, L, w.shape[1], 1 if act else 0, abi.stream_of(x)))
    torch.cuda.synchronize()
    return dw, db


@pytest.mark.parametrize("world", [1, 2, 4])
@pytest.mark.parametrize("W,act,with_bias", [(4, "silu", True), (2, None, False), (4, None, True)])
def test_conv_dense(world, W, act, with_bias):
    _run(world, 2, 48, 64, W, act, with_bias)


def test_conv_wide_and_unit_width():
    _run(3, 1, 8, 16, 9, "silu", True)
    _run(2, 1, 8, 16, 1, None, True)


@pytest.mark.parametrize("docs", [[30, 2, 1, 95], [128], [7, 64, 57]])
def test_conv_packed(docs):
    cu = torch.tensor([0, *torch.tensor(docs).cumsum(0).tolist()], dtype=torch.int32)
    _run(4, 1, 32, 32, 4, "silu", True, cu=cu)


def test_conv_packed_batch_rows():
    # two packed rows flattened into one cu_seqlens, as the reference's runtime passes them
    cu = torch.tensor([0, 20, 64, 100, 101, 128], dtype=torch.int32)
    _run(2, 2, 16, 32, 4, "silu", True, cu=cu)


def test_conv_medium_size():
    _run(8, 1, 256, 1024, 4, "silu", True, seed=7)


def test_conv_rows_over_several_workgroups():
    # 257 runs of 8 tokens per row: the row's last run is lane 0 of a second workgroup,
    # whose neighbour chunks cross a workgroup (neighbour loads, not lane shuffles)
    _run(2, 1, 16, 2056, 4, "silu", True, seed=9, elementwise=True)
    _run(3, 1, 8, 4120, 9, None, False, seed=10, elementwise=True)


def test_conv_host_validation():
    from ringmaster_amd.strategies.mamba import causal_conv1d_cp

    x = torch.zeros(2, 1, 8, 12, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 4, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError):  # local length not a multiple of 8
        causal_conv1d_cp(x, w)
    with pytest.raises(ValueError):
        causal_conv1d_cp(x[..., :2], w)  # shard shorter than the halo
