"""ctypes binding of the C ABI in ``include/ringmaster_amd.h``.

The shared library is loaded lazily, after ``torch`` (so that it binds to the HIP
runtime torch already loaded: both carry the SONAME ``libamdhip64.so.7``), and is
never replaced by a Python fallback: if it is missing, or a tensor is not on a
ROCm device, calls raise. Error codes map to the exceptions the reference raises
for the same conditions (``ValueError`` for bad arguments, e.g. GQA divisibility
``ring/kernels.py:57-58``; ``RuntimeError`` for device failures).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libringmaster_amd.so"
ABI_VERSION = 18  # RMX_ABI_VERSION of include/ringmaster_amd.h

RMX_OK = 0
RMX_EINVAL = -1
RMX_EUNSUPPORTED = -2
RMX_EDEVICE = -3

DTYPE_BF16 = 0
DTYPE_F16 = 1

MASK_FULL = 0
MASK_CAUSAL = 1
MASK_DOC = 2

FWD_WRITE = 0
FWD_ACC_INIT = 1
FWD_ACC_MERGE = 2
FWD_ACC_FINAL = 3

GRAD_WRITE_BF16 = 0
GRAD_WRITE_F32 = 1
GRAD_ACC_F32 = 2
GRAD_ACC_FINAL = 3
GRAD_NONE = 4

MAX_BATCHED = 16

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class AttnLayout(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("hq", _i32), ("hkv", _i32), ("head_dim", _i32),
        ("scale", ctypes.c_float), ("mask", _i32), ("dtype", _i32),
        ("dropout_p", ctypes.c_float), ("drop_seed_lo", ctypes.c_uint32),
        ("drop_seed_hi", ctypes.c_uint32),
        ("q_sb", _i64), ("q_ss", _i64), ("q_sh", _i64),
        ("k_sb", _i64), ("k_ss", _i64), ("k_sh", _i64),
        ("v_sb", _i64), ("v_ss", _i64), ("v_sh", _i64),
        ("o_sb", _i64), ("o_ss", _i64), ("o_sh", _i64),
        ("a_sb", _i64), ("a_ss", _i64), ("a_sh", _i64),
        ("l_sb", _i64), ("l_sh", _i64),
        ("dk_sb", _i64), ("dk_ss", _i64), ("dk_sh", _i64),
        ("ka_sb", _i64), ("ka_ss", _i64), ("ka_sh", _i64),
        ("m_sb", _i64),
    ]


class FwdProblem(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("lse", _vp),
        ("acc_out", _vp), ("acc_lse", _vp),
        ("q_gidx", _vp), ("k_gidx", _vp), ("q_doc", _vp), ("k_doc", _vp),
        ("sq", _i32), ("sk", _i32), ("mode", _i32), ("has_window", _i32), ("window_left", _i32),
        ("drop_q0", _i32), ("drop_k0", _i32), ("window_right", _i32),
    ]


class BwdProblem(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("dout", _vp), ("lse", _vp), ("delta", _vp),
        ("nlse", _vp), ("dq_acc", _vp), ("dq", _vp), ("dk_acc", _vp), ("dv_acc", _vp), ("dk", _vp), ("dv", _vp),
        ("q_gidx", _vp), ("k_gidx", _vp), ("q_doc", _vp), ("k_doc", _vp),
        ("sq", _i32), ("sk", _i32), ("dq_mode", _i32), ("dkv_mode", _i32),
        ("has_window", _i32), ("window_left", _i32), ("drop_q0", _i32), ("drop_k0", _i32),
        ("window_right", _i32),
    ]


# name -> (restype, argtypes); every symbol declared in include/ringmaster_amd.h
SIGNATURES = {
    "rmx_abi_version": (_i32, []),
    "rmx_last_error": (ctypes.c_char_p, []),
    "rmx_attn_fwd": (_i32, [ctypes.POINTER(AttnLayout), ctypes.POINTER(FwdProblem), _i32, _vp]),
    "rmx_attn_bwd_delta": (_i32, [ctypes.POINTER(AttnLayout), _vp, _i32, _vp, _vp, _vp, _vp, _i32,
                                  _vp]),
    "rmx_attn_bwd": (_i32, [ctypes.POINTER(AttnLayout), ctypes.POINTER(BwdProblem), _i32, _vp]),
    "rmx_lse_merge": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32,
                             ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                             ctypes.POINTER(_i64), _i32, _vp]),
    "rmx_zigzag_gather": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i64, _i64, _vp, _vp]),
    "rmx_zigzag_scatter": (_i32, [_vp, _vp, _i32, _i32, _i32, _i64, _i64, _vp]),
    "rmx_linear_scan_fwd": (_i32, [_vp] * 5 + [_i32] * 5 + [_vp, ctypes.c_size_t, _vp]),
    "rmx_linear_scan_workspace": (ctypes.c_size_t, [_i32] * 4 + [ctypes.POINTER(_i32)]),
    "rmx_linear_scan_status": (_i32, [_vp, ctypes.c_size_t, _vp]),
    "rmx_linear_scan_bwd": (_i32, [_vp] * 7 + [_i32] * 5 + [_vp, ctypes.c_size_t, _vp]),
    "rmx_mamba2_cp_correction": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                                        _i32, _i32, _i32, _vp]),
    "rmx_mamba2_cp_correction_bwd_workspace": (ctypes.c_size_t, [_i32] * 6),
    "rmx_mamba2_cp_correction_bwd": (_i32, [_vp] * 10 + [ctypes.c_size_t] + [_i32] * 6 + [_vp]),
    "rmx_mamba2_cp_correction_bwd_noalloc": (_i32, [_vp] * 9 + [_i32] * 6 + [_vp]),
    "rmx_mamba2_dt_cumsum": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32,
                                    _vp]),
    "rmx_mamba2_dt_cumsum_bwd": (_i32, [_vp, _i32, _vp, _vp, _i32] + [_vp] * 7
                                 + [_i32, _i32, _i32, _vp]),
    "rmx_mamba2_chunk_state": (_i32, [_vp] * 6 + [_i32] * 6 + [_vp]),
    "rmx_mamba2_chunk_state_bwd_workspace": (ctypes.c_size_t, [_i32] * 4),
    "rmx_mamba2_chunk_state_bwd": (_i32, [_vp] * 10 + [_i32] * 6 + [_vp, ctypes.c_size_t, _vp]),
    "rmx_causal_conv1d_cp": (_i32, [_vp] * 5 + [_i32] * 6 + [_vp]),
    "rmx_causal_conv1d_cp_bwd": (_i32, [_vp] * 8 + [_i32] * 6 + [_vp]),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded C-ABI library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"ringmaster_amd native library missing ({LIB_PATH}); build it with "
                        "`python -c 'import __graft_entry__ as g; g.build()'`")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                if handle.rmx_abi_version() != ABI_VERSION:
                    raise RuntimeError("ringmaster_amd ABI version mismatch")
                _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc == RMX_OK:
        return
    msg = (lib().rmx_last_error() or b"").decode(errors="replace")
    if rc == RMX_EINVAL:
        raise ValueError(msg)
    if rc == RMX_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def require_device(*tensors: torch.Tensor | None) -> None:
    """The HIP kernels run only on ROCm device tensors; there is no CPU path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "ringmaster_amd runs its kernels on the MI355X only: tensors must be on a ROCm "
                f"device (got {t.device})")


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64_array(vals) -> ctypes.Array:
    arr = (_i64 * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr
