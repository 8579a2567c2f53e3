"""Online-softmax LSE merge on the MI355X (``update_out_and_lse``, ring/merge.py:13-31).

Same contract as the reference: ``out/block_out`` ``[b, s, h, d]``, ``lse``
``[b, s, h, 1]`` fp32, ``block_lse`` ``[b, h, s]`` (flash layout); the first block
initialises the running pair (``out is None``). The update runs as one HBM-bound
kernel instead of the reference's chain of elementwise ops; it is applied in place
to the running fp32 tensors (callers rebind ``out, lse = update_out_and_lse(...)``
as the reference's do) and is not differentiable. Inside the ring forward the
same merge is fused into the attention epilogue instead (rmx_attn_fwd modes).
"""

from __future__ import annotations

import torch

from ringmaster_amd import abi


def _lse_to_bshd(block_lse: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """Flash LSE ``[b, h, s]`` -> ``[b, s, h, 1]`` fp32 (ring/merge.py:13-17)."""
    if block_lse.dim() == 3 and block_lse.shape[1] == like.shape[2]:
        block_lse = block_lse.transpose(1, 2)
    return block_lse.unsqueeze(-1).contiguous().to(torch.float32)


def update_out_and_lse(out, lse, block_out: torch.Tensor, block_lse: torch.Tensor):
    """Merge one block's (out, lse) into the running (out, lse); returns the pair."""
    abi.require_device(block_out, block_lse, out, lse)
    b, s, h, d = block_out.shape
    if block_lse.shape != (b, h, s):
        raise ValueError(f"block_lse must be [b, h, s] = {(b, h, s)} (got {tuple(block_lse.shape)})")
    blk_types = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}  # RMX_BLK_*
    if block_out.dtype not in blk_types:
        raise NotImplementedError(f"block_out dtype {block_out.dtype} (bf16, fp16 or fp32)")
    if block_out.stride(-1) != 1 or block_out.data_ptr() % 16:
        block_out = block_out.contiguous()
    if block_lse.dtype != torch.float32 or block_lse.stride(-1) != 1:
        block_lse = block_lse.float().contiguous()
    init = out is None
    if init:
        out = torch.empty((b, s, h, d), dtype=torch.float32, device=block_out.device)
        lse = torch.empty((b, s, h, 1), dtype=torch.float32, device=block_out.device)
    else:
        if out.dtype != torch.float32 or lse.dtype != torch.float32:
            raise ValueError("the running out/lse must be fp32")
        if out.shape != (b, s, h, d) or lse.shape != (b, s, h, 1):
            raise ValueError("running out/lse shapes do not match the block")
    lse3 = lse.squeeze(-1)
    lib = abi.lib()
    abi.check(lib.rmx_lse_merge(
        out.data_ptr(), lse3.data_ptr(), block_out.data_ptr(),
        blk_types[block_out.dtype], block_lse.data_ptr(), b, s, h, d,
        abi.i64_array(out.stride()[:3]), abi.i64_array(lse3.stride()),
        abi.i64_array(block_out.stride()[:3]), abi.i64_array(block_lse.stride()[:2]),
        int(init), abi.stream_of(block_out)))
    return out, lse
