"""Unmasked multi-head attention over [B, H, T, 64] on MI355X: the drop-in for
`megaqwen/triton_flash_attn.py` (the Qwen3-ASR audio tower's self-attention).

Same functions, arguments and ValueError contracts as the reference
(triton_flash_attn.py:18-50); the compute is the hand-written gfx950 kernel behind
`mq_flash_attn_bhwd` (include/megaqwen_hip.h, megaqwen_amd/csrc/flash_attn.hip).  There is no
Triton path and no PyTorch fallback: without the HIP library the call raises.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib


def is_triton_available() -> bool:
    """False: this build has no Triton kernel (triton_flash_attn.py:18-24 probes an import of
    triton; here nothing imports it, and `flash_attn_bhwd` does not depend on it)."""
    return False


def flash_attn_bhwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Compute attention(q, k, v) for q/k/v shaped [B, H, T, D] (no mask), D = 64.

    softmax(scale * q k^T) v per (batch, head) with fp32 scores, softmax and accumulation;
    the output has q's dtype (bf16 or fp16) and shape.  `scale` defaults to 1/sqrt(D)
    (triton_flash_attn.py:27-57).
    """
    # argument checks of triton_flash_attn.py:38-50, same order and messages
    if q.device.type != "cuda":
        raise ValueError("flash_attn_bhwd expects CUDA tensors")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"flash_attn_bhwd only supports fp16/bf16, got {q.dtype}")
    if q.ndim != 4:
        raise ValueError(f"Expected q.ndim=4 [B,H,T,D], got {tuple(q.shape)}")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"Shape mismatch q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    b, h, t, d = q.shape
    if d != 64:
        raise ValueError(f"Only head_dim=64 supported, got {d}")
    # the kernel reads k and v as q's element type on q's device
    for name, x in (("k", k), ("v", v)):
        if x.device != q.device:
            raise ValueError(f"{name} is on {x.device}, q on {q.device}")
        if x.dtype != q.dtype:
            raise ValueError(f"{name} has dtype {x.dtype}, q has {q.dtype}")

    if scale is None:
        scale = 1.0 / math.sqrt(d)

    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    out = torch.empty_like(q)
    if out.numel() == 0:
        return out
    lib = _lib.load()
    dtype = _lib.MQ_DTYPE_F16 if q.dtype == torch.float16 else _lib.MQ_DTYPE_BF16
    ws_bytes = lib.mq_flash_attn_workspace_bytes(b, h, t, d)
    if ws_bytes == 0:
        _lib.check(_lib.MQ_ERR_INVALID_ARG)
    # K and V^T in MFMA-operand order, written and consumed within the call (stream-ordered, so
    # the caching allocator may hand the block out again once the call is queued)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.check(lib.mq_flash_attn_bhwd(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          out.data_ptr(), b, h, t, d, dtype, float(scale),
                                          ws.data_ptr(), ws_bytes, stream))
    return out
