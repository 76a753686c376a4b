"""RoPE tables, following csrc/megakernel/megakernel_weights.py:131-137 (`_build_rope_tables`).

inv_freq[i] = 1 / theta^(2i/D) for i < D/2; freqs = outer(pos, inv_freq); the table row for a
position is [cos(freqs), cos(freqs)] (the half is repeated), then rounded to bf16.  The reference
builds them on the CUDA device; here they are built once on the host in fp32 and shared by the
GPU path and the CPU oracle, so both read identical bf16 tables.
"""
from __future__ import annotations

import torch


def build_rope_tables(max_seq_len: int, rope_theta: float, head_dim: int,
                      dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    inv_freq = 1.0 / (rope_theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    positions = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    cos = torch.cos(freqs).repeat(1, 2).to(dtype).contiguous()
    sin = torch.sin(freqs).repeat(1, 2).to(dtype).contiguous()
    return cos, sin
