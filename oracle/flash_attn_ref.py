"""CPU oracle for the unmasked [B, H, T, D] attention of flash_attn_bhwd.  TEST INFRASTRUCTURE
ONLY: only `tests/` (and `bench.py`'s CPU baseline) may import it; the product path never does.

Restates megaqwen/triton_flash_attn.py:27-171 (kernel body :63-129): per (batch, head),
S = scale * q k^T over all T keys (no mask), the row softmax, O = softmax(S) v, and the result
rounded to q's 16-bit type (:126-127).  The reference evaluates blockwise with an online softmax
(running max m_i, sum l_i, rescale alpha = exp(m_i - m_ij), :101-122); that is the same function
as the direct softmax up to rounding, so the oracle computes it directly, in float64 from the
16-bit inputs widened exactly.  `scale` defaults to 1/sqrt(D) (:55-56).

Pinned (tests/test_flash_attn_cpu.py) against torch's scaled_dot_product_attention on the CPU
in float64 and against closed forms: T = 1 gives v; scale = 0 gives the mean of v over keys;
one dominant key gives its v row; a permutation of the keys (with v) changes nothing.
"""
from __future__ import annotations

import math

import numpy as np


def attention_bhwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    """softmax(scale * q k^T) v over the last two axes of [..., T, D] arrays, float64."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    v64 = np.asarray(v, dtype=np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q64.shape[-1])
    s = np.matmul(q64, np.swapaxes(k64, -1, -2)) * scale           # [..., Tq, Tk]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v64)
