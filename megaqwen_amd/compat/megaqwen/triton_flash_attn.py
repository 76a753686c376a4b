"""Drop-in for the reference's `megaqwen/triton_flash_attn.py` (`is_triton_available`,
`flash_attn_bhwd`, :18-171), for callers that put `megaqwen_amd/compat` on `sys.path`:

    sys.path.insert(0, "<repo>/megaqwen_amd/compat")
    from megaqwen.triton_flash_attn import flash_attn_bhwd

The implementation is megaqwen_amd.flash_attn (a hand-written gfx950 kernel; no Triton).
"""
from __future__ import annotations

import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

from megaqwen_amd.flash_attn import flash_attn_bhwd, is_triton_available  # noqa: E402,F401

__all__ = ["flash_attn_bhwd", "is_triton_available"]
