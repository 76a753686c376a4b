"""Drop-in for the reference's `megakernel_decode` module (csrc/megakernel/megakernel_decode.py,
megakernel_decode_impl.py:10-79).

The reference's callers put its kernel directory on `sys.path` and import this module by name
(verify_correctness.py:6,19; demo.py:4-6; benchmark_suite.py:81). Here the directory is
`megaqwen_amd/compat`:

    sys.path.insert(0, "<repo>/megaqwen_amd/compat")
    from megakernel_decode import MegakernelGenerator, load_qwen3_weights, ...

The module re-exports:
- the generators;
- the weight loader;
- the model-spec functions, and the `HIDDEN_SIZE … VOCAB_SIZE` constants, refreshed after each
  `configure_model_spec*` call as the reference's `_refresh_spec_aliases` does;
- the `_compile_*_kernel()` factories, which return objects holding the decoder classes (the
  HIP library is prebuilt, so nothing compiles).
"""
from __future__ import annotations

import os
import sys
import types

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

from megaqwen_amd import spec as _spec  # noqa: E402
from megaqwen_amd.decoder import (  # noqa: E402
    MegakernelDecoder, MegakernelFusedPrefillDecoder, MegakernelPrefillDecoder,
)
from megaqwen_amd.generators import (  # noqa: E402
    MegakernelFusedPrefillGenerator, MegakernelGenerator, MegakernelPrefillGenerator,
)
from megaqwen_amd.weights import load_qwen3_weights  # noqa: E402

HIDDEN_SIZE = INTERMEDIATE_SIZE = NUM_Q_HEADS = NUM_KV_HEADS = HEAD_DIM = 0
Q_SIZE = KV_SIZE = NUM_LAYERS = VOCAB_SIZE = 0


def _refresh_spec_aliases() -> None:
    g = globals()
    for name in ("HIDDEN_SIZE", "INTERMEDIATE_SIZE", "NUM_Q_HEADS", "NUM_KV_HEADS", "HEAD_DIM",
                 "Q_SIZE", "KV_SIZE", "NUM_LAYERS", "VOCAB_SIZE"):
        g[name] = getattr(_spec, name)


def get_active_model_spec() -> dict:
    return _spec.get_active_model_spec()


def configure_model_spec(**kwargs) -> dict:
    out = _spec.configure_model_spec(**kwargs)
    _refresh_spec_aliases()
    return out


def configure_model_spec_from_model_dir(model_dir: str) -> dict:
    out = _spec.configure_model_spec_from_model_dir(model_dir)
    _refresh_spec_aliases()
    return out


def _compile_decode_kernel():
    return types.SimpleNamespace(MegakernelDecoder=MegakernelDecoder)


def _compile_prefill_kernel():
    return types.SimpleNamespace(MegakernelPrefillDecoder=MegakernelPrefillDecoder)


def _compile_fused_prefill_kernel():
    return types.SimpleNamespace(MegakernelFusedPrefillDecoder=MegakernelFusedPrefillDecoder)


_refresh_spec_aliases()

__all__ = [
    "HIDDEN_SIZE", "INTERMEDIATE_SIZE", "NUM_Q_HEADS", "NUM_KV_HEADS", "HEAD_DIM", "Q_SIZE",
    "KV_SIZE", "NUM_LAYERS", "VOCAB_SIZE", "_compile_decode_kernel", "_compile_prefill_kernel",
    "_compile_fused_prefill_kernel", "configure_model_spec", "configure_model_spec_from_model_dir",
    "get_active_model_spec", "_refresh_spec_aliases", "load_qwen3_weights", "MegakernelGenerator",
    "MegakernelPrefillGenerator", "MegakernelFusedPrefillGenerator",
]
