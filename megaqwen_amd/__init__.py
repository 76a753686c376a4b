"""MI355X-native batch-1 Qwen3-0.6B decode/prefill behind the MegaQwen Python API.

The compute path is libmegaqwen_hip.so (hand-written HIP for gfx950, C ABI in
include/megaqwen_hip.h), loaded with ctypes by `megaqwen_amd.decoder`.  Importing this package
does not load the library; constructing a decoder does, and fails loudly if it is missing.
"""
from .spec import (  # noqa: F401
    configure_model_spec, configure_model_spec_from_model_dir, get_active_model_spec,
)
