"""MI355X-native batch-1 Qwen3-0.6B decode/prefill behind the MegaQwen Python API.

The compute path is libmegaqwen_hip.so: hand-written HIP for gfx950, with its C ABI declared in
include/megaqwen_hip.h. `megaqwen_amd.decoder` loads it with ctypes.

Importing this package does not load the library. Constructing a decoder does, and fails
loudly if the library is missing.

Modules:
- `decoder`: `MegakernelDecoder`, `MegakernelPrefillDecoder`.
- `generators`: `MegakernelGenerator`, `MegakernelPrefillGenerator`,
  `MegakernelFusedPrefillGenerator`.
- `weights`: `load_qwen3_weights`.
- `chat_ops`: the chat.py / generate.py function surfaces.
- `compat/megakernel_decode.py`: the reference's module name, for callers that put its
  directory on `sys.path`.
"""
from .spec import (  # noqa: F401
    configure_model_spec, configure_model_spec_from_model_dir, get_active_model_spec,
)
