"""ctypes binding of libmegaqwen_hip.so (C ABI: include/megaqwen_hip.h).

The library is loaded from this package directory only.  There is no fallback: if the HIP
library is missing, importing the decoder classes raises, so nothing can silently run a CPU
path in its place.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmegaqwen_hip.so")
ABI_VERSION = 1

MQ_OK = 0
MQ_ERR_INVALID_ARG = -1
MQ_ERR_HIP = -2
MQ_ERR_POSITION = -3
MQ_ERR_DEVICE = -4
MQ_ERR_UNSUPPORTED = -5
MQ_MODE_PERSISTENT = 0
MQ_MODE_MULTI_KERNEL = 1
MQ_DTYPE_BF16 = 0
MQ_DTYPE_F16 = 1

# Every symbol include/megaqwen_hip.h declares (tests check the library exports all of them).
EXPORTED = (
    "mq_abi_version", "mq_last_error", "mq_workspace_bytes", "mq_kv_cache_bytes",
    "mq_decoder_create", "mq_decoder_destroy", "mq_decoder_reset", "mq_decoder_position",
    "mq_decoder_set_host_position", "mq_decoder_set_position", "mq_decoder_set_mode", "mq_decoder_get_mode", "mq_decoder_grid", "mq_decode_step",
    "mq_decode_steps", "mq_debug_decode_step_layers", "mq_debug_decode_step_timing", "mq_decoder_check", "mq_prefill", "mq_prefill_embeds", "mq_prefill_fused", "mq_debug_prefill_layers", "mq_debug_prefill_buffers", "mq_op_qkv_rope", "mq_op_attention", "mq_op_attention_noalloc",
    "mq_op_mlp", "mq_op_decode_layer", "mq_op_lm_head", "mq_flash_attn_workspace_bytes",
    "mq_flash_attn_bhwd", "mq_exchange_epoch", "mq_exchange_epoch_advance", "mq_exchange_tag",
    "mq_exchange_epoch_period", "mq_debug_set_exchange_epoch", "mq_debug_get_exchange_epoch",
)


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
        "post_attn_layernorm", "gate_proj", "up_proj", "down_proj")]


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int), ("intermediate_size", ctypes.c_int),
        ("num_q_heads", ctypes.c_int), ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("num_layers", ctypes.c_int), ("vocab_size", ctypes.c_int),
        ("max_seq_len", ctypes.c_int), ("max_prefill_len", ctypes.c_int),
        ("embed", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
        ("lm_head", ctypes.c_void_p), ("cos_table", ctypes.c_void_p),
        ("sin_table", ctypes.c_void_p), ("layers", ctypes.POINTER(LayerWeights)),
    ]


class MegaQwenError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m megaqwen_amd.build`")
    lib = ctypes.CDLL(path)
    P, I, S, U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint32
    sig = {
        "mq_abi_version": (I, []),
        "mq_last_error": (ctypes.c_char_p, []),
        "mq_workspace_bytes": (S, [ctypes.POINTER(ModelDesc)]),
        "mq_kv_cache_bytes": (S, [ctypes.POINTER(ModelDesc)]),
        "mq_decoder_create": (I, [ctypes.POINTER(ModelDesc), P, P, P, S, ctypes.POINTER(P)]),
        "mq_decoder_destroy": (I, [P]),
        "mq_decoder_reset": (I, [P, P]),
        "mq_decoder_position": (I, [P]),
        "mq_decoder_set_host_position": (I, [P, I]),
        "mq_decoder_set_position": (I, [P, I, P]),
        "mq_decoder_set_mode": (I, [P, I]),
        "mq_decoder_get_mode": (I, [P]),
        "mq_decoder_grid": (I, [P]),
        "mq_decode_step": (I, [P, P, P, P, P]),
        "mq_decode_steps": (I, [P, P, I, P]),
        "mq_debug_decode_step_layers": (I, [P, P, P, P, P, P]),
        "mq_debug_decode_step_timing": (I, [P, P, P, P, P]),
        "mq_decoder_check": (I, [P, P]),
        "mq_prefill": (I, [P, P, I, P, P, P]),
        "mq_prefill_embeds": (I, [P, P, I, P, I, I, P, P, P]),
        "mq_prefill_fused": (I, [P, P, I, P, I, I, P, P, P]),
        "mq_debug_prefill_layers": (I, [P, P, I, P, P, P, P]),
        "mq_debug_prefill_buffers": (I, [P, ctypes.POINTER(P)]),
        "mq_op_qkv_rope": (I, [P, I, P, I, P, P]),
        "mq_op_attention": (I, [P, I, P, I, P, P]),
        "mq_op_attention_noalloc": (I, [P, I, P, I, P, P]),
        "mq_op_mlp": (I, [P, I, P, P, P]),
        "mq_op_decode_layer": (I, [P, I, P, I, P, P]),
        "mq_op_lm_head": (I, [P, P, P, P, P]),
        "mq_flash_attn_workspace_bytes": (S, [I, I, I, I]),
        "mq_flash_attn_bhwd": (I, [P, P, P, P, I, I, I, I, I, ctypes.c_float, P, S, P]),
        "mq_exchange_epoch": (U32, [U32, ctypes.c_uint64]),
        "mq_exchange_epoch_advance": (U32, [U32, ctypes.c_uint64]),
        "mq_exchange_tag": (U32, [U32]),
        "mq_exchange_epoch_period": (U32, []),
        "mq_debug_set_exchange_epoch": (I, [P, U32, P]),
        "mq_debug_get_exchange_epoch": (I, [P, ctypes.POINTER(U32), P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mq_abi_version() != ABI_VERSION:
        raise ImportError(f"{path}: ABI version {lib.mq_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != MQ_OK:
        msg = _lib.mq_last_error().decode() if _lib is not None else "libmegaqwen_hip error"
        raise MegaQwenError(rc, msg)
