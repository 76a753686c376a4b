"""Model-spec registry for the Qwen3 decode/prefill path.

Mirrors the reference's spec API (`configure_model_spec`, `configure_model_spec_from_model_dir`,
`get_active_model_spec` and the module constants `HIDDEN_SIZE ... VOCAB_SIZE`) from
csrc/megakernel/megakernel_kernels.py:13-22,45-122 and the re-export layer in
csrc/megakernel/megakernel_decode_impl.py:24-70.

The HIP library compiles the per-layer shape (hidden 1024, intermediate 3072, 16 Q / 8 KV heads,
head_dim 128) as constants; `num_layers` and `vocab_size` are run-time values.  A spec whose
layer shape differs from the compiled one is rejected by the library at model creation.
"""
from __future__ import annotations

import json
import os
from pathlib import Path

_DEFAULT_MODEL_SPEC = {
    "hidden_size": 1024,
    "intermediate_size": 3072,
    "num_q_heads": 16,
    "num_kv_heads": 8,
    "head_dim": 128,
    "num_layers": 28,
    "vocab_size": 151936,
}

# Layer shape the HIP kernels are compiled for (csrc/megaqwen_config.h).
COMPILED_LAYER_SHAPE = {
    "hidden_size": 1024,
    "intermediate_size": 3072,
    "num_q_heads": 16,
    "num_kv_heads": 8,
    "head_dim": 128,
}

RMS_EPS = 1e-6
ROPE_THETA = 1000000.0

_ACTIVE_MODEL_SPEC = dict(_DEFAULT_MODEL_SPEC)

HIDDEN_SIZE = INTERMEDIATE_SIZE = NUM_Q_HEADS = NUM_KV_HEADS = HEAD_DIM = 0
Q_SIZE = KV_SIZE = NUM_LAYERS = VOCAB_SIZE = 0


def _sync_constants() -> None:
    global HIDDEN_SIZE, INTERMEDIATE_SIZE, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM
    global Q_SIZE, KV_SIZE, NUM_LAYERS, VOCAB_SIZE
    s = _ACTIVE_MODEL_SPEC
    HIDDEN_SIZE = int(s["hidden_size"])
    INTERMEDIATE_SIZE = int(s["intermediate_size"])
    NUM_Q_HEADS = int(s["num_q_heads"])
    NUM_KV_HEADS = int(s["num_kv_heads"])
    HEAD_DIM = int(s["head_dim"])
    Q_SIZE = NUM_Q_HEADS * HEAD_DIM
    KV_SIZE = NUM_KV_HEADS * HEAD_DIM
    NUM_LAYERS = int(s["num_layers"])
    VOCAB_SIZE = int(s["vocab_size"])


def normalize_model_spec(spec: dict) -> dict:
    """Validation rules of the reference (megakernel_kernels.py:56-81)."""
    out = {k: int(spec[k]) for k in _DEFAULT_MODEL_SPEC}
    if out["hidden_size"] <= 0 or out["intermediate_size"] <= 0:
        raise ValueError(f"Invalid model spec: {out}")
    if out["num_q_heads"] <= 0 or out["num_kv_heads"] <= 0 or out["head_dim"] <= 0:
        raise ValueError(f"Invalid attention spec: {out}")
    if out["num_q_heads"] % out["num_kv_heads"] != 0:
        raise ValueError(f"num_q_heads must be divisible by num_kv_heads: {out}")
    if out["num_layers"] <= 0 or out["vocab_size"] <= 0:
        raise ValueError(f"Invalid model spec: {out}")
    return out


def get_active_model_spec() -> dict:
    return dict(_ACTIVE_MODEL_SPEC)


def configure_model_spec(*, hidden_size: int, intermediate_size: int, num_q_heads: int,
                         num_kv_heads: int, head_dim: int, num_layers: int,
                         vocab_size: int) -> dict:
    global _ACTIVE_MODEL_SPEC
    _ACTIVE_MODEL_SPEC = normalize_model_spec(dict(
        hidden_size=hidden_size, intermediate_size=intermediate_size, num_q_heads=num_q_heads,
        num_kv_heads=num_kv_heads, head_dim=head_dim, num_layers=num_layers,
        vocab_size=vocab_size))
    _sync_constants()
    return get_active_model_spec()


def spec_from_config_dict(cfg: dict) -> dict:
    """Reads a HF `config.json` dict (plain Qwen3 or the Qwen3-ASR thinker layout)."""
    text = cfg
    if cfg.get("model_type") == "qwen3_asr" or "thinker_config" in cfg:
        text = cfg["thinker_config"]["text_config"]
    hidden = int(text["hidden_size"])
    heads = int(text["num_attention_heads"])
    return normalize_model_spec(dict(
        hidden_size=hidden,
        intermediate_size=int(text["intermediate_size"]),
        num_q_heads=heads,
        num_kv_heads=int(text["num_key_value_heads"]),
        head_dim=int(text.get("head_dim", hidden // heads)),
        num_layers=int(text["num_hidden_layers"]),
        vocab_size=int(text.get("vocab_size", cfg.get("vocab_size", 151936))),
    ))


def configure_model_spec_from_model_dir(model_dir: str | os.PathLike) -> dict:
    cfg = json.loads((Path(model_dir) / "config.json").read_text(encoding="utf-8"))
    return configure_model_spec(**spec_from_config_dict(cfg))


def check_compiled_layer_shape(spec: dict) -> None:
    """Raises ValueError when the layer shape differs from the one the kernels are built for."""
    bad = {k: (spec[k], v) for k, v in COMPILED_LAYER_SHAPE.items() if int(spec[k]) != v}
    if bad:
        raise ValueError(f"HIP kernels are compiled for the Qwen3-0.6B layer shape; mismatched: {bad}")


_sync_constants()
