"""Weight loading with the reference's `load_qwen3_weights` contract
(csrc/megakernel/megakernel_weights.py:220-505).

`load_qwen3_weights(model_name, max_seq_len)` returns the reference's dict:
- `embed_weight`;
- the flat `layer_weights`, 11 per layer in the order input_layernorm, q, k, v, q_norm, k_norm,
  o, post_attention_layernorm, gate, up, down (megakernel_weights.py:11-33,109-128);
- `final_norm_weight` and `lm_head_weight` (tied to the embedding when the checkpoint has no
  `lm_head.weight`, :270-277,478);
- bf16 RoPE `cos_table` / `sin_table` for `max_seq_len` positions;
- `tokenizer`;
- the empty W4 lists the bf16 path carries.

Every tensor is contiguous bf16 on the CUDA device.

Two sources are supported, because there is no network here:
- **A local checkpoint directory** (`config.json` + `model.safetensors` or a sharded
  `model.safetensors.index.json`), read with safetensors. That covers plain Qwen3 keys
  (`model.`) and the Qwen3-ASR thinker layout (`thinker.model.`), as :236-262 do. The tokenizer
  is loaded from the same directory with `transformers.AutoTokenizer` (local files only).
- **`model_name` of the form `random` or `random:<seed>`**: the seeded N(0, 0.02) random-init
  weights of the Qwen3-0.6B architecture (`megaqwen_amd.synthetic`), with the byte-level
  `SyntheticTokenizer` below.

A hub model name such as "Qwen/Qwen3-0.6B" resolves like the reference's
`_resolve_local_model_dir` (:140-148): the path itself, else its last component as a local
directory. Otherwise it raises FileNotFoundError instead of downloading.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from . import spec as _spec
from .rope import build_rope_tables
from .synthetic import make_weights

W4_KEYS = tuple(f"split_{m}_w4_{k}" for m in ("q", "k", "v", "o", "gateup", "down")
                for k in ("packed", "scales", "codebook"))

_LAYER_SUFFIXES = (
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
    "self_attn.v_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
    "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
    "mlp.up_proj.weight", "mlp.down_proj.weight",
)


class SyntheticTokenizer:
    """Byte-level stand-in tokenizer for random-init runs (no vocabulary files offline).

    Text is encoded as its UTF-8 bytes mapped to ids 0..255. Decoding maps ids below 256 back
    to bytes and renders any other id as `<id>`. `eos_token_id` is Qwen3's `<|im_end|>`
    (151645).
    """

    eos_token_id = 151645

    def encode(self, text: str, add_special_tokens: bool = True) -> list[int]:
        return list(text.encode("utf-8")) or [0]

    def decode(self, ids, skip_special_tokens: bool = True) -> str:
        out = bytearray()
        parts = []
        for t in (int(i) for i in ids):
            if t < 256:
                out.append(t)
            else:
                if out:
                    parts.append(out.decode("utf-8", errors="replace"))
                    out = bytearray()
                if not (skip_special_tokens and t == self.eos_token_id):
                    parts.append(f"<{t}>")
        if out:
            parts.append(out.decode("utf-8", errors="replace"))
        return "".join(parts)

    def __call__(self, text: str, return_tensors=None):
        ids = self.encode(text)
        if return_tensors == "pt":
            return {"input_ids": torch.tensor([ids], dtype=torch.long)}
        return {"input_ids": ids}


def _bf16(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.bfloat16).contiguous()


def resolve_local_model_dir(model_name: str) -> Path | None:
    """megakernel_weights.py:140-148: the path itself, else its last '/' component."""
    d = Path(model_name)
    if not d.exists() and "/" in str(model_name):
        alt = Path(str(model_name).split("/")[-1])
        if alt.is_dir():
            d = alt
    return d if d.is_dir() else None


def _checkpoint_files(model_dir: Path) -> dict[str, Path]:
    """tensor key -> safetensors file (sharded index or a single model.safetensors)."""
    index = model_dir / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text(encoding="utf-8")).get("weight_map")
        if not isinstance(weight_map, dict):
            raise ValueError(f"Invalid safetensors index: {index}")
        return {str(k): model_dir / str(v) for k, v in weight_map.items()}
    ckpt = model_dir / "model.safetensors"
    if not ckpt.exists():
        raise FileNotFoundError(f"Missing checkpoint: {ckpt}")
    from safetensors import safe_open
    with safe_open(str(ckpt), framework="pt", device="cpu") as f:
        return {k: ckpt for k in f.keys()}


def _read_tensors(files: dict[str, Path], keys: list[str], device) -> dict[str, torch.Tensor]:
    from safetensors import safe_open
    by_file: dict[Path, list[str]] = {}
    for k in keys:
        if k not in files:
            raise KeyError(f"checkpoint has no tensor {k!r}")
        by_file.setdefault(files[k], []).append(k)
    out = {}
    for path, ks in by_file.items():
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for k in ks:
                out[k] = _bf16(f.get_tensor(k), device)
    return out


def load_local_checkpoint(model_dir: Path, max_seq_len: int, device="cuda") -> dict:
    cfg_path = model_dir / "config.json"
    cfg = json.loads(cfg_path.read_text(encoding="utf-8")) if cfg_path.exists() else {}
    asr = cfg.get("model_type") == "qwen3_asr" or "thinker_config" in cfg
    prefix = "thinker.model." if asr else "model."
    lm_key = "thinker.lm_head.weight" if asr else "lm_head.weight"
    text_cfg = cfg["thinker_config"]["text_config"] if asr else cfg
    if "hidden_size" in text_cfg:
        _spec.configure_model_spec(**_spec.spec_from_config_dict(cfg))
    spec = _spec.get_active_model_spec()
    _spec.check_compiled_layer_shape(spec)
    rope_theta = float(text_cfg.get("rope_theta", _spec.ROPE_THETA))
    files = _checkpoint_files(model_dir)
    n = int(spec["num_layers"])
    keys = [prefix + "embed_tokens.weight", prefix + "norm.weight"]
    keys += [f"{prefix}layers.{i}.{s}" for i in range(n) for s in _LAYER_SUFFIXES]
    if lm_key in files:
        keys.append(lm_key)
    t = _read_tensors(files, keys, device)
    if any(v.dtype == torch.uint8 for v in t.values()):
        raise NotImplementedError("quantised (uint8) checkpoints are not supported")
    embed = t[prefix + "embed_tokens.weight"]
    cos, sin = build_rope_tables(max_seq_len, rope_theta, int(spec["head_dim"]))
    # the tokenizer only from this directory's own files: without them AutoTokenizer can resolve
    # config.json's model type to a tokenizer found elsewhere, whose ids need not fit this vocab
    tokenizer = None
    if any((model_dir / f).exists() for f in ("tokenizer.json", "tokenizer_config.json",
                                              "vocab.json")):
        try:
            from transformers import AutoTokenizer
            tokenizer = AutoTokenizer.from_pretrained(str(model_dir), local_files_only=True)
        except Exception:  # unreadable tokenizer files still leave usable weights
            tokenizer = None
    out = {
        "embed_weight": embed,
        "layer_weights": [t[f"{prefix}layers.{i}.{s}"] for i in range(n) for s in _LAYER_SUFFIXES],
        "final_norm_weight": t[prefix + "norm.weight"],
        "lm_head_weight": t.get(lm_key, embed),
        "cos_table": cos.to(device),
        "sin_table": sin.to(device),
        "tokenizer": tokenizer,
    }
    out.update({k: [] for k in W4_KEYS})
    return out


def load_random_init(max_seq_len: int, seed: int = 0, device="cuda") -> dict:
    spec = _spec.get_active_model_spec()
    _spec.check_compiled_layer_shape(spec)
    w = make_weights(spec, seed=seed)
    embed = _bf16(w["embed_weight"], device)
    cos, sin = build_rope_tables(max_seq_len, _spec.ROPE_THETA, int(spec["head_dim"]))
    out = {
        "embed_weight": embed,
        "layer_weights": [_bf16(x, device) for x in w["layer_weights"]],
        "final_norm_weight": _bf16(w["final_norm_weight"], device),
        "lm_head_weight": embed,
        "cos_table": cos.to(device),
        "sin_table": sin.to(device),
        "tokenizer": SyntheticTokenizer(),
    }
    out.update({k: [] for k in W4_KEYS})
    return out


def load_qwen3_weights(model_name: str = "Qwen/Qwen3-0.6B", max_seq_len: int = 2048):
    """megakernel_weights.py:220-505, restricted to the two offline sources described in the
    module docstring."""
    name = str(model_name)
    if name == "random" or name.startswith("random:"):
        seed = int(name.split(":", 1)[1]) if ":" in name else 0
        return load_random_init(max_seq_len, seed=seed)
    model_dir = resolve_local_model_dir(name)
    if model_dir is None:
        raise FileNotFoundError(
            f"{name!r} is not a local model directory. Weights are not downloaded: pass a "
            f"directory with config.json + model.safetensors, or 'random[:seed]' for "
            f"seeded random-init weights")
    return load_local_checkpoint(model_dir, max_seq_len)
