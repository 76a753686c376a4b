"""Host-side parts of the drop-in surface that need no GPU:
- the safetensors checkpoint loader (key map, tied LM head, ASR prefix, sharded index);
- the byte tokenizer of random-init runs;
- the `megakernel_decode` compatibility module and its spec constants.
"""
import importlib
import json
import os
import sys

import pytest
import torch

from megaqwen_amd import spec as mq_spec
from megaqwen_amd.weights import (SyntheticTokenizer, W4_KEYS, load_local_checkpoint,
                                  load_qwen3_weights, resolve_local_model_dir)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUFFIXES = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
            "self_attn.v_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
            "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
            "mlp.up_proj.weight", "mlp.down_proj.weight")
SHAPES = ((1024,), (2048, 1024), (1024, 1024), (1024, 1024), (128,), (128,), (1024, 2048),
          (1024,), (3072, 1024), (3072, 1024), (1024, 3072))


@pytest.fixture
def restore_spec():
    saved = mq_spec.get_active_model_spec()
    yield
    mq_spec.configure_model_spec(**saved)


def _write_ckpt(d, prefix="model.", lm_key=None, vocab=64, layers=2, shards=1, asr=False):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    t = {prefix + "embed_tokens.weight": torch.randn(vocab, 1024, generator=g),
         prefix + "norm.weight": torch.randn(1024, generator=g)}
    for i in range(layers):
        for s, shp in zip(SUFFIXES, SHAPES):
            t[f"{prefix}layers.{i}.{s}"] = torch.randn(*shp, generator=g)
    if lm_key:
        t[lm_key] = torch.randn(vocab, 1024, generator=g)
    text = dict(hidden_size=1024, intermediate_size=3072, num_attention_heads=16,
                num_key_value_heads=8, head_dim=128, num_hidden_layers=layers, vocab_size=vocab,
                rope_theta=1e6)
    cfg = {"model_type": "qwen3_asr", "thinker_config": {"text_config": text}} if asr else \
        dict(text, model_type="qwen3")
    (d / "config.json").write_text(json.dumps(cfg))
    keys = sorted(t)
    if shards == 1:
        save_file({k: t[k].to(torch.bfloat16) for k in keys}, str(d / "model.safetensors"))
    else:
        wm = {}
        for s in range(shards):
            part = keys[s::shards]
            name = f"model-{s:05d}.safetensors"
            save_file({k: t[k].to(torch.bfloat16) for k in part}, str(d / name))
            wm.update({k: name for k in part})
        (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    return {k: v.to(torch.bfloat16) for k, v in t.items()}


@pytest.mark.parametrize("shards", [1, 3])
def test_local_checkpoint_key_map_and_tied_head(tmp_path, restore_spec, shards):
    ref = _write_ckpt(tmp_path, shards=shards)
    w = load_local_checkpoint(tmp_path, max_seq_len=16, device="cpu")
    assert mq_spec.get_active_model_spec()["num_layers"] == 2
    assert mq_spec.VOCAB_SIZE == 64
    assert len(w["layer_weights"]) == 22
    for i in range(2):
        for j, s in enumerate(SUFFIXES):
            assert torch.equal(w["layer_weights"][11 * i + j], ref[f"model.layers.{i}.{s}"])
    assert torch.equal(w["embed_weight"], ref["model.embed_tokens.weight"])
    assert w["lm_head_weight"] is w["embed_weight"]            # tied fallback
    assert torch.equal(w["final_norm_weight"], ref["model.norm.weight"])
    assert w["cos_table"].shape == (16, 128) and w["cos_table"].dtype == torch.bfloat16
    assert all(w[k] == [] for k in W4_KEYS)


def test_local_checkpoint_asr_prefix_and_untied_head(tmp_path, restore_spec):
    ref = _write_ckpt(tmp_path, prefix="thinker.model.", lm_key="thinker.lm_head.weight", asr=True,
                      layers=1)
    w = load_local_checkpoint(tmp_path, max_seq_len=8, device="cpu")
    assert torch.equal(w["lm_head_weight"], ref["thinker.lm_head.weight"])
    assert torch.equal(w["layer_weights"][1], ref["thinker.model.layers.0.self_attn.q_proj.weight"])


def test_loader_rejects_other_layer_shapes_and_missing_dirs(tmp_path, restore_spec):
    _write_ckpt(tmp_path, layers=1)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["hidden_size"] = 2048
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError):
        load_local_checkpoint(tmp_path, max_seq_len=8, device="cpu")
    with pytest.raises(FileNotFoundError):
        load_qwen3_weights("Qwen/definitely-not-a-local-dir")
    assert resolve_local_model_dir(str(tmp_path)) == tmp_path


def test_synthetic_tokenizer_round_trip():
    tok = SyntheticTokenizer()
    ids = tok.encode("héllo, 世界")
    assert all(0 <= i < 256 for i in ids)
    assert tok.decode(ids) == "héllo, 世界"
    assert tok.decode(ids + [tok.eos_token_id]) == "héllo, 世界"
    assert tok.decode([104, 151000, 105]) == "h<151000>i"
    assert tok("ab", return_tensors="pt")["input_ids"].tolist() == [[97, 98]]


def test_megakernel_decode_module_surface(restore_spec):
    sys.path.insert(0, os.path.join(ROOT, "megaqwen_amd", "compat"))
    try:
        mk = importlib.import_module("megakernel_decode")
    finally:
        sys.path.pop(0)
    for name in mk.__all__:
        assert hasattr(mk, name), name
    assert mk.HIDDEN_SIZE == 1024 and mk.Q_SIZE == 2048 and mk.KV_SIZE == 1024
    mk.configure_model_spec(hidden_size=1024, intermediate_size=3072, num_q_heads=16,
                            num_kv_heads=8, head_dim=128, num_layers=3, vocab_size=1000)
    assert mk.NUM_LAYERS == 3 and mk.VOCAB_SIZE == 1000
    assert mk.get_active_model_spec()["num_layers"] == 3
    assert mk._compile_prefill_kernel().MegakernelPrefillDecoder.__name__ == "MegakernelPrefillDecoder"
    with pytest.raises(ValueError):
        mk.configure_model_spec(hidden_size=1024, intermediate_size=3072, num_q_heads=16,
                                num_kv_heads=6, head_dim=128, num_layers=3, vocab_size=1000)
