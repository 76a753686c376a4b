"""The HuggingFace side of megaqwen_amd.verify_correctness without a GPU: a checkpoint directory
in the Qwen3 safetensors layout (a small shape) read by `AutoModelForCausalLM`, and the same
weights loaded into a `Qwen3Config` model, give the unrounded fp32 oracle's logits and greedy
tokens."""
import json

import torch

from megaqwen_amd.rope import build_rope_tables
from megaqwen_amd.synthetic import make_tokens, make_weights
from megaqwen_amd.verify_correctness import _hf_from_dir, _hf_from_weights, _hf_greedy, main
from oracle.ref_cpu import OracleModel

SPEC = dict(hidden_size=256, intermediate_size=512, num_q_heads=4, num_kv_heads=2, head_dim=64,
            num_layers=2, vocab_size=1000)
NAMES = ["input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
         "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj", "post_attention_layernorm",
         "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]


def _write_checkpoint(d, w):
    from safetensors.torch import save_file
    t = {"model.embed_tokens.weight": w["embed_weight"], "model.norm.weight": w["final_norm_weight"]}
    for i in range(SPEC["num_layers"]):
        for j, n in enumerate(NAMES):
            t[f"model.layers.{i}.{n}.weight"] = w["layer_weights"][11 * i + j]
    save_file({k: v.contiguous() for k, v in t.items()}, str(d / "model.safetensors"))
    cfg = {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
           "hidden_size": SPEC["hidden_size"], "intermediate_size": SPEC["intermediate_size"],
           "num_attention_heads": SPEC["num_q_heads"], "num_key_value_heads": SPEC["num_kv_heads"],
           "head_dim": SPEC["head_dim"], "num_hidden_layers": SPEC["num_layers"],
           "vocab_size": SPEC["vocab_size"], "rms_norm_eps": 1e-6, "rope_theta": 1000000.0,
           "max_position_embeddings": 4096, "tie_word_embeddings": True, "attention_bias": False,
           "hidden_act": "silu", "torch_dtype": "bfloat16"}
    (d / "config.json").write_text(json.dumps(cfg))


def test_hf_models_match_unrounded_oracle(tmp_path):
    w = make_weights(SPEC, seed=7, norm_jitter=0.2)
    _write_checkpoint(tmp_path, w)
    prompt = make_tokens(6, SPEC["vocab_size"], seed=8).tolist()
    cos, sin = build_rope_tables(64, 1e6, SPEC["head_dim"], dtype=torch.float32)
    orc = OracleModel(make_weights(SPEC, seed=7, norm_jitter=0.2, dtype=torch.float32), SPEC,
                      cos, sin, 64, round_bf16=False)
    for t in prompt[:-1]:
        orc.decode_step(t, return_logits=False)
    ref_toks, ref_logits, cur = [], [], prompt[-1]
    for _ in range(5):
        tok, lg = orc.decode_step(cur)
        ref_toks.append(tok)
        ref_logits.append(lg)
        cur = tok
    for model in (_hf_from_dir(str(tmp_path)), _hf_from_weights(w, SPEC, 1e6)):
        toks, logits = _hf_greedy(model, prompt, 5)
        assert toks == ref_toks
        for a, b in zip(logits, ref_logits):
            assert float((a - b).abs().max()) < 1e-4


def test_cli_help(capsys):
    try:
        main(["--help"])
    except SystemExit as e:
        assert e.code == 0
    assert "--model" in capsys.readouterr().out
