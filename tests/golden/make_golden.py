"""Writes the golden fixtures that pin the CPU oracle (tests/golden/*.npz).

The reference has no committed golden vectors (it verifies against HuggingFace
`Qwen3ForCausalLM` at run time: verify_correctness.py:8-63, qwen3-0.6b.py:832-931).  These
fixtures come from that same model class, `transformers` 5.15.0 (`Qwen3ForCausalLM`, built from a
local `Qwen3Config`, random init, nothing fetched), in fp32 with its own eager attention, loaded
with the seeded synthetic weights of megaqwen_amd.synthetic.  They pin the model math the oracle
restates: RMSNorm placement and eps, per-head q/k RMSNorm, rotate-half RoPE with theta 1e6, the
GQA head mapping, attention scale, causal masking, SwiGLU, the tied LM head and incremental
decoding with a KV cache.

Stored per case: the config, the weight seed / jitter, prompt tokens, fp32 logits at every prompt
position, greedy continuation tokens (HF incremental decode) and the fp32 logits of each decode
step.  Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from megaqwen_amd.synthetic import make_weights, make_tokens  # noqa: E402

CASES = {
    # real Qwen3-0.6B layer shape, 2 layers, small vocab
    "qwen3_layer_2l": dict(hidden_size=1024, intermediate_size=3072, num_q_heads=16, num_kv_heads=8,
                           head_dim=128, num_layers=2, vocab_size=2048, seed=3, norm_jitter=0.1,
                           n_prompt=12, n_decode=6),
    # a different shape (head_dim 64, 4 Q / 2 KV heads) so shape-specific slips surface
    "small_shape_3l": dict(hidden_size=256, intermediate_size=512, num_q_heads=4, num_kv_heads=2,
                           head_dim=64, num_layers=3, vocab_size=1000, seed=5, norm_jitter=0.2,
                           n_prompt=9, n_decode=5),
}


def hf_model(spec: dict, weights: dict):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(
        vocab_size=spec["vocab_size"], hidden_size=spec["hidden_size"],
        intermediate_size=spec["intermediate_size"], num_hidden_layers=spec["num_layers"],
        num_attention_heads=spec["num_q_heads"], num_key_value_heads=spec["num_kv_heads"],
        head_dim=spec["head_dim"], rms_norm_eps=1e-6, max_position_embeddings=4096,
        rope_parameters={"rope_type": "default", "rope_theta": 1000000.0},
        tie_word_embeddings=True, attention_bias=False, use_sliding_window=False,
        attn_implementation="eager", dtype=torch.float32)
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).to(torch.float32).eval()
    sd = model.state_dict()
    f = lambda t: t.to(torch.float32)
    new = {"model.embed_tokens.weight": f(weights["embed_weight"]),
           "model.norm.weight": f(weights["final_norm_weight"]),
           "lm_head.weight": f(weights["lm_head_weight"])}
    names = ["input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
             "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj",
             "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    for i in range(spec["num_layers"]):
        for j, nm in enumerate(names):
            new[f"model.layers.{i}.{nm}.weight"] = f(weights["layer_weights"][i * 11 + j])
    missing = set(sd) - set(new)
    assert not missing, missing
    model.load_state_dict(new, strict=True)
    return model


@torch.no_grad()
def run_case(name: str, c: dict) -> dict:
    spec = {k: c[k] for k in ("hidden_size", "intermediate_size", "num_q_heads", "num_kv_heads",
                               "head_dim", "num_layers", "vocab_size")}
    w = make_weights(spec, seed=c["seed"], norm_jitter=c["norm_jitter"])
    model = hf_model(spec, w)
    toks = make_tokens(c["n_prompt"], spec["vocab_size"], seed=c["seed"]).to(torch.long)
    out = model(input_ids=toks.unsqueeze(0), use_cache=True)
    prompt_logits = out.logits[0].float().numpy()
    past = out.past_key_values
    nxt = int(np.argmax(prompt_logits[-1]))
    gen, dec_logits = [], []
    for _ in range(c["n_decode"]):
        gen.append(nxt)
        o = model(input_ids=torch.tensor([[nxt]]), past_key_values=past, use_cache=True)
        past = o.past_key_values
        lg = o.logits[0, -1].float().numpy()
        dec_logits.append(lg)
        nxt = int(np.argmax(lg))
    return dict(
        spec=np.array([spec[k] for k in ("hidden_size", "intermediate_size", "num_q_heads",
                                         "num_kv_heads", "head_dim", "num_layers", "vocab_size")],
                      dtype=np.int64),
        seed=np.int64(c["seed"]), norm_jitter=np.float64(c["norm_jitter"]),
        prompt=toks.numpy().astype(np.int64), prompt_logits=prompt_logits.astype(np.float32),
        gen_tokens=np.array(gen, dtype=np.int64), decode_logits=np.stack(dec_logits).astype(np.float32),
    )


def main():
    outdir = os.path.dirname(os.path.abspath(__file__))
    for name, c in CASES.items():
        d = run_case(name, c)
        path = os.path.join(outdir, f"hf_{name}.npz")
        np.savez_compressed(path, **d)
        print(f"wrote {path}: prompt {d['prompt'].shape} logits {d['prompt_logits'].shape} "
              f"gen {d['gen_tokens'].tolist()}")


if __name__ == "__main__":
    main()
