"""Greedy decode of this library against HuggingFace `Qwen3ForCausalLM` on the same weights: the
counterpart of the reference's `verify_correctness.py` (:8-63).

    python -m megaqwen_amd.verify_correctness --model /path/to/Qwen3-0.6B
    python -m megaqwen_amd.verify_correctness --model random:0        # seeded random init

The reference loads "Qwen/Qwen3-0.6B" from the hub, generates 20 tokens with HF (bf16, on the
GPU) and with `MegakernelGenerator`, and compares the first generated word (:38-60).  Here:
- `--model` is a local checkpoint directory (`config.json` + safetensors, as
  `megaqwen_amd.weights.load_qwen3_weights` reads it) or `random[:seed]`; nothing is downloaded;
- the HF model runs on the CPU in float32 from the same bf16 weights (a directory is read by
  `AutoModelForCausalLM.from_pretrained`, random init is loaded into a `Qwen3Config` model), so
  it is the unrounded fp32 model this library's bf16 path approximates;
- both decode greedily token by token on the same prompt, and the comparison is by token id at
  every step, with HF's top-2 logit margin and the largest logit difference of each step;
- the verdict is the reference's: PASS when the first generated token matches.  A mismatch
  where HF's top-2 margin is below twice the largest logit difference seen is reported as a
  near tie (also PASS).  The exit status is 0 on PASS and 1 otherwise.

Without tokenizer files (random init, or a directory without them) the prompt is encoded with
the byte-level `SyntheticTokenizer` of `megaqwen_amd.weights`.
"""
from __future__ import annotations

import argparse
import sys

import torch


def _hf_from_dir(model_dir: str):
    from transformers import AutoModelForCausalLM
    model = AutoModelForCausalLM.from_pretrained(model_dir, local_files_only=True,
                                                 dtype=torch.float32,
                                                 attn_implementation="eager")
    return model.eval()


def _hf_from_weights(weights: dict, spec: dict, rope_theta: float):
    """`Qwen3ForCausalLM` (float32, CPU) holding the given flat weight list."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(
        vocab_size=spec["vocab_size"], hidden_size=spec["hidden_size"],
        intermediate_size=spec["intermediate_size"], num_hidden_layers=spec["num_layers"],
        num_attention_heads=spec["num_q_heads"], num_key_value_heads=spec["num_kv_heads"],
        head_dim=spec["head_dim"], rms_norm_eps=1e-6, max_position_embeddings=40960,
        rope_parameters={"rope_type": "default", "rope_theta": rope_theta},
        tie_word_embeddings=True, attention_bias=False, use_sliding_window=False,
        attn_implementation="eager", dtype=torch.float32)
    model = Qwen3ForCausalLM(cfg).to(torch.float32).eval()
    names = ["input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
             "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj",
             "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    f = lambda t: t.detach().to("cpu", torch.float32)
    sd = {"model.embed_tokens.weight": f(weights["embed_weight"]),
          "model.norm.weight": f(weights["final_norm_weight"]),
          "lm_head.weight": f(weights["lm_head_weight"])}
    lw = weights["layer_weights"]
    for i in range(spec["num_layers"]):
        for j, n in enumerate(names):
            sd[f"model.layers.{i}.{n}.weight"] = f(lw[11 * i + j])
    model.load_state_dict(sd, strict=True)
    return model


@torch.no_grad()
def _hf_greedy(model, ids: list[int], n: int):
    """Greedy tokens and the logits that chose each of them (incremental decode with a cache)."""
    out = model(input_ids=torch.tensor([ids]), use_cache=True)
    past, logits = out.past_key_values, out.logits[0, -1]
    toks, lgs = [], []
    for _ in range(n):
        t = int(torch.argmax(logits))
        toks.append(t)
        lgs.append(logits.clone())
        out = model(input_ids=torch.tensor([[t]]), past_key_values=past, use_cache=True)
        past, logits = out.past_key_values, out.logits[0, -1]
    return toks, lgs


def verify(model: str = "Qwen/Qwen3-0.6B", prompt: str = "The capital of France is",
           max_new_tokens: int = 20, max_seq_len: int = 512) -> dict:
    """Runs the comparison; returns a dict with both token lists, per-step margins and logit
    differences, the first divergence (or None) and `passed`."""
    from . import spec as _spec
    from .generators import MegakernelGenerator
    from .weights import SyntheticTokenizer, load_qwen3_weights, resolve_local_model_dir

    gen = MegakernelGenerator(model, max_seq_len=max_seq_len)
    spec = _spec.get_active_model_spec()
    tok = gen.tokenizer if gen.tokenizer is not None else SyntheticTokenizer()
    ids = list(tok.encode(prompt, add_special_tokens=True))
    if not ids or max(ids) >= spec["vocab_size"]:
        raise ValueError("the prompt does not encode to token ids of this model's vocabulary")
    if len(ids) + max_new_tokens >= max_seq_len:
        raise ValueError("prompt + max_new_tokens does not fit max_seq_len")

    name = str(model)
    if name == "random" or name.startswith("random:"):
        weights = load_qwen3_weights(name, max_seq_len=max_seq_len)
        hf = _hf_from_weights(weights, spec, _spec.ROPE_THETA)
        del weights
    else:
        hf = _hf_from_dir(str(resolve_local_model_dir(name)))
    hf_toks, hf_logits = _hf_greedy(hf, ids, max_new_tokens)

    dec = gen.decoder
    dec.reset()
    for t in ids[:-1]:
        dec.decode_step(t)
    cur, mk_toks, diffs, margins = ids[-1], [], [], []
    for i in range(max_new_tokens):
        t, lg = dec.decode_step_with_logits(cur)
        mk_toks.append(int(t))
        ref = hf_logits[i]
        diffs.append(float((lg.float().cpu() - ref).abs().max()))
        top = torch.topk(ref, 2).values
        margins.append(float(top[0] - top[1]))
        cur = int(t)
        if hf_toks[i] != mk_toks[i]:
            break       # later steps would compare different prefixes
    first_div = next((i for i, (a, b) in enumerate(zip(hf_toks, mk_toks)) if a != b), None)
    bound = 2.0 * max(diffs)
    near_tie = first_div is not None and margins[first_div] < bound
    passed = hf_toks[0] == mk_toks[0] or (first_div == 0 and near_tie)
    return {"prompt_ids": ids, "hf_tokens": hf_toks, "megakernel_tokens": mk_toks,
            "hf_text": tok.decode(hf_toks), "megakernel_text": tok.decode(mk_toks),
            "max_logit_diff": diffs, "hf_top2_margin": margins, "first_divergence": first_div,
            "near_tie": near_tie, "passed": passed}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", default="Qwen/Qwen3-0.6B",
                    help="local checkpoint directory, or random[:seed] (default: Qwen/Qwen3-0.6B, "
                         "resolved as a local directory)")
    ap.add_argument("--prompt", default="The capital of France is")
    ap.add_argument("--max-new-tokens", type=int, default=20)
    ap.add_argument("--max-seq-len", type=int, default=512)
    args = ap.parse_args(argv)
    r = verify(args.model, args.prompt, args.max_new_tokens, args.max_seq_len)
    print(f"Prompt: {args.prompt!r} ({len(r['prompt_ids'])} tokens)")
    print(f"HuggingFace (fp32, CPU): {r['hf_text']!r}")
    print(f"Megakernel (bf16, GPU):  {r['megakernel_text']!r}")
    n = len(r["megakernel_tokens"])
    for i in range(n):
        mark = "" if r["hf_tokens"][i] == r["megakernel_tokens"][i] else "  <- differs"
        print(f"  step {i:2d}: hf {r['hf_tokens'][i]:6d}  megakernel {r['megakernel_tokens'][i]:6d}"
              f"  hf top-2 margin {r['hf_top2_margin'][i]:.4f}  max |logit diff| "
              f"{r['max_logit_diff'][i]:.4f}{mark}")
    if r["first_divergence"] is None:
        print(f"\n[PASS] all {n} generated tokens match")
    elif r["passed"]:
        what = "near tie" if r["near_tie"] else "first token matches"
        print(f"\n[PASS] {what}; first divergence at step {r['first_divergence']}")
    else:
        print(f"\n[FAIL] first generated token differs (HF margin {r['hf_top2_margin'][0]:.4f})")
    return 0 if r["passed"] else 1


if __name__ == "__main__":
    sys.exit(main())
