"""Shared helpers for the parity tests: seeded models on the GPU and the matching CPU oracle."""
from __future__ import annotations

import torch

from megaqwen_amd.rope import build_rope_tables
from megaqwen_amd.synthetic import make_weights

QWEN3_LAYER = dict(hidden_size=1024, intermediate_size=3072, num_q_heads=16, num_kv_heads=8,
                   head_dim=128)


def spec(num_layers: int, vocab_size: int) -> dict:
    return dict(QWEN3_LAYER, num_layers=num_layers, vocab_size=vocab_size)


def to_cuda(weights: dict) -> dict:
    emb = weights["embed_weight"].cuda()
    out = {
        "embed_weight": emb,
        "layer_weights": [t.cuda() for t in weights["layer_weights"]],
        "final_norm_weight": weights["final_norm_weight"].cuda(),
    }
    out["lm_head_weight"] = emb if weights["lm_head_weight"] is weights["embed_weight"] \
        else weights["lm_head_weight"].cuda()
    return out


def build_pair(num_layers: int, vocab: int, max_seq: int, seed: int = 0, norm_jitter: float = 0.0,
               max_prefill: int = 0, oracle: bool = True):
    """(GPU decoder, CPU oracle or None, spec, cpu weights) on identical bf16 weights and tables."""
    from megaqwen_amd.decoder import MegakernelPrefillDecoder
    from oracle.ref_cpu import OracleModel

    sp = spec(num_layers, vocab)
    w = make_weights(sp, seed=seed, norm_jitter=norm_jitter)
    cos, sin = build_rope_tables(max_seq, 1e6, 128)
    g = to_cuda(w)
    dec = MegakernelPrefillDecoder(g["embed_weight"], g["layer_weights"], g["final_norm_weight"],
                                   g["lm_head_weight"], cos.cuda(), sin.cuda(), num_layers,
                                   max_seq, max_prefill_len=max_prefill)
    orc = OracleModel(w, sp, cos, sin, max_seq, round_bf16=True) if oracle else None
    return dec, orc, sp, w


def top2_margin(logits: torch.Tensor) -> float:
    v = torch.topk(logits.float(), 2).values
    return float(v[0] - v[1])
