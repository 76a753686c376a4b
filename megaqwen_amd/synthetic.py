"""Seeded synthetic weights and tokens for the Qwen3 decode/prefill path.

There is no checkpoint offline, so every benchmark and parity test runs on random-init
weights drawn in ONE canonical order from `torch.Generator().manual_seed(seed)`:

    embed[vocab, hidden]
    per layer: q[Hq*D, H], k[Hkv*D, H], v[Hkv*D, H], o[H, Hq*D], gate[I, H], up[I, H], down[H, I]

each `normal(0, 0.02)` in fp32.  Norm weights (input_ln, post_ln, q_norm, k_norm, final norm)
are 1.0 unless `norm_jitter > 0`, in which case they are `1 + norm_jitter * N(0,1)` drawn
after all matrices (tests use this so a dropped norm-weight multiply cannot pass).
The LM head is tied to the embedding, as Qwen3-0.6B's checkpoint is
(csrc/megakernel/megakernel_weights.py:270-277,478 falls back to embed_tokens).

The returned dict has the layout of the reference's weight loader
(megakernel_weights.py:109-128,469-505): `embed_weight`, flat `layer_weights` (11 per layer,
order input_ln, q, k, v, q_norm, k_norm, o, post_ln, gate, up, down), `final_norm_weight`,
`lm_head_weight`.  Values are bf16-representable fp32 (so fp32 consumers see exactly the
weights a bf16 consumer sees).
"""
from __future__ import annotations

import torch

LAYER_KEYS = ("input_ln", "q", "k", "v", "q_norm", "k_norm", "o", "post_ln", "gate", "up", "down")


def _normal(gen: torch.Generator, shape, std: float) -> torch.Tensor:
    t = torch.empty(shape, dtype=torch.float32)
    t.normal_(0.0, std, generator=gen)
    return t.to(torch.bfloat16)


def make_weights(spec: dict, seed: int = 0, std: float = 0.02, norm_jitter: float = 0.0,
                 dtype: torch.dtype = torch.bfloat16) -> dict:
    """Returns CPU tensors (bf16 by default; `dtype=torch.float32` gives the same values in fp32)."""
    H = int(spec["hidden_size"])
    I = int(spec["intermediate_size"])
    D = int(spec["head_dim"])
    Hq = int(spec["num_q_heads"]) * D
    Hkv = int(spec["num_kv_heads"]) * D
    L = int(spec["num_layers"])
    V = int(spec["vocab_size"])
    gen = torch.Generator().manual_seed(int(seed))
    embed = _normal(gen, (V, H), std)
    mats = []
    for _ in range(L):
        mats.append(dict(
            q=_normal(gen, (Hq, H), std),
            k=_normal(gen, (Hkv, H), std),
            v=_normal(gen, (Hkv, H), std),
            o=_normal(gen, (H, Hq), std),
            gate=_normal(gen, (I, H), std),
            up=_normal(gen, (I, H), std),
            down=_normal(gen, (H, I), std),
        ))

    def norm(n: int) -> torch.Tensor:
        if norm_jitter > 0.0:
            t = torch.empty(n, dtype=torch.float32)
            t.normal_(0.0, 1.0, generator=gen)
            return (1.0 + norm_jitter * t).to(torch.bfloat16)
        return torch.ones(n, dtype=torch.bfloat16)

    layer_weights = []
    for i in range(L):
        m = mats[i]
        layer_weights.extend([norm(H), m["q"], m["k"], m["v"], norm(D), norm(D), m["o"], norm(H),
                              m["gate"], m["up"], m["down"]])
    final_norm = norm(H)
    out = {
        "embed_weight": embed,
        "layer_weights": layer_weights,
        "final_norm_weight": final_norm,
        "lm_head_weight": embed,
    }
    if dtype != torch.bfloat16:
        conv = {}
        for k, v in out.items():
            conv[k] = [t.to(dtype) for t in v] if isinstance(v, list) else v.to(dtype)
        conv["lm_head_weight"] = conv["embed_weight"]
        out = conv
    return out


def make_tokens(n: int, vocab_size: int, seed: int = 0) -> torch.Tensor:
    """`n` uniform-random token ids in [0, vocab_size) as int32 (BASELINE configs 1/3/4/5)."""
    gen = torch.Generator().manual_seed(int(seed))
    return torch.randint(0, int(vocab_size), (int(n),), generator=gen, dtype=torch.int64).to(torch.int32)


def layer_dict(weights: dict, layer: int) -> dict:
    """Named view of layer `layer` of the flat 11-per-layer list."""
    flat = weights["layer_weights"][layer * 11:(layer + 1) * 11]
    return dict(zip(LAYER_KEYS, flat))
