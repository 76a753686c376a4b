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
               max_prefill: int = 0, oracle: bool = True, cls=None):
    """(GPU decoder, CPU oracle or None, spec, cpu weights) on identical bf16 weights and tables.
    `cls`: the decoder class (MegakernelPrefillDecoder by default)."""
    from megaqwen_amd.decoder import MegakernelPrefillDecoder
    from oracle.ref_cpu import OracleModel

    cls = cls or MegakernelPrefillDecoder

    sp = spec(num_layers, vocab)
    w = make_weights(sp, seed=seed, norm_jitter=norm_jitter)
    cos, sin = build_rope_tables(max_seq, 1e6, 128)
    g = to_cuda(w)
    dec = cls(g["embed_weight"], g["layer_weights"], g["final_norm_weight"], g["lm_head_weight"],
              cos.cuda(), sin.cuda(), num_layers, max_seq, max_prefill_len=max_prefill)
    orc = OracleModel(w, sp, cos, sin, max_seq, round_bf16=True) if oracle else None
    return dec, orc, sp, w


def top2_margin(logits: torch.Tensor) -> float:
    v = torch.topk(logits.float(), 2).values
    return float(v[0] - v[1])


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (8 significant bits)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


def oracle_kv_row(orc, li: int, x: torch.Tensor, pos: int):
    """The bf16 K and V rows the oracle's decode layer li writes at `pos` for input x."""
    from oracle.ref_cpu import bf16, rms_norm, rope
    w = orc.layers[li]
    n = rms_norm(x, w["input_ln"])
    k = rope(rms_norm((w["k"] @ n).view(orc.nkv, orc.D), w["k_norm"]), orc.cos[pos], orc.sin[pos])
    v = (w["v"] @ n).view(orc.nkv, orc.D)
    return bf16(k), bf16(v)


def check_decode_step_layerwise(dec, orc, token: int, pos: int, exact_frac: float = 0.99):
    """One GPU decode step at `pos` checked layer by layer against the oracle.

    The oracle takes over the GPU's KV cache (including the row the GPU wrote for `pos`) and, at
    every layer, the GPU's input hidden state, so rounding-order differences cannot compound.
    Bounds: new K/V rows within one bf16 ulp + 2e-5 x max|row| of the oracle's own rows from the
    same input; layer outputs within one bf16 ulp + 2e-5 x max|output|, and at least `exact_frac`
    of all layer-output elements bit-equal; logits of the GPU's final hidden state within 1e-4 of
    the GPU's own logits.  Returns (gpu token, gpu logits)."""
    assert dec.position() == pos
    tok, lg, trace = dec.debug_decode_step_layers(token)
    trace = trace.cpu()
    kc = dec.k_cache.float().cpu()
    vc = dec.v_cache.float().cpu()
    orc.k_cache = kc
    orc.v_cache = vc
    x = orc.embed[token].clone()
    exact = 0
    L = orc.L
    for li in range(L):
        own = oracle_kv_row(orc, li, x, pos)
        for got, ref in ((kc[li, :, pos], own[0]), (vc[li, :, pos], own[1])):
            kb = bf16_ulp(ref) + 2e-5 * ref.abs().amax(dim=-1, keepdim=True)
            assert ((got - ref).abs() <= kb).all(), ("kv row", pos, li)
        y = orc.decode_layer(li, x, pos, write_kv=False)
        g = trace[li]
        bound = bf16_ulp(y) + 2e-5 * float(y.abs().max())
        bad = (g - y).abs() > bound
        assert not bad.any(), ("layer", pos, li, g[bad][:4].tolist(), y[bad][:4].tolist())
        exact += int((g == y).sum())
        x = g
    assert exact >= exact_frac * L * trace.shape[1], (pos, exact)
    ref = orc.lm_head_logits(trace[-1])
    assert float((lg.cpu() - ref).abs().max()) < 1e-4, pos
    assert tok == int(torch.argmax(lg))
    return tok, lg
