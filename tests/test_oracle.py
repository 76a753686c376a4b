"""Pins the CPU oracle (oracle/ref_cpu.py) before it is used to check the HIP path.

* golden: the oracle's pure-fp32 mode reproduces HuggingFace Qwen3ForCausalLM fp32 logits
  (tests/golden/make_golden.py) for a full prompt forward, token-by-token decode and greedy decode.
* closed forms / invariants for each building block, chosen so that a plausible slip (dropped
  norm weight, sign or half-swap in RoPE, wrong GQA mapping, missing scale, wrong silu) fails.
* the bf16 rounding points of the reference (decode: K/V cache and layer-end hidden state;
  prefill: every op) are live: removing them changes the result, and the values they produce are
  bf16-representable.
"""
import math

import numpy as np
import pytest
import torch

from megaqwen_amd.rope import build_rope_tables
from megaqwen_amd.synthetic import make_tokens, make_weights
from oracle.ref_cpu import OracleModel, attend, bf16, rms_norm, rope, silu

SPEC_KEYS = ("hidden_size", "intermediate_size", "num_q_heads", "num_kv_heads", "head_dim",
             "num_layers", "vocab_size")


def load_case(golden_dir, name):
    d = np.load(f"{golden_dir}/hf_{name}.npz")
    spec = dict(zip(SPEC_KEYS, [int(x) for x in d["spec"]]))
    w = make_weights(spec, seed=int(d["seed"]), norm_jitter=float(d["norm_jitter"]))
    return d, spec, w


@pytest.mark.parametrize("name", ["qwen3_layer_2l", "small_shape_3l"])
def test_golden_hf_prefill_and_decode(golden_dir, name):
    d, spec, w = load_case(golden_dir, name)
    cos, sin = build_rope_tables(64, 1e6, spec["head_dim"], dtype=torch.float32)
    m = OracleModel(w, spec, cos, sin, 64, round_bf16=False)
    lg = m.prefill_hidden_all(d["prompt"]).numpy()
    assert np.abs(lg - d["prompt_logits"]).max() < 2e-5
    tok, last = m.prefill(d["prompt"])
    assert tok == int(d["gen_tokens"][0])
    assert np.abs(last.numpy() - d["prompt_logits"][-1]).max() < 2e-5
    m.reset()
    for t in d["prompt"][:-1]:
        m.decode_step(int(t))
    tok, lg = m.decode_step(int(d["prompt"][-1]))
    assert tok == int(d["gen_tokens"][0])
    assert np.abs(lg.numpy() - d["prompt_logits"][-1]).max() < 2e-5
    for i, g in enumerate(d["gen_tokens"]):
        tok, lg = m.decode_step(int(g))
        assert np.abs(lg.numpy() - d["decode_logits"][i]).max() < 2e-5
        if i + 1 < len(d["gen_tokens"]):
            assert tok == int(d["gen_tokens"][i + 1])


def test_golden_detects_planted_mistakes(golden_dir):
    """A wrong GQA mapping or a dropped q-norm weight must break the golden match."""
    d, spec, w = load_case(golden_dir, "qwen3_layer_2l")
    cos, sin = build_rope_tables(64, 1e6, spec["head_dim"], dtype=torch.float32)
    m = OracleModel(w, spec, cos, sin, 64, round_bf16=False)
    for lay in m.layers:
        lay["q_norm"] = torch.ones_like(lay["q_norm"])
    lg = m.prefill_hidden_all(d["prompt"]).numpy()
    assert np.abs(lg - d["prompt_logits"]).max() > 1e-3
    m = OracleModel(w, spec, cos, sin, 64, round_bf16=False)
    # swap KV head order: a wrong qh -> kv mapping
    for lay in m.layers:
        D = spec["head_dim"]
        lay["k"] = lay["k"].view(-1, D, lay["k"].shape[1]).flip(0).reshape(lay["k"].shape)
    lg = m.prefill_hidden_all(d["prompt"]).numpy()
    assert np.abs(lg - d["prompt_logits"]).max() > 1e-3


def test_rms_norm_closed_form():
    x = torch.tensor([3.0, 4.0])
    w = torch.tensor([1.0, 2.0])
    r = 1.0 / math.sqrt((9 + 16) / 2 + 1e-6)
    assert torch.allclose(rms_norm(x, w), torch.tensor([3 * r, 8 * r]))
    g = torch.Generator().manual_seed(1)
    y = torch.randn(1024, generator=g)
    one = torch.ones(1024)
    assert abs(float(rms_norm(y, one).pow(2).mean()) - 1.0) < 1e-5
    assert torch.allclose(rms_norm(7.5 * y, one), rms_norm(y, one), atol=1e-5)


def test_rope_identity_rotation_and_relative_position():
    D = 128
    cos, sin = build_rope_tables(300, 1e6, D, dtype=torch.float32)
    g = torch.Generator().manual_seed(2)
    q, k = torch.randn(D, generator=g), torch.randn(D, generator=g)
    assert torch.equal(rope(q, cos[0], sin[0]), q)
    # norm preserving
    assert abs(float(rope(q, cos[77], sin[77]).norm() - q.norm())) < 1e-4
    # <rope(q,m), rope(k,n)> depends only on m - n
    a = torch.dot(rope(q, cos[50], sin[50]), rope(k, cos[20], sin[20]))
    b = torch.dot(rope(q, cos[130], sin[130]), rope(k, cos[100], sin[100]))
    assert abs(float(a - b)) < 1e-4
    # explicit rotation of the pair (i, i+64) by angle pos * theta^(-2i/D)
    i, pos = 5, 9
    ang = pos * (1e6 ** (-2 * i / D))
    o = rope(q, cos[pos], sin[pos])
    assert abs(float(o[i]) - (float(q[i]) * math.cos(ang) - float(q[i + 64]) * math.sin(ang))) < 1e-5
    assert abs(float(o[i + 64]) - (float(q[i]) * math.sin(ang) + float(q[i + 64]) * math.cos(ang))) < 1e-5


def test_rope_tables_bf16_rounded():
    cos, sin = build_rope_tables(4353, 1e6, 128)
    assert cos.dtype == torch.bfloat16 and cos.shape == (4353, 128)
    assert torch.equal(cos[:, :64], cos[:, 64:])
    ref = torch.cos(torch.tensor(4352.0) * (1e6 ** (-torch.arange(0, 128, 2).float() / 128)))
    assert torch.allclose(cos[4352, :64].float(), ref, atol=4e-3)


def test_attention_closed_forms():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 1, 16, generator=g)
    v = torch.randn(2, 5, 16, generator=g)
    # L = 1 returns V[0]
    assert torch.allclose(attend(q, torch.randn(2, 1, 16, generator=g), v[:, :1], 0.25), v[:, :1])
    # K == 0 gives the mean of V
    assert torch.allclose(attend(q, torch.zeros(2, 5, 16), v, 0.25), v.mean(dim=1, keepdim=True), atol=1e-6)
    # brute force
    k = torch.randn(2, 5, 16, generator=g)
    s = (q * k).sum(-1) * 0.25
    p = torch.exp(s - s.max(-1, keepdim=True).values)
    p = p / p.sum(-1, keepdim=True)
    assert torch.allclose(attend(q, k, v, 0.25)[:, 0], (p.unsqueeze(-1) * v).sum(1), atol=1e-6)


def test_silu_closed_form():
    assert float(silu(torch.tensor(0.0))) == 0.0
    x = torch.linspace(-6, 6, 25)
    assert torch.allclose(silu(x), x * torch.sigmoid(x), atol=1e-6)


def test_bf16_rounding_is_round_to_nearest_even():
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: RNE picks the even mantissa (1.0)
    assert float(bf16(torch.tensor(1.0 + 2 ** -8))) == 1.0
    assert float(bf16(torch.tensor(1.0 + 3 * 2 ** -8))) == 1.0 + 2 ** -6


def _tiny_model(round_bf16=True, layers=2, vocab=512, seed=7):
    spec = dict(hidden_size=1024, intermediate_size=3072, num_q_heads=16, num_kv_heads=8,
                head_dim=128, num_layers=layers, vocab_size=vocab)
    w = make_weights(spec, seed=seed, norm_jitter=0.1)
    cos, sin = build_rope_tables(64, 1e6, 128)
    return OracleModel(w, spec, cos, sin, 64, round_bf16=round_bf16), spec


def test_decode_rounding_points_live_and_bf16_valued():
    m, spec = _tiny_model()
    toks = make_tokens(6, spec["vocab_size"], seed=1)
    outs = [m.decode_step(int(t)) for t in toks]
    # cache rows hold bf16-representable values
    kc = m.k_cache[:, :, :6]
    assert torch.equal(kc, bf16(kc)) and kc.abs().sum() > 0
    f, _ = _tiny_model(round_bf16=False)
    outs_f = [f.decode_step(int(t)) for t in toks]
    diffs = [float((a[1] - b[1]).abs().max()) for a, b in zip(outs, outs_f)]
    assert max(diffs) > 1e-5           # the rounding points change the numbers ...
    assert max(diffs) < 2e-2           # ... by bf16-noise amounts only


def test_prefill_and_decode_agree_to_bf16_noise():
    """Prefill (bf16 after every op) and token-by-token decode (fp32 intermediates) differ only by
    rounding (the reason the reference has test_compare.py)."""
    m, spec = _tiny_model()
    toks = make_tokens(10, spec["vocab_size"], seed=2)
    _, lp = m.prefill(toks)
    kp = m.k_cache.clone()
    m.reset()
    for t in toks[:-1]:
        m.decode_step(int(t))
    _, ld = m.decode_step(int(toks[-1]))
    assert float((lp - ld).abs().max()) < 5e-2
    assert float((kp[:, :, :10] - m.k_cache[:, :, :10]).abs().max()) < 5e-2
    assert m.position == 10


def test_prefill_fused_is_the_pure_fp32_prefill_with_bf16_cache_rows():
    """The prefill megakernel's arithmetic (prefill_fused) is the pure-fp32 model, which the
    HuggingFace fixtures pin (round_bf16=False, test_golden_hf_prefill_and_decode): identical
    logits, and cache rows that are exactly the bf16 rounding of that model's fp32 K/V rows.
    It ignores the model's own rounding mode (the megakernel has no rounding points); a mistake
    in the fused branch (a rounding left in, the cache rows unrounded) fails here."""
    f, spec = _tiny_model(round_bf16=False)
    r, _ = _tiny_model(round_bf16=True)
    toks = make_tokens(13, spec["vocab_size"], seed=8)
    _, lf = f.prefill(toks)
    kf, vf = f.k_cache.clone(), f.v_cache.clone()
    for m in (f, r):
        m.reset()
        _, lg = m.prefill_fused(toks)
        assert torch.equal(lg, lf)
        assert torch.equal(m.k_cache[:, :, :13], bf16(kf[:, :, :13]))
        assert torch.equal(m.v_cache[:, :, :13], bf16(vf[:, :, :13]))
        assert not torch.equal(m.k_cache[:, :, :13], kf[:, :, :13])
        assert m.position == 13
    # the embedding patch acts as in prefill
    audio = bf16(torch.randn(3, 1024, generator=torch.Generator().manual_seed(5)))
    f.reset()
    _, lp = f.prefill(toks, embeds=audio, embeds_start=4)
    f.reset()
    _, lq = f.prefill_fused(toks, embeds=audio, embeds_start=4)
    assert torch.equal(lp, lq)
    with pytest.raises(RuntimeError):
        f.prefill_fused([])


def test_prefill_errors_and_position():
    m, spec = _tiny_model(layers=1)
    with pytest.raises(RuntimeError):
        m.prefill([])
    with pytest.raises(RuntimeError):
        m.prefill(list(range(65)))
    m.prefill([1, 2, 3])
    assert m.position == 3
    m.reset()
    assert m.position == 0 and float(m.k_cache.abs().sum()) == 0.0


def test_prefill_embedding_patch_pins():
    """The prefill_asr embedding patch (bindings_prefill.cpp:835-955): patching a span with the
    token embeddings it replaces is the identity; a different span changes the logits but, by
    causality, leaves every K/V row before the span bit-identical in every layer."""
    m, spec = _tiny_model()
    toks = make_tokens(12, spec["vocab_size"], seed=4)
    _, l0 = m.prefill(toks)
    k0, v0 = m.k_cache.clone(), m.v_cache.clone()
    _, l1 = m.prefill(toks, embeds=m.embed[toks[5:9]], embeds_start=5)
    assert torch.equal(l0, l1) and torch.equal(k0, m.k_cache)
    audio = bf16(torch.randn(4, m.embed.shape[1], generator=torch.Generator().manual_seed(3)))
    _, l2 = m.prefill(toks, embeds=audio, embeds_start=5)
    assert float((l2 - l0).abs().max()) > 1e-3
    assert torch.equal(k0[:, :, :5], m.k_cache[:, :, :5])
    assert torch.equal(v0[:, :, :5], m.v_cache[:, :, :5])
    assert not torch.equal(k0[:, :, 5:12], m.k_cache[:, :, 5:12])
    with pytest.raises(RuntimeError):
        m.prefill(toks, embeds=audio, embeds_start=9)


def test_synthetic_weights_are_seeded_and_canonical():
    spec = dict(hidden_size=64, intermediate_size=96, num_q_heads=4, num_kv_heads=2, head_dim=16,
                num_layers=2, vocab_size=50)
    a = make_weights(spec, seed=0)
    b = make_weights(spec, seed=0)
    c = make_weights(spec, seed=1)
    assert torch.equal(a["embed_weight"], b["embed_weight"])
    assert not torch.equal(a["embed_weight"], c["embed_weight"])
    assert len(a["layer_weights"]) == 22
    assert a["lm_head_weight"] is a["embed_weight"]
    assert a["layer_weights"][1].shape == (64, 64) and a["layer_weights"][10].shape == (64, 96)
    assert float(a["layer_weights"][0].float().mean()) == 1.0
    std = float(a["embed_weight"].float().std())
    assert 0.015 < std < 0.025
