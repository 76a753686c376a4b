"""The reference's Python binding surfaces on the HIP library:
- chat.py's `decode_ldg` / `decode_ldg_with_logits` over caller-owned KV caches;
- generate.py's per-layer `decode_layer` / `lm_head_last`;
- the position setter;
- the LM-head-only (zero-layer) decoder;
- the text generators on seeded random-init weights.

Oracles:
- Op-level results are compared with the CPU oracle layer (`OracleModel.decode_layer`) at the
  layerwise tolerance of test_gpu_decode.py: one bf16 ulp + 2e-5 x max|y|.
- Calls that run the same kernels as the decoder are compared with the decoder's own results
  bit for bit.
"""
import pytest
import torch

from megaqwen_amd.chat_ops import compile_kernel, compile_kernels
from megaqwen_amd.decoder import MegakernelDecoder
from megaqwen_amd.rope import build_rope_tables
from megaqwen_amd.synthetic import make_tokens
from oracle.ref_cpu import rms_norm
from tests.helpers import build_pair, to_cuda, top2_margin

pytestmark = pytest.mark.gpu

VOCAB = 151936


def _bf16_ulp(x):
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


@pytest.fixture(scope="module")
def pair():
    return build_pair(2, VOCAB, 256, seed=4, norm_jitter=0.1)


def test_set_position_replays_a_step(pair):
    dec, _, sp, _ = pair
    dec.reset()
    toks = make_tokens(6, sp["vocab_size"], seed=3).tolist()
    outs = [dec.decode_step_with_logits(t) for t in toks]
    dec.set_position(3)
    assert dec.position() == 3
    tok, lg = dec.decode_step_with_logits(toks[3])
    assert tok == outs[3][0]
    assert torch.equal(lg, outs[3][1])
    assert dec.position() == 4
    with pytest.raises(RuntimeError):
        dec.set_position(257)
    dec.check()


def test_op_decode_layer_matches_oracle_and_decoder(pair):
    """mq_op_decode_layer against the oracle layer and against the decoder's own layer
    outputs."""
    dec, orc, sp, _ = pair
    dec.reset()
    orc.reset()
    toks = make_tokens(5, sp["vocab_size"], seed=8).tolist()
    for pos, t in enumerate(toks):
        _, _, trace = dec.debug_decode_step_layers(t)
        trace = trace.cpu()
        # replay layer 0 and 1 of this step through the op entry point on the decoder's caches
        # (it rewrites row `pos` with the same values)
        x0 = dec.embed_weight[t]
        y0 = dec.op_decode_layer(0, x0, pos)
        y1 = dec.op_decode_layer(1, trace[0].to(torch.bfloat16).cuda(), pos)
        torch.cuda.synchronize()
        for li, (g, x_in) in enumerate(((y0, x0), (y1, trace[0]))):
            g = g.float().cpu()
            orc.k_cache.copy_(dec.k_cache.float().cpu())
            orc.v_cache.copy_(dec.v_cache.float().cpu())
            ref = orc.decode_layer(li, x_in.float().cpu(), pos, write_kv=False)
            bound = _bf16_ulp(ref) + 2e-5 * float(ref.abs().max())
            assert ((g - ref).abs() <= bound).all(), (pos, li)
            dec_out = trace[li]
            same = float((g == dec_out).float().mean())
            print(f"pos {pos} layer {li}: op vs persistent bit-equal fraction {same:.4f}")
            assert ((g - dec_out).abs() <= _bf16_ulp(dec_out) + 1e-6).all()
    dec.check()


def test_chat_decode_ldg_matches_decoder(pair):
    """chat.py's decode_ldg / decode_ldg_with_logits over caller-owned caches: against the CPU
    oracle directly (teacher-forced, north-star 2e-2 on the logits, greedy tokens wherever the
    oracle's top-2 margin exceeds twice the error) and against the decoder bit for bit."""
    from tests import tolerances as T
    dec, orc, sp, w = pair
    g = to_cuda(w)
    L, S = sp["num_layers"], 256
    cos, sin = build_rope_tables(S, 1e6, 128)
    cos, sin = cos.cuda(), sin.cuda()
    k = compile_kernel()
    lists = [[g["layer_weights"][11 * l + j] for l in range(L)] for j in range(11)]
    k.init_ldg_layer_weights(*lists)
    k.init_ldg_embed_weight(g["embed_weight"])
    kc = torch.zeros(L, 8, S, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    scratch = [torch.zeros(16, device="cuda") for _ in range(11)]
    dec.reset()
    orc.reset()
    toks = make_tokens(8, sp["vocab_size"], seed=21).tolist()
    for pos, t in enumerate(toks):
        args = (t, g["final_norm_weight"], g["lm_head_weight"], cos, sin, kc, vc, *scratch,
                L, pos, pos + 1, S)
        otok, olg = orc.decode_step(t)
        if pos % 2:
            got, lg = k.decode_ldg_with_logits(*args)
            err = float((lg.cpu() - olg).abs().max())
            assert err <= T.DECODE_LOGITS, (pos, err)
            if top2_margin(olg) > 2 * err + 1e-6:
                assert got == otok, pos
            ref, rlg = dec.decode_step_with_logits(t)
            assert torch.equal(lg, rlg), pos
        else:
            got, ref = k.decode_ldg(*args), dec.decode_step(t)
        assert got == ref, pos
    # the caller's caches hold exactly what the decoder's own caches hold
    assert torch.equal(kc[:, :, :8], dec.k_cache[:, :, :8])
    assert torch.equal(vc[:, :, :8], dec.v_cache[:, :, :8])
    with pytest.raises(ValueError):
        k.decode_ldg(toks[0], g["final_norm_weight"], g["lm_head_weight"], cos, sin, kc, vc,
                     *scratch, L, 3, 5, S)


def test_generate_py_layer_api_matches_decoder(pair):
    dec, _, sp, w = pair
    g = to_cuda(w)
    S = 256
    cos, sin = build_rope_tables(S, 1e6, 128)
    cos, sin = cos.cuda(), sin.cuda()
    k = compile_kernels()
    caches = [(torch.zeros(8, S, 128, dtype=torch.bfloat16, device="cuda"),
               torch.zeros(8, S, 128, dtype=torch.bfloat16, device="cuda"))
              for _ in range(sp["num_layers"])]
    dec.reset()
    toks = make_tokens(4, sp["vocab_size"], seed=5).tolist()
    for pos, t in enumerate(toks):
        h = g["embed_weight"][t]
        for li in range(sp["num_layers"]):
            ws = g["layer_weights"][11 * li:11 * (li + 1)]
            h = k.decode_layer(h, *ws, cos, sin, caches[li][0], caches[li][1], pos, pos + 1, S)
        logits = k.lm_head_last(h.view(1, -1), g["final_norm_weight"], g["lm_head_weight"])
        tok, rlg = dec.decode_step_with_logits(t)
        assert logits.dtype == torch.bfloat16 and logits.shape == (VOCAB,)
        err = float((logits.float() - rlg).abs().max())
        assert err <= 1.5e-2, (pos, err)     # bf16 output rounding of the logits (|x| < 4)
        # Layer 0 sees the same input in both paths, so its rows are bit-equal. Deeper layers
        # see the op path's hidden state, which can differ from the fused kernel's by a bf16
        # ulp in a few elements: attention is normalised in a separate merge kernel there.
        # Every K/V element sums over all 1024 inputs, so such flips move many rows across a
        # rounding boundary (about 13% of elements measured at layer 1). The check is one ulp,
        # plus the head's largest ulp for K through RoPE.
        assert torch.equal(caches[0][0][:, pos], dec.k_cache[0, :, pos]), pos
        assert torch.equal(caches[0][1][:, pos], dec.v_cache[0, :, pos]), pos
        for li in range(1, sp["num_layers"]):
            for got, ref in ((caches[li][0][:, pos], dec.k_cache[li, :, pos]),
                             (caches[li][1][:, pos], dec.v_cache[li, :, pos])):
                got, ref = got.float(), ref.float()
                bound = _bf16_ulp(ref) + _bf16_ulp(ref.abs().amax(dim=-1, keepdim=True))
                assert ((got - ref).abs() <= bound).all(), (pos, li)
                assert float((got == ref).float().mean()) > 0.5, (pos, li)


def test_zero_layer_decoder_is_lm_head_of_embedding(pair):
    _, orc, sp, w = pair
    g = to_cuda(w)
    cos, sin = build_rope_tables(8, 1e6, 128)
    d0 = MegakernelDecoder(g["embed_weight"], [], g["final_norm_weight"], g["lm_head_weight"],
                           cos.cuda(), sin.cuda(), 0, 8)
    for t in make_tokens(3, sp["vocab_size"], seed=9).tolist():
        tok, lg = d0.decode_step_with_logits(t)
        ref = orc.lm_head_logits(w["embed_weight"][t].float())
        assert float((lg.cpu() - ref).abs().max()) < 1e-4
        assert tok == int(torch.argmax(lg))
    d0.check()


def test_op_lm_head_matches_rmsnorm_oracle(pair):
    dec, _, _, w = pair
    x = torch.randn(1024, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    logits = torch.empty(VOCAB, device="cuda")
    dec.op_lm_head(x.cuda(), logits=logits)
    ref = w["embed_weight"].float() @ rms_norm(x.float(), w["final_norm_weight"].float())
    assert float((logits.cpu() - ref).abs().max()) < 1e-4


def test_quality_harness_against_oracle(pair):
    """quality_metrics.py's megakernel flow on the HIP decoder: KL(P_oracle || P_decoder) of the
    last-position logits and argmax agreement over five prompts (the reference records KL 6e-4
    and 100% argmax against HuggingFace, experiments/RESULTS.md:66)."""
    from megaqwen_amd.quality import evaluate
    dec, orc, sp, _ = pair
    prompts = [make_tokens(k, sp["vocab_size"], seed=60 + k).tolist() for k in (3, 5, 8, 13, 21)]
    refs = []
    for ids in prompts:
        orc.reset()
        for t in ids[:-1]:
            orc.decode_step(t)
        refs.append(orc.decode_step(ids[-1])[1])
    r = evaluate("hip", dec, prompts, refs)
    print(f"quality: KL {r.kl_div:.3e}, argmax {r.argmax_match:.0%}")
    # argmax must agree wherever the oracle's top-2 margin exceeds twice the 2e-2 logit bound
    safe = sum(top2_margin(lg) > 4e-2 for lg in refs)
    assert r.kl_div < 1e-4 and r.argmax_match >= safe / len(prompts)


@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_generators_random_init(kind):
    """MegakernelGenerator / MegakernelPrefillGenerator on 'random' (seeded Qwen3-0.6B)
    weights: the generated ids equal the decoder driven by hand, and the text decodes."""
    from megaqwen_amd.generators import MegakernelGenerator, MegakernelPrefillGenerator
    if kind == "decode":
        gen = MegakernelGenerator("random", max_seq_len=64)
    else:
        gen = MegakernelPrefillGenerator("random", max_seq_len=64, max_prefill_len=32)
    prompt = "The capital of France is"
    ids = gen.tokenizer.encode(prompt)
    stream = list(gen.generate_stream(prompt, max_new_tokens=6))
    text = gen.generate(prompt, max_new_tokens=6)
    assert "".join(stream) == text
    d = gen.decoder
    d.reset()
    if kind == "decode":
        for t in ids[:-1]:
            d.decode_step(t)
        nxt = d.decode_step(ids[-1])
    else:
        nxt = d.prefill_step(torch.tensor(ids, dtype=torch.int32))
    hand = [nxt]
    for _ in range(5):
        hand.append(d.decode_step(hand[-1]))
    assert text == gen.tokenizer.decode(hand, skip_special_tokens=True)
    if kind == "prefill":
        tok, pos = gen.prefill_only(prompt)
        assert tok == hand[0] and pos == len(ids)
        with pytest.raises(ValueError):
            gen.prefill_only("x" * 40)
    d.check()
