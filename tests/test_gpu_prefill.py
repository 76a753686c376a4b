"""Prefill parity: MFMA GEMMs, q/k norm + RoPE, causal attention and the last-token LM head
(prefill_step) against the CPU oracle's prefill, which rounds to bf16 after every op as the
reference's launch_prefill_float does (fused_prefill_launch.inl:245-657).

Tolerances: layer-0 KV-cache rows (RMSNorm -> bf16 -> q|k|v GEMM -> bf16, k also through the
q/k norm and RoPE) within one bf16 ulp plus 5e-4 absolute and >= 98% bit-equal.  The absolute
term covers one legitimate rounding flip of the bf16 RMSNorm output: fp32 summation order moves
rstd by ~1e-7, which can flip an element of xn by one bf16 ulp (~8e-3 at |xn| ~ 1-2), moving a
dot product by |w| * ulp ~ 2e-4.  Deeper layers compound such flips through bf16 rounding after
every op, so here they are checked through the last-position logits.  Prefill rounds to bf16
after every op, so its logits carry more rounding noise than decode's: the oracle's own prefill run in
fp32 and in fp64 arithmetic (same bf16 rounding points) differs by 1.69e-2 - 2.03e-2 already at
2 layers (n = 7..512; tests/test_oracle_spread.py), so the prefill logits bound is
T.PREFILL_2L = 4e-2 (twice that spread); decode continuing after prefill is held to the
north-star 2e-2 (teacher-forced).  Deeper prefill layers are checked one by one in
tests/test_gpu_configs.py (config 4).  K rows pass through RoPE, whose
a*c - b*s can cancel: a one-ulp input flip of a large element becomes several ulps of a small
output, so K is bounded by ulp(ref) + ulp(max |k| of the head).
"""
import pytest
import torch

from megaqwen_amd.synthetic import make_tokens
from tests import tolerances as T
from tests.helpers import build_pair, top2_margin

pytestmark = pytest.mark.gpu


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


def _close_bf16(got, ref, floor_abs=5e-4, head_ulp=False):
    bound = _bf16_ulp(ref) + floor_abs
    if head_ulp:
        bound = bound + _bf16_ulp(ref.abs().amax(dim=-1, keepdim=True))
    bad = (got - ref).abs() > bound
    eq = float((got == ref).float().mean())
    if bad.any() or eq <= 0.98:
        idx = bad.nonzero()[:4].tolist()
        print(f"  mismatch: {int(bad.sum())} outside bound, {eq:.4f} bit-equal, "
              f"max |d| {float((got - ref).abs().max()):.3e}, first bad {idx}, "
              f"got {got[bad][:4].tolist()} ref {ref[bad][:4].tolist()}")
    return (not bad.any()) and eq > 0.98


@pytest.fixture(scope="module")
def small():
    return build_pair(2, 151936, 640, seed=2, norm_jitter=0.1, max_prefill=512)


@pytest.mark.parametrize("n", [1, 7, 64, 100, 512])
def test_prefill_matches_oracle(small, n):
    dec, orc, sp, _ = small
    toks = make_tokens(n, sp["vocab_size"], seed=n)
    dec.reset()
    orc.reset()
    tok, lg = dec.prefill_step_with_logits(toks)
    otok, olg = orc.prefill(toks)
    assert dec.position() == n and orc.position == n
    kc = dec.k_cache.float().cpu()
    vc = dec.v_cache.float().cpu()
    assert _close_bf16(vc[0, :, :n], orc.v_cache[0, :, :n]), "v"
    assert _close_bf16(kc[0, :, :n], orc.k_cache[0, :, :n], head_ulp=True), "k"
    err = float((lg.cpu() - olg).abs().max())
    print(f"prefill n={n}: logit error {err:.3e}")
    assert err <= T.PREFILL_2L, err
    if top2_margin(olg) > 2 * err + 1e-6:
        assert tok == otok
    dec.check()


@pytest.mark.parametrize("n", [7, 64, 512])
def test_prefill_vs_unrounded_fp32_model(small, n):
    """The GPU prefill against the unrounded fp32 oracle (the HF-pinned model, no bf16 rounding
    points): the distance is the reference's bf16 rounding (PREFILL_ROUNDING_2L on the CPU
    oracle) plus the GPU's own summation order, within T.PREFILL_VS_FP32_2L, with the same
    greedy token wherever the pinned model's top-2 margin exceeds twice the error."""
    from oracle.ref_cpu import OracleModel
    dec, orc, sp, w = small
    pinned = OracleModel(w, sp, orc.cos, orc.sin, orc.max_seq_len, round_bf16=False)
    toks = make_tokens(n, sp["vocab_size"], seed=n)
    dec.reset()
    tok, lg = dec.prefill_step_with_logits(toks)
    otok, olg = pinned.prefill(toks)
    err = float((lg.cpu() - olg).abs().max())
    print(f"prefill n={n} vs the unrounded fp32 model: logit error {err:.3e}")
    assert err <= T.PREFILL_VS_FP32_2L, err
    if top2_margin(olg) > 2 * err + 1e-6:
        assert tok == otok
    dec.check()


def test_decode_after_prefill(small):
    dec, orc, sp, _ = small
    toks = make_tokens(37, sp["vocab_size"], seed=11)
    dec.reset()
    orc.reset()
    nxt = dec.prefill_step(toks)
    onxt, _ = orc.prefill(toks)
    feed = make_tokens(20, sp["vocab_size"], seed=12).tolist()
    for i, t in enumerate(feed):
        tok, lg = dec.decode_step_with_logits(t)
        otok, olg = orc.decode_step(t)
        err = float((lg.cpu() - olg).abs().max())
        assert err <= T.DECODE_LOGITS, (i, err)
        if top2_margin(olg) > 2 * err + 1e-6:
            assert tok == otok
    assert dec.position() == 57
    dec.check()


def test_prefill_vs_decode_only_next_token(small):
    """test_single.py / test_compare.py of the reference: the prompt fed token by token through
    decode and through prefill give the same next token unless it is a near tie (the two paths
    round differently by design)."""
    dec, orc, sp, _ = small
    for seed in range(3):
        toks = make_tokens(24, sp["vocab_size"], seed=100 + seed).tolist()
        dec.reset()
        for t in toks[:-1]:
            dec.decode_step(t)
        t_dec, lg_dec = dec.decode_step_with_logits(toks[-1])
        dec.reset()
        t_pf, lg_pf = dec.prefill_step_with_logits(toks)
        assert float((lg_dec - lg_pf).abs().max()) < 5e-2
        if top2_margin(lg_dec) > 0.1:
            assert t_dec == t_pf


def _attention_fp32(q, k, v):
    """Causal GQA attention in fp32 on the CPU: q [n, 16, 128], k/v [8, n, 128] -> [n, 16, 128]."""
    n = q.shape[0]
    out = torch.empty(n, 16, 128)
    mask = torch.ones(n, n, dtype=torch.bool).triu(1)
    for qh in range(16):
        s = (q[:, qh] @ k[qh // 2].T) / 128 ** 0.5
        s.masked_fill_(mask, float("-inf"))
        out[:, qh] = torch.softmax(s, dim=-1) @ v[qh // 2]
    return out


@pytest.mark.parametrize("n", [33, 512, 2000])
def test_prefill_attention_kernel_vs_fp32(small, n):
    """The causal attention kernel alone: the last layer's bf16 output against fp32 attention of
    the same bf16 q (rotated, from the q|k|v buffer) and K/V cache rows.  Bound: one bf16 ulp of
    the result (the output rounding) plus 2e-3 x max |v| for the fp32 reductions and the bf16
    hi + lo split of the softmax weights."""
    if n > 512:
        dec, _, sp, _ = build_pair(1, 4096, n + 8, seed=5, norm_jitter=0.1, max_prefill=n,
                                   oracle=False)
    else:
        dec, _, sp, _ = small
    layer = sp["num_layers"] - 1
    dec.reset()
    dec.prefill_step(make_tokens(n, sp["vocab_size"], seed=40 + n))
    torch.cuda.synchronize()
    bufs = dec.debug_prefill_buffers(n)
    q = bufs["qkv"][:, :2048].float().cpu().view(n, 16, 128)
    k = dec.k_cache[layer, :, :n].float().cpu()
    v = dec.v_cache[layer, :, :n].float().cpu()
    got = bufs["att"].float().cpu().view(n, 16, 128)
    ref = _attention_fp32(q, k, v)
    d = (got - ref).abs()
    bound = _bf16_ulp(ref) + 2e-3 * float(v.abs().max())
    print(f"attention n={n}: max |d| {float(d.max()):.3e}, max |d| / ulp "
          f"{float((d / _bf16_ulp(ref)).max()):.2f}, bit-equal to bf16(ref) "
          f"{float((got == ref.to(torch.bfloat16).float()).float().mean()):.4f}")
    assert (d <= bound).all()
    dec.check()


def test_prefill_asr_embedding_patch(small):
    """prefill_asr (bindings_prefill.cpp:835-955): the patched prefill against the oracle's
    patched prefill at the prefill tolerances; patching with the span's own token embeddings
    reproduces prefill_step bit for bit; the K/V rows before the span are bit-identical to a plain
    prefill (causality); the reference's argument errors."""
    dec, orc, sp, _ = small
    n, a, m = 40, 7, 12
    toks = make_tokens(n, sp["vocab_size"], seed=77)
    audio = (torch.randn(m, 1024, generator=torch.Generator().manual_seed(5)) * 0.05).to(torch.bfloat16)
    dec.reset()
    t_plain = dec.prefill_step(toks)
    kp, vp = dec.k_cache.clone(), dec.v_cache.clone()
    dec.reset()
    assert dec.prefill_asr(toks, dec.embed_weight[toks[a:a + m].cuda()], a) == t_plain
    assert torch.equal(dec.k_cache, kp) and torch.equal(dec.v_cache, vp)
    dec.reset()
    orc.reset()
    tok = dec.prefill_asr(toks, audio.cuda(), a)
    otok, olg = orc.prefill(toks, embeds=audio.float(), embeds_start=a)
    assert dec.position() == n
    assert torch.equal(dec.k_cache[:, :, :a], kp[:, :, :a])
    assert torch.equal(dec.v_cache[:, :, :a], vp[:, :, :a])
    kc = dec.k_cache.float().cpu()
    assert _close_bf16(dec.v_cache[0, :, :n].float().cpu(), orc.v_cache[0, :, :n])
    assert _close_bf16(kc[0, :, :n], orc.k_cache[0, :, :n], head_ulp=True)
    dec.reset()
    tok2, lg = dec.prefill_asr(toks, audio.cuda(), a, return_logits=True)
    err = float((lg.cpu() - olg).abs().max())
    print(f"prefill_asr: logit error {err:.3e}")
    assert tok2 == tok and err <= T.PREFILL_2L
    if top2_margin(olg) > 2 * err + 1e-6:
        assert tok == otok
    dec.reset()
    _, glg = dec.prefill_step_with_logits(toks)   # unpatched logits differ from the patched ones
    assert float((glg.cpu() - olg).abs().max()) > 1e-3
    for bad_start, emb in ((n - m + 1, audio.cuda()), (-1, audio.cuda()),
                           (0, audio.cuda()[:0]), (0, audio.float().cuda()), (0, audio)):
        with pytest.raises(RuntimeError):
            dec.prefill_asr(toks, emb, bad_start)
    with pytest.raises(RuntimeError):
        dec.prefill_asr(torch.zeros(513, dtype=torch.int32), audio.cuda(), 0)
    dec.check()


def test_prefill_errors(small):
    dec, _, sp, _ = small
    with pytest.raises(RuntimeError):
        dec.prefill_step(torch.zeros(0, dtype=torch.int32))
    with pytest.raises(RuntimeError):
        dec.prefill_step(torch.zeros(513, dtype=torch.int32))


def test_prefill_28_layers_real_shape():
    """28 layers, 512-token prompt (BASELINE config 4 shape): layer-0 KV rows tightly, the final
    logits within T.PREFILL_28L = 7e-2, twice the oracle's own fp32-vs-fp64 spread of 3.66e-2 on
    this case (tests/test_oracle_spread.py).  Every layer is checked on its own in
    tests/test_gpu_configs.py."""
    dec, orc, sp, _ = build_pair(28, 151936, 520, seed=0, max_prefill=512)
    toks = make_tokens(512, sp["vocab_size"], seed=1)
    tok, lg = dec.prefill_step_with_logits(toks)
    otok, olg = orc.prefill(toks)
    assert _close_bf16(dec.v_cache[0, :, :512].float().cpu(), orc.v_cache[0, :, :512])
    assert _close_bf16(dec.k_cache[0, :, :512].float().cpu(), orc.k_cache[0, :, :512],
                       head_ulp=True)
    err = float((lg.cpu() - olg).abs().max())
    print(f"28-layer prefill logit error {err:.3e}")
    assert err <= T.PREFILL_28L
    dec.check()


def test_prefill_out_of_vocab_id_sets_device_error(small):
    """Token ids stay on the device through the C ABI (mq_prefill), so the embedding gather checks
    them there: an id outside the vocabulary reads row 0 instead of memory past the table and
    sets the error flag that mq_decoder_check reports; reset() clears it."""
    dec = small[0]
    dec.reset()
    d = torch.tensor([5, dec.vocab_size, 7], dtype=torch.int32, device="cuda")
    rc = dec._lib.mq_prefill(dec._h, d.data_ptr(), 3, dec._tok.data_ptr() + 4, None,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    with pytest.raises(RuntimeError):
        dec.check()
    dec.reset()
    dec.check()
