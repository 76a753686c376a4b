"""The fused short-prompt prefill (`mq_prefill_fused`, MegakernelFusedPrefillDecoder for prompts
of up to 64 tokens) against the oracle's restatement of the reference's prefill megakernel
(`OracleModel.prefill_fused`: fp32 activations, bf16 weights, only the K/V cache rows rounded to
bf16; fused_prefill_megakernel_core.inl:658-745).

The GPU forms every product exactly (fp32 activations split into three bf16 parts on MFMA) and
differs from the oracle only in the order of fp32 sums, in applying the RMSNorm scale after
the dot product and in the two tag bits of each activation handed between workgroups (a
truncation below 2^-22), so the prefill logits are held to T.FUSED_PREFILL (2e-5; measured
2.7e-6 .. 4.7e-6 at 2 layers, 8.5e-6 at 28), which a bf16 activation anywhere, or the split
without its lo part, would exceed
(tests/test_oracle_spread.py plants both in the oracle).  Decode steps that follow the prefill
run the decode kernel and are held to the north-star 2e-2.  K/V cache rows are bf16 roundings
of fp32 values that agree to ~1e-6, so a few round the other way: within one bf16 ulp (K: plus
the head's ulp, RoPE can cancel) and >= 98% bit-equal.
"""
import ctypes

import pytest
import torch

from megaqwen_amd import _lib
from megaqwen_amd.decoder import MegakernelFusedPrefillDecoder
from megaqwen_amd.synthetic import make_tokens
from tests import tolerances as T
from tests.helpers import build_pair, top2_margin
from tests.test_gpu_prefill import _close_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small():
    return build_pair(2, 151936, 256, seed=5, norm_jitter=0.1, max_prefill=64,
                      cls=MegakernelFusedPrefillDecoder)


def _check_prefill(dec, orc, n, seed, **kw):
    toks = make_tokens(n, dec.vocab_size, seed=seed)
    dec.reset()
    orc.reset()
    emb = kw.get("embeds")
    if emb is not None:
        tok, lg = dec.prefill_asr(toks, emb.cuda(), kw["start"], return_logits=True)
        otok, olg = orc.prefill_fused(toks, embeds=emb.float(), embeds_start=kw["start"])
    else:
        tok, lg = dec.prefill_step_with_logits(toks)
        otok, olg = orc.prefill_fused(toks)
    assert dec.position() == n and orc.position == n
    kc = dec.k_cache.float().cpu()
    vc = dec.v_cache.float().cpu()
    for li in range(dec.num_layers):
        assert _close_bf16(vc[li, :, :n], orc.v_cache[li, :, :n]), f"v layer {li}"
        assert _close_bf16(kc[li, :, :n], orc.k_cache[li, :, :n], head_ulp=True), f"k layer {li}"
    err = float((lg.cpu() - olg).abs().max())
    print(f"fused prefill n={n}: logit error {err:.3e} (max |logit| {float(olg.abs().max()):.2f})")
    assert err <= T.FUSED_PREFILL, err
    if top2_margin(olg) > 2 * err + 1e-6:
        assert tok == otok
    dec.check()
    return toks, tok, otok


# lengths at every change of the work split: O / down row groups of 1, 2, 4, 8, 16 rows (n = 1,
# 5, 9, 17, 33), q|k|v and gate|up column tiles per workgroup (n = 16 / 17, 32 / 33, 48 / 49),
# attention query blocks of 4 (n = 3, 4, 5), and the longest prompt
@pytest.mark.parametrize("n", [1, 3, 4, 5, 7, 9, 16, 17, 32, 33, 48, 49, 64])
def test_fused_prefill_matches_oracle(small, n):
    dec, orc, _, _ = small
    _check_prefill(dec, orc, n, seed=100 + n)


def test_fused_prefill_then_decode(small):
    """Decode continues from the fused prefill's bf16 cache rows (teacher-forced, 2e-2)."""
    dec, orc, _, _ = small
    _, tok, otok = _check_prefill(dec, orc, 20, seed=7)
    t = otok
    for _ in range(6):
        g, lg = dec.decode_step_with_logits(t)
        o, olg = orc.decode_step(t)
        err = float((lg.cpu() - olg).abs().max())
        assert err <= T.DECODE_LOGITS, err
        t = o
    dec.check()


def test_fused_prefill_asr_rows(small):
    dec, orc, _, _ = small
    g = torch.Generator().manual_seed(3)
    emb = (torch.randn(10, 1024, generator=g) * 0.05).to(torch.bfloat16)
    _check_prefill(dec, orc, 24, seed=9, embeds=emb, start=5)


def test_fused_prefill_deterministic(small):
    dec, _, _, _ = small
    toks = make_tokens(40, dec.vocab_size, seed=4)
    out = []
    for _ in range(2):
        dec.reset()
        tok, lg = dec.prefill_step_with_logits(toks)
        out.append((tok, lg, dec.k_cache.clone(), dec.v_cache.clone()))
    assert out[0][0] == out[1][0]
    assert torch.equal(out[0][1], out[1][1])
    assert torch.equal(out[0][2], out[1][2]) and torch.equal(out[0][3], out[1][3])


def test_fused_prefill_tags_across_launches(small):
    """The fused prefill hands activations between workgroups as words tagged with the launch's
    tag (1..3), which the host picks so that no row the launch reads still holds it from an
    earlier launch; when rows hold all three tags, the buffers are cleared first.  Prompts of 64,
    32 and 16 tokens leave all three tags in rows 0..63, so the next 64-token prompt takes the
    clearing path; the others reuse rows last written one, two or more launches back.  With no
    reset in between, every launch must give exactly the result of the same prompt after a reset
    (token, logits and its K/V cache rows, bit for bit: the tag bits are removed before use)."""
    dec, _, _, _ = small
    lens = [64, 32, 16, 64, 7, 64, 1, 48, 33, 33, 16, 64]
    prompts = {n: make_tokens(n, dec.vocab_size, seed=100 + n) for n in set(lens)}
    ref = {}
    for n, toks in prompts.items():
        dec.reset()
        tok, lg = dec.prefill_step_with_logits(toks)
        ref[n] = (tok, lg.clone(), dec.k_cache[:, :, :n].clone(), dec.v_cache[:, :, :n].clone())
    dec.reset()
    for i, n in enumerate(lens):
        tok, lg = dec.prefill_step_with_logits(prompts[n])
        rtok, rlg, rk, rv = ref[n]
        assert tok == rtok, (i, n)
        assert torch.equal(lg, rlg), (i, n)
        assert torch.equal(dec.k_cache[:, :, :n], rk) and torch.equal(dec.v_cache[:, :, :n], rv), (i, n)
        assert dec.position() == n
    dec.check()


def test_fused_prefill_errors(small):
    dec, _, _, _ = small
    with pytest.raises(RuntimeError, match="Empty input sequence"):
        dec.prefill_step([])
    with pytest.raises(RuntimeError, match="exceeds maximum"):
        dec.prefill_step(list(range(65)))
    with pytest.raises(ValueError):
        dec.prefill_step([dec.vocab_size])
    lib = _lib.load()
    d = torch.zeros(8, dtype=torch.int32, device="cuda")
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    # embeddings length without embeddings, and a length above the fused limit
    assert lib.mq_prefill_fused(dec._h, d.data_ptr(), 8, None, 0, 3, out.data_ptr(), None,
                                None) != 0
    assert b"embeds_len" in lib.mq_last_error()
    big = torch.zeros(65, dtype=torch.int32, device="cuda")
    assert lib.mq_prefill_fused(dec._h, big.data_ptr(), 65, None, 0, 0, out.data_ptr(), None,
                                None) != 0
    # an id outside the vocabulary on the device reads row 0 and sets the device error flag
    bad = torch.tensor([1, 2, dec.vocab_size + 5], dtype=torch.int32, device="cuda")
    dec.reset()
    assert lib.mq_prefill_fused(dec._h, bad.data_ptr(), 3, None, 0, 0, out.data_ptr(), None,
                                None) == 0
    with pytest.raises(RuntimeError):
        dec.check()
    dec.reset()


def test_fused_prefill_28_layers_real_shape():
    dec, orc, _, _ = build_pair(28, 151936, 128, seed=11, max_prefill=64,
                                cls=MegakernelFusedPrefillDecoder)
    toks, tok, otok = _check_prefill(dec, orc, 16, seed=12)
    del dec, orc
    torch.cuda.empty_cache()


def test_fused_class_long_prompt_runs_multikernel_prefill():
    """max_prefill_len above 64: a longer prompt runs the bf16 multi-kernel prefill."""
    dec, orc, _, _ = build_pair(2, 151936, 256, seed=6, max_prefill=128,
                                cls=MegakernelFusedPrefillDecoder)
    toks = make_tokens(100, dec.vocab_size, seed=1)
    tok, lg = dec.prefill_step_with_logits(toks)
    otok, olg = orc.prefill(toks)
    err = float((lg.cpu() - olg).abs().max())
    assert err <= T.PREFILL_2L, err
    dec.check()


def test_fused_prefill_then_both_decode_modes(small):
    """The fused prefill leaves the decoder ready for either decode mode: after the same fused
    prefill, 5 steps of the one-kernel-per-phase mode equal the persistent kernel's bit for bit."""
    dec, _, _, _ = small
    toks = make_tokens(30, dec.vocab_size, seed=21)
    runs = []
    for mode in ("persistent", "multi_kernel"):
        dec.set_mode(mode)
        dec.reset()
        t = dec.prefill_step(toks)
        lgs = []
        for _ in range(5):
            t, lg = dec.decode_step_with_logits(t)
            lgs.append(lg)
        runs.append(torch.stack(lgs))
        dec.check()
    dec.set_mode("persistent")
    assert torch.equal(runs[0], runs[1])
