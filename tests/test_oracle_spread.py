"""The oracle's own fp32-vs-fp64 spread, measured on the CPU for every case where a GPU parity
test holds a logit bound looser than the north-star 2e-2 (tests/tolerances.py).

Both evaluations use the same bf16 weights, tokens, bf16 RoPE tables and bf16 rounding points
(`OracleModel(dtype=torch.float64)` changes only the arithmetic), so their difference is what
fp32 summation order alone does to the result.  Each relaxed GPU bound must be at most twice the
spread measured here (and at least the spread itself), or it must be tightened.
"""
import pytest
import torch

from megaqwen_amd.rope import build_rope_tables
from megaqwen_amd.synthetic import make_tokens, make_weights
from oracle.ref_cpu import OracleModel
from tests import tolerances as T
from tests.helpers import spec

VOCAB = 151936


def _pair(sp, seed, jitter, max_seq, round_bf16=True):
    w = make_weights(sp, seed=seed, norm_jitter=jitter)
    cos, sin = build_rope_tables(max_seq, 1e6, 128)
    m32 = OracleModel(w, sp, cos, sin, max_seq, round_bf16=round_bf16)
    m64 = OracleModel(w, sp, cos, sin, max_seq, round_bf16=round_bf16, dtype=torch.float64)
    return m32, m64


def _check(bound, spread, name):
    print(f"{name}: oracle fp32-vs-fp64 spread {spread:.3e}, GPU bound {bound:.3e}")
    assert spread <= bound <= 2 * spread, (name, spread, bound)


def test_decode_28_layers_spread():
    """The 28-layer free-running decode case of test_gpu_decode.py (seed 0, 8 tokens of seed 0)."""
    m32, m64 = _pair(spec(28, VOCAB), 0, 0.0, 64)
    worst = 0.0
    for t in make_tokens(8, VOCAB, seed=0).tolist():
        a = m32.decode_step(t)[1]
        b = m64.decode_step(t)[1]
        worst = max(worst, float((a.double() - b).abs().max()))
    _check(T.DECODE_28L, worst, "decode 28 layers")
    assert abs(worst - T.DECODE_28L_SPREAD) <= 0.25 * T.DECODE_28L_SPREAD


def test_prefill_2_layers_spread():
    """The 2-layer prefill cases of test_gpu_prefill.py (seed 2, jitter 0.1, tokens of seed n)."""
    m32, m64 = _pair(spec(2, VOCAB), 2, 0.1, 640)
    worst = 0.0
    for n in (1, 7, 64, 100, 512):
        toks = make_tokens(n, VOCAB, seed=n)
        a = m32.prefill(toks)[1]
        b = m64.prefill(toks)[1]
        worst = max(worst, float((a.double() - b).abs().max()))
    _check(T.PREFILL_2L, worst, "prefill 2 layers")
    assert abs(worst - T.PREFILL_2L_SPREAD) <= 0.25 * T.PREFILL_2L_SPREAD


def test_prefill_28_layers_spread():
    """The 28-layer, 512-token prefill case (seed 0 weights, tokens of seed 1)."""
    m32, m64 = _pair(spec(28, VOCAB), 0, 0.0, 520)
    toks = make_tokens(512, VOCAB, seed=1)
    a = m32.prefill(toks)[1]
    b = m64.prefill(toks)[1]
    worst = float((a.double() - b).abs().max())
    _check(T.PREFILL_28L, worst, "prefill 28 layers")
    assert abs(worst - T.PREFILL_28L_SPREAD) <= 0.25 * T.PREFILL_28L_SPREAD


def test_unrounded_oracle_within_north_star_at_2_layers():
    """The reference's rounding points (bf16 KV cache and layer outputs) against the unrounded
    fp32 model (the HF-pinned mode) on the 2-layer decode case of test_gpu_decode.py: the
    rounding itself stays inside the 2e-2 bar, so the GPU can be held to it against either."""
    sp = spec(2, VOCAB)
    w = make_weights(sp, seed=1, norm_jitter=0.1)
    cos, sin = build_rope_tables(512, 1e6, 128)
    mr = OracleModel(w, sp, cos, sin, 512, round_bf16=True)
    mp = OracleModel(w, sp, cos, sin, 512, round_bf16=False)
    worst = 0.0
    for t in make_tokens(80, VOCAB, seed=3).tolist():
        worst = max(worst, float((mr.decode_step(t)[1] - mp.decode_step(t)[1]).abs().max()))
    print(f"rounded vs unrounded fp32 oracle, 2 layers: {worst:.3e}")
    assert worst < T.DECODE_LOGITS


def test_prefill_rounding_points_vs_unrounded_model_2_layers():
    """The multi-kernel prefill's bf16 rounding points (fused_prefill_launch.inl:245-657) against
    the unrounded fp32 model that the HF fixtures pin (tests/test_oracle.py), on the 2-layer
    prefill cases of test_gpu_prefill.py.  The rounded oracle must stay within bf16 noise of the
    pinned model (PREFILL_ROUNDING_2L) with the same argmax, and must differ from it by at least
    PREFILL_ROUNDING_2L_MIN: a rounding point lost from the oracle (and so possibly from the
    kernel it checks) shrinks the distance.  The unrounded fp32 model's own fp32-vs-fp64 spread
    is ~4e-6 here, so the distance is the rounding's alone."""
    sp = spec(2, VOCAB)
    w = make_weights(sp, seed=2, norm_jitter=0.1)
    cos, sin = build_rope_tables(640, 1e6, 128)
    mr = OracleModel(w, sp, cos, sin, 640, round_bf16=True)
    mp = OracleModel(w, sp, cos, sin, 640, round_bf16=False)
    mp64 = OracleModel(w, sp, cos, sin, 640, round_bf16=False, dtype=torch.float64)
    worst = 0.0
    for n in (1, 7, 64, 100, 512):
        toks = make_tokens(n, VOCAB, seed=n)
        a, b, c = mr.prefill(toks)[1], mp.prefill(toks)[1], mp64.prefill(toks)[1]
        d = float((a - b).abs().max())
        print(f"prefill n={n}: rounded vs unrounded {d:.3e}, unrounded fp32 vs fp64 "
              f"{float((b.double() - c).abs().max()):.1e}")
        assert float((b.double() - c).abs().max()) < 1e-4
        assert int(a.argmax()) == int(b.argmax()), n
        worst = max(worst, d)
    assert T.PREFILL_ROUNDING_2L_MIN <= worst <= T.PREFILL_ROUNDING_2L, worst


def test_fused_prefill_bound_separates_reduced_precision():
    """FUSED_PREFILL (the fused prefill's logit bound against its fp32 oracle) is tight enough
    to fail a fused prefill that lost precision: planted in the CPU oracle, activations kept to
    16 significant bits at the RMSNorm outputs (the GPU's three-part bf16 split of an fp32
    activation without its lo part) or rounded to bf16 there move the logits beyond it."""
    import oracle.ref_cpu as R
    sp = spec(2, VOCAB)
    w = make_weights(sp, seed=5, norm_jitter=0.1)
    cos, sin = build_rope_tables(64, 1e6, 128)
    m = OracleModel(w, sp, cos, sin, 64)
    orig = R.rms_norm

    def keep16(x):                      # 16 significant bits: the hi and mid parts only
        mant, ex = torch.frexp(x)
        return torch.ldexp(torch.round(mant * 2 ** 16) / 2 ** 16, ex)

    try:
        for n in (1, 16):
            toks = make_tokens(n, VOCAB, seed=100 + n)
            m.reset()
            ref = m.prefill_fused(toks)[1]
            R.rms_norm = lambda x, w_, eps=R.EPS: keep16(orig(x, w_, eps))
            m.reset()
            d16 = float((m.prefill_fused(toks)[1] - ref).abs().max())
            R.rms_norm = lambda x, w_, eps=R.EPS: R.bf16(orig(x, w_, eps))
            m.reset()
            d8 = float((m.prefill_fused(toks)[1] - ref).abs().max())
            R.rms_norm = orig
            print(f"n={n}: lo part dropped {d16:.2e}, bf16 norms {d8:.2e}")
            assert d16 > T.FUSED_PREFILL and d8 > 100 * T.FUSED_PREFILL, (n, d16, d8)
    finally:
        R.rms_norm = orig


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_dtype_mode_keeps_rounding_points(dtype):
    """The fp64 mode rounds where the fp32 mode does: the K/V cache rows and every layer output
    are bf16 values in both."""
    sp = spec(2, 4096)
    w = make_weights(sp, seed=3, norm_jitter=0.1)
    cos, sin = build_rope_tables(16, 1e6, 128)
    m = OracleModel(w, sp, cos, sin, 16, dtype=dtype)
    x = m.embed[5].clone()
    y = m.decode_layer(0, x, 0)
    assert y.dtype == dtype and m.k_cache.dtype == dtype
    for t in (y, m.k_cache[0, :, 0], m.v_cache[0, :, 0]):
        assert torch.equal(t, t.to(torch.bfloat16).to(dtype))
    with pytest.raises(ValueError):
        OracleModel(w, sp, cos, sin, 16, dtype=torch.float16)
