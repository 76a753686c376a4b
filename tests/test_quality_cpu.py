"""The quality harness (experiments/framework_bench/quality_metrics.py:70-238): KL divergence and
perplexity against closed forms and scipy's elementwise relative entropy, and the decoder flow
(prompt through decode, last position with logits) on a host-side stub decoder."""
import math

import numpy as np
import pytest
import torch
from scipy.special import rel_entr

from megaqwen_amd.quality import (QualityResult, decoder_last_logits, evaluate,
                                  format_markdown_table, kl_divergence, perplexity_from_logits)


def test_kl_closed_forms():
    # p = (1/4, 3/4), q = (1/2, 1/2): KL = 1/4 ln(1/2) + 3/4 ln(3/2)
    p = torch.tensor([0.0, math.log(3.0)])
    q = torch.tensor([0.0, 0.0])
    assert kl_divergence(p, q) == pytest.approx(0.25 * math.log(0.5) + 0.75 * math.log(1.5), rel=1e-6)
    assert kl_divergence(q, q) == 0.0
    x = torch.randn(3, 1000, generator=torch.Generator().manual_seed(0))
    assert abs(kl_divergence(x, x + 7.0)) < 1e-6          # softmax is shift invariant


def test_kl_matches_scipy_and_is_asymmetric():
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn(4, 500, generator=g) * 3, torch.randn(4, 500, generator=g) * 3
    pa = torch.softmax(a.double(), -1).numpy()
    pb = torch.softmax(b.double(), -1).numpy()
    ref = float(np.mean(rel_entr(pa, pb).sum(-1)))
    assert kl_divergence(a, b) == pytest.approx(ref, rel=1e-4)
    assert kl_divergence(a, b) > 0
    assert abs(kl_divergence(a, b) - kl_divergence(b, a)) > 1e-3


def test_perplexity_closed_forms():
    ids = torch.tensor([3, 1, 4, 1, 5])
    assert perplexity_from_logits(torch.zeros(5, 10), ids) == pytest.approx(10.0, rel=1e-6)
    sure = torch.full((5, 10), -30.0)
    sure[torch.arange(4), ids[1:]] = 30.0
    assert perplexity_from_logits(sure.unsqueeze(0), ids) == pytest.approx(1.0, abs=1e-6)
    two = torch.tensor([[0.0, math.log(3.0)], [0.0, 0.0]])
    assert perplexity_from_logits(two, torch.tensor([0, 1])) == pytest.approx(4.0 / 3.0, rel=1e-6)


class _StubDecoder:
    """Returns fixed logits for the last token and records the decode calls."""

    def __init__(self, logits):
        self.logits, self.calls = logits, []

    def reset(self):
        self.calls.append("reset")

    def decode_step(self, t):
        self.calls.append(t)
        return 0

    def decode_step_with_logits(self, t):
        self.calls.append(("last", t))
        return int(self.logits.argmax()), self.logits


def test_decoder_flow_and_table():
    ref = torch.randn(50, generator=torch.Generator().manual_seed(2))
    stub = _StubDecoder(ref.clone())
    got = decoder_last_logits(stub, [7, 8, 9])
    assert stub.calls == ["reset", 7, 8, ("last", 9)]
    assert torch.equal(got, ref)
    r = evaluate("stub", _StubDecoder(ref.clone()), [[1, 2], [3]], [ref, ref])
    assert r.kl_div == 0.0 and r.argmax_match == 1.0
    other = ref.clone()
    other[int(ref.argmin())] = 100.0
    r2 = evaluate("stub", _StubDecoder(other), [[1]], [ref])
    assert r2.argmax_match == 0.0 and r2.kl_div > 1.0
    table = format_markdown_table([r, QualityResult("x", False, None, None, None, "no GPU")])
    assert "| stub | 0.000000 | n/a | 100.0% | ok |" in table
    assert "| x | n/a | n/a | n/a | no GPU |" in table
    with pytest.raises(ValueError):
        evaluate("stub", stub, [[1]], [])
