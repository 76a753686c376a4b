"""The allocation-free attention entry point (mq_op_attention_noalloc) against the allocating one
(mq_op_attention) through the C ABI: both run the same kernels in the same order, so their
outputs must be bit-identical.  Two calls in a row on the shared static scratch, the second with
a smaller cache length (fewer partials than the first call left behind), and once more with a
length that uses the most chunks."""
import ctypes

import pytest
import torch

from megaqwen_amd.synthetic import make_tokens
from tests.helpers import build_pair

pytestmark = pytest.mark.gpu


def _attention(dec, fn, layer, q, cache_len):
    out = torch.full((16 * 128,), float("nan"), dtype=torch.float32, device="cuda")
    rc = fn(dec._h, layer, q.data_ptr(), cache_len, out.data_ptr(),
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, dec._lib.mq_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu()


def test_noalloc_attention_matches_workspace_attention():
    dec, _, sp, _ = build_pair(2, 4096, 2048, seed=3, norm_jitter=0.1, max_prefill=2048,
                               oracle=False)
    lib = dec._lib
    dec.reset()
    dec.prefill_step(make_tokens(2000, sp["vocab_size"], seed=4))   # fills KV rows 0..1999
    gen = torch.Generator().manual_seed(9)
    for layer, cache_len in ((1, 1999), (0, 37), (1, 1500)):
        q = torch.randn(16 * 128, generator=gen).cuda()
        ref = _attention(dec, lib.mq_op_attention, layer, q, cache_len)
        got = _attention(dec, lib.mq_op_attention_noalloc, layer, q, cache_len)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), (layer, cache_len)
    # sizes are validated before anything runs
    q = torch.zeros(16 * 128, dtype=torch.float32, device="cuda")
    out = torch.empty_like(q)
    assert lib.mq_op_attention_noalloc(dec._h, 0, q.data_ptr(), 2049, out.data_ptr(),
                                       None) != 0
    assert lib.mq_op_attention_noalloc(dec._h, 2, q.data_ptr(), 10, out.data_ptr(), None) != 0
    assert lib.mq_op_attention_noalloc(None, 0, q.data_ptr(), 10, out.data_ptr(), None) != 0
    dec.check()
