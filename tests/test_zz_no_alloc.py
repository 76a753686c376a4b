"""The allocation-free attention entry point (mq_op_attention_noalloc) against the allocating one
(mq_op_attention) through the C ABI: both run the same kernels in the same order, so their
outputs must be bit-identical.  Calls in a row share the static scratch: first a cache length
whose split fills every partial slot the grid can use (8192 positions: ceil(8192 / 224) chunks,
capped at grid / 8 = 32 per kv head on a 256-CU MI355X), then a much smaller one (fewer partials
than the first call left behind), then two more full splits (7500 and 6945 positions) and a
single-chunk length."""
import pytest
import torch

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
    max_seq = 8192
    dec, _, sp, _ = build_pair(2, 4096, max_seq, seed=3, norm_jitter=0.1, oracle=False)
    lib = dec._lib
    dec.reset()
    gen = torch.Generator().manual_seed(9)
    # K/V rows N(0, 1) over the whole cache of both layers (the op reads rows [0, cache_len))
    dec.k_cache.copy_(torch.randn(dec.k_cache.shape, generator=gen).to(torch.bfloat16))
    dec.v_cache.copy_(torch.randn(dec.v_cache.shape, generator=gen).to(torch.bfloat16))
    for layer, cache_len in ((1, 8192), (0, 37), (1, 7500), (0, 6945), (1, 200)):
        q = torch.randn(16 * 128, generator=gen).cuda()
        ref = _attention(dec, lib.mq_op_attention, layer, q, cache_len)
        got = _attention(dec, lib.mq_op_attention_noalloc, layer, q, cache_len)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), (layer, cache_len)
    # sizes are validated before anything runs
    q = torch.zeros(16 * 128, dtype=torch.float32, device="cuda")
    out = torch.empty_like(q)
    assert lib.mq_op_attention_noalloc(dec._h, 0, q.data_ptr(), max_seq + 1, out.data_ptr(),
                                       None) != 0
    assert b"cache_len" in lib.mq_last_error()
    assert lib.mq_op_attention_noalloc(dec._h, 0, q.data_ptr(), 0, out.data_ptr(), None) != 0
    assert lib.mq_op_attention_noalloc(dec._h, 2, q.data_ptr(), 10, out.data_ptr(), None) != 0
    assert lib.mq_op_attention_noalloc(None, 0, q.data_ptr(), 10, out.data_ptr(), None) != 0
    dec.check()
