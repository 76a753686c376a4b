"""flash_attn_bhwd without a GPU: the oracle pinned against torch's SDPA and closed forms, the
front end's argument contracts (triton_flash_attn.py:38-50) as far as they precede the device
check, and the C ABI's rejections (no kernel launches)."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle.flash_attn_ref import attention_bhwd
from megaqwen_amd import _lib


def _rand(shape, seed, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape) * scale).astype(np.float64)


@pytest.mark.parametrize("b,h,t,scale", [(1, 14, 37, None), (2, 3, 65, 0.3), (1, 2, 1, None)])
def test_oracle_matches_torch_sdpa(b, h, t, scale):
    q, k, v = (_rand((b, h, t, 64), s) for s in (1, 2, 3))
    ref = attention_bhwd(q, k, v, scale)
    sd = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
        scale=(1.0 / math.sqrt(64) if scale is None else scale)).numpy()
    np.testing.assert_allclose(ref, sd, rtol=1e-12, atol=1e-12)


def test_oracle_closed_forms():
    q, k, v = (_rand((1, 2, 9, 64), s) for s in (4, 5, 6))
    # one key: the output is its v row
    np.testing.assert_allclose(attention_bhwd(q[:, :, :1], k[:, :, :1], v[:, :, :1]),
                               v[:, :, :1], rtol=0, atol=1e-15)
    # scale 0: uniform weights, the mean of v over the keys
    np.testing.assert_allclose(attention_bhwd(q, k, v, 0.0),
                               np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape),
                               rtol=1e-13, atol=1e-13)
    # one dominant key: its v row
    k2 = k.copy()
    k2[:, :, 4] = q[:, :, 0] * 100.0
    out = attention_bhwd(q[:, :, :1], k2, v)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 4], rtol=0, atol=1e-12)
    # keys permuted together with their values: no change
    perm = np.random.default_rng(7).permutation(9)
    np.testing.assert_allclose(attention_bhwd(q, k[:, :, perm], v[:, :, perm]),
                               attention_bhwd(q, k, v), rtol=1e-13, atol=1e-13)


def test_oracle_catches_a_dropped_scale():
    """A planted mistake (scale ignored) in a copy of the oracle fails the SDPA check."""
    q, k, v = (_rand((1, 2, 17, 64), s) for s in (8, 9, 10))
    wrong = attention_bhwd(q, k, v, 1.0)
    sd = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v)).numpy()
    assert np.abs(wrong - sd).max() > 1e-3


def test_front_end_contracts_on_cpu():
    sys.modules.pop("triton", None)
    from megaqwen_amd.flash_attn import flash_attn_bhwd, is_triton_available
    assert is_triton_available() is False
    assert "triton" not in sys.modules
    t = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="expects CUDA tensors"):
        flash_attn_bhwd(t, t, t)


def test_compat_import_path():
    import os
    compat = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                          "megaqwen_amd", "compat")
    sys.path.insert(0, compat)
    try:
        from megaqwen.triton_flash_attn import flash_attn_bhwd, is_triton_available
        from megaqwen_amd import flash_attn
        assert flash_attn_bhwd is flash_attn.flash_attn_bhwd
        assert is_triton_available() is False
    finally:
        sys.path.remove(compat)


def test_c_abi_rejections():
    lib = _lib.load()
    fake = 1 << 20
    f = lib.mq_flash_attn_bhwd
    ws = lib.mq_flash_attn_workspace_bytes(1, 14, 1500, 64)
    assert ws == 2 * 14 * 47 * 32 * 64 * 2                  # K and V^T copies, 32-key tiles
    assert lib.mq_flash_attn_workspace_bytes(1, 1, 4, 128) == 0
    W = 1 << 24
    bf = _lib.MQ_DTYPE_BF16
    assert f(fake, fake, fake, fake, 1, 1, 4, 128, bf, 1.0, W, 1 << 20, None) == _lib.MQ_ERR_INVALID_ARG
    assert b"head_dim=64" in lib.mq_last_error()
    assert f(fake, fake, fake, fake, 1, 1, 4, 64, 7, 1.0, W, 1 << 20, None) == _lib.MQ_ERR_INVALID_ARG
    assert f(None, fake, fake, fake, 1, 1, 4, 64, bf, 1.0, W, 1 << 20, None) == _lib.MQ_ERR_INVALID_ARG
    assert f(fake, fake, fake, fake, -1, 1, 4, 64, bf, 1.0, W, 1 << 20, None) == _lib.MQ_ERR_INVALID_ARG
    assert f(fake, fake, fake, fake, 300, 300, 4, 64, _lib.MQ_DTYPE_F16, 1.0, W, 1 << 20, None) \
        == _lib.MQ_ERR_INVALID_ARG
    assert b"65535" in lib.mq_last_error()
    # out overlapping v
    assert f(fake, 2 * fake, 3 * fake, 3 * fake + 64, 1, 1, 4, 64, bf, 1.0, W, 1 << 20, None) \
        == _lib.MQ_ERR_INVALID_ARG
    assert b"overlap" in lib.mq_last_error()
    # workspace too small, or missing
    assert f(fake, 2 * fake, 3 * fake, 4 * fake, 1, 1, 40, 64, bf, 1.0, W, 100, None) \
        == _lib.MQ_ERR_INVALID_ARG
    assert b"workspace" in lib.mq_last_error()
    assert f(fake, 2 * fake, 3 * fake, 4 * fake, 1, 1, 40, 64, bf, 1.0, None, 1 << 20, None) \
        == _lib.MQ_ERR_INVALID_ARG
    # empty problems are no-ops (nothing is launched)
    assert f(None, None, None, None, 1, 14, 0, 64, bf, 1.0, None, 0, None) == _lib.MQ_OK
