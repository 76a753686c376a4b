"""flash_attn_bhwd (megaqwen/triton_flash_attn.py:27-171) on the GPU against the float64 oracle
(oracle/flash_attn_ref.py): every output within half an ulp of the output type of the exact
attention, plus FLASH_ATTN_ABS * max|v| (tests/tolerances.py); the argument contracts of
triton_flash_attn.py:38-50 on CUDA tensors."""
import numpy as np
import pytest
import torch

from oracle.flash_attn_ref import attention_bhwd
from tests.tolerances import FLASH_ATTN_ABS

pytestmark = pytest.mark.gpu


def _fa():
    from megaqwen_amd.flash_attn import flash_attn_bhwd
    return flash_attn_bhwd


def _inputs(shape, dtype, seed, mag=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g) * mag).to(dtype) for _ in range(3)]


def _half_ulp(x, dtype):
    mant, emin = (7, -126) if dtype == torch.bfloat16 else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return 0.5 * 2.0 ** (e - mant)


def _check(out, q, k, v, scale=None):
    assert out.dtype == q.dtype and out.shape == q.shape
    ref = attention_bhwd(q.double().numpy(), k.double().numpy(), v.double().numpy(), scale)
    o = out.double().cpu().numpy()
    assert np.isfinite(o).all()
    err = np.abs(o - ref)
    bound = _half_ulp(np.maximum(np.abs(ref), np.abs(o)), q.dtype) + \
        FLASH_ATTN_ABS * float(v.double().abs().max())
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert (err <= bound).all(), (
        f"{int((err > bound).sum())} outputs out of bound; worst at {worst}: "
        f"got {o[worst]}, oracle {ref[worst]}, bound {bound[worst]}")
    return float(err.max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t", [1, 37, 1500])
def test_audio_tower_shapes(dtype, t):
    """B = 1, 14 heads of 64 (Qwen3-ASR-0.6B audio tower), default scale 1/8."""
    q, k, v = _inputs((1, 14, t, 64), dtype, seed=t)
    out = _fa()(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    _check(out.cpu(), q, k, v)


def test_batches_heads_scale_and_strided_inputs():
    """B = 2, H = 3, explicit scale, inputs that are [B, T, H, D] tensors viewed as [B, H, T, D]
    (non-contiguous: the front end makes them contiguous, as the reference does)."""
    g = torch.Generator().manual_seed(5)
    base = [torch.randn(2, 100, 3, 64, generator=g).to(torch.float16) for _ in range(3)]
    q, k, v = (x.transpose(1, 2) for x in base)
    out = _fa()(*(x.cuda() for x in (q, k, v)), scale=0.37)
    torch.cuda.synchronize()
    _check(out.cpu(), q.contiguous(), k.contiguous(), v.contiguous(), scale=0.37)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_peaked_softmax(dtype):
    """Scores spanning hundreds (inputs of std 6): the running max moves often and most weights
    underflow; the online rescale must keep the result exact to the bound."""
    q, k, v = _inputs((1, 4, 700, 64), dtype, seed=11, mag=6.0)
    v = torch.randn(v.shape, generator=torch.Generator().manual_seed(12)).to(dtype)
    out = _fa()(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    _check(out.cpu(), q, k, v)


def test_deterministic_and_stream_ordered():
    q, k, v = (x.cuda() for x in _inputs((1, 14, 333, 64), torch.bfloat16, seed=3))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a = _fa()(q, k, v)
        b = _fa()(q, k, v)
    s.synchronize()
    assert torch.equal(a, b)


def test_empty_and_argument_contracts():
    fa = _fa()
    z = torch.zeros(1, 14, 0, 64, dtype=torch.bfloat16, device="cuda")
    out = fa(z, z, z)
    assert out.shape == z.shape and out.dtype == z.dtype
    x = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="only supports fp16/bf16"):
        fa(x.float(), x.float(), x.float())
    with pytest.raises(ValueError, match=r"Expected q.ndim=4"):
        fa(x[0], x[0], x[0])
    with pytest.raises(ValueError, match="Shape mismatch"):
        fa(x, x[:, :, :3], x)
    y = torch.zeros(1, 2, 4, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="Only head_dim=64 supported, got 128"):
        fa(y, y, y)
    with pytest.raises(ValueError, match="dtype"):
        fa(x, x.half(), x)
