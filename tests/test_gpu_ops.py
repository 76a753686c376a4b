"""Per-op parity of the HIP decode kernels against the CPU oracle (BASELINE config 2 ops).

Each op runs through the C ABI (op-level entry points of libmegaqwen_hip.so) at the real
Qwen3-0.6B layer shape and is compared with the oracle's primitives (oracle/ref_cpu.py) on the
same seeded bf16 weights.  Tolerances: fp32 results 1e-4 absolute (different summation order
only); bf16 outputs within one bf16 ulp of the fp32-then-rounded oracle value.
"""
import math

import pytest
import torch

from megaqwen_amd.rope import build_rope_tables
from oracle.ref_cpu import attend, bf16, rms_norm, rope, silu
from tests.helpers import build_pair

pytestmark = pytest.mark.gpu

VOCAB = 151936
MAX_SEQ = 32768


@pytest.fixture(scope="module")
def pair():
    dec, _, sp, w = build_pair(1, VOCAB, MAX_SEQ, seed=11, norm_jitter=0.1, oracle=False)
    lw = {k: t.float() for k, t in zip(
        ("input_ln", "q", "k", "v", "q_norm", "k_norm", "o", "post_ln", "gate", "up", "down"),
        w["layer_weights"][:11])}
    return dec, lw, w


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


def test_op_qkv_rope(pair):
    dec, lw, _ = pair
    g = torch.Generator().manual_seed(1)
    cos, sin = build_rope_tables(MAX_SEQ, 1e6, 128)
    for pos in (0, 5, 4096, MAX_SEQ - 1):
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        q = dec.op_qkv_rope(0, x.cuda(), pos).cpu()
        torch.cuda.synchronize()
        n = rms_norm(x.float(), lw["input_ln"])
        c, s = cos[pos].float(), sin[pos].float()
        q_ref = rope(rms_norm((lw["q"] @ n).view(16, 128), lw["q_norm"]), c, s).reshape(-1)
        k_ref = rope(rms_norm((lw["k"] @ n).view(8, 128), lw["k_norm"]), c, s)
        v_ref = (lw["v"] @ n).view(8, 128)
        assert (q - q_ref).abs().max() < 1e-4, pos
        kc = dec.k_cache[0, :, pos].float().cpu()
        vc = dec.v_cache[0, :, pos].float().cpu()
        assert ((kc - k_ref).abs() <= _bf16_ulp(k_ref)).all(), pos
        assert ((vc - v_ref).abs() <= _bf16_ulp(v_ref) + 1e-6).all(), pos
        assert (kc == bf16(k_ref)).float().mean() > 0.98


@pytest.mark.parametrize("L", [1, 7, 128, 1024, 4097, 8192, 32768])
def test_op_attention(pair, L):
    dec, _, _ = pair
    g = torch.Generator().manual_seed(L)
    K = torch.randn(8, L, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(8, L, 128, generator=g).to(torch.bfloat16)
    dec.k_cache[0, :, :L] = K.cuda()
    dec.v_cache[0, :, :L] = V.cuda()
    q = torch.randn(16 * 128, generator=g)
    out = dec.op_attention(0, q.cuda(), L).cpu()
    ref = attend(q.view(16, 1, 128).double(), K.double().repeat_interleave(2, 0),
                 V.double().repeat_interleave(2, 0), 1.0 / math.sqrt(128)).reshape(-1)
    err = float((out.double() - ref).abs().max())
    print(f"attention L={L}: max |err| vs fp64 = {err:.3e}, max |ref| = {float(ref.abs().max()):.3f}")
    assert err < 1e-4


def test_op_attention_closed_forms(pair):
    dec, _, _ = pair
    g = torch.Generator().manual_seed(5)
    V = torch.randn(8, 300, 128, generator=g).to(torch.bfloat16)
    dec.v_cache[0, :, :300] = V.cuda()
    # L = 1: output is V[0] of the query's kv head exactly
    dec.k_cache[0, :, :1] = torch.randn(8, 1, 128, generator=g).to(torch.bfloat16).cuda()
    out = dec.op_attention(0, torch.randn(2048, generator=g).cuda(), 1).cpu().view(16, 128)
    assert torch.allclose(out, V[:, 0].float().repeat_interleave(2, 0), atol=1e-6)
    # K == 0: uniform weights -> mean of V
    dec.k_cache[0, :, :300] = 0
    out = dec.op_attention(0, torch.randn(2048, generator=g).cuda(), 300).cpu().view(16, 128)
    assert torch.allclose(out, V.float().mean(1).repeat_interleave(2, 0), atol=1e-5)


def test_op_mlp(pair):
    dec, lw, _ = pair
    g = torch.Generator().manual_seed(3)
    for _ in range(3):
        a = torch.randn(1024, generator=g)
        x = dec.op_mlp(0, a.cuda()).float().cpu()
        n2 = rms_norm(a, lw["post_ln"])
        ref = lw["down"] @ (silu(lw["gate"] @ n2) * (lw["up"] @ n2)) + a
        assert ((x - ref).abs() <= _bf16_ulp(ref) + 1e-6).all()
        assert (x == bf16(ref)).float().mean() > 0.98


def test_op_lm_head(pair):
    dec, _, w = pair
    g = torch.Generator().manual_seed(4)
    E = w["embed_weight"].float()
    fn = w["final_norm_weight"].float()
    logits = torch.empty(VOCAB, dtype=torch.float32, device="cuda")
    for i in range(4):
        x = torch.randn(1024, generator=g).to(torch.bfloat16)
        tok = dec.op_lm_head(x.cuda(), logits=logits)
        lg = logits.cpu()
        ref = E @ rms_norm(x.float(), fn)
        assert (lg - ref).abs().max() < 1e-4
        assert int(tok.item()) == int(torch.argmax(lg))           # exact argmax of its own logits
        if (torch.topk(ref, 2).values[0] - torch.topk(ref, 2).values[1]) > 2e-4:
            assert int(tok.item()) == int(torch.argmax(ref))


def test_op_lm_head_planted_max_and_ties(pair):
    """A planted maximum row wins; among exactly equal maxima the lowest index wins."""
    dec, _, w = pair
    x = torch.zeros(1024, dtype=torch.bfloat16)
    x[7] = 1.0
    E = dec.lm_head_weight
    saved = E[:, 7].clone()
    try:
        E[:, 7] = -1.0
        E[150000, 7] = 2.0
        assert int(dec.op_lm_head(x.cuda()).item()) == 150000
        E[3, 7] = 2.0
        E[151935, 7] = 2.0
        assert int(dec.op_lm_head(x.cuda()).item()) == 3
    finally:
        E[:, 7] = saved
