"""C-ABI checks that need no GPU: the library loads, exports every function the public header
declares, sizes buffers, and rejects bad arguments with error codes and messages."""
import ctypes
import os
import re

import pytest

from megaqwen_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "megaqwen_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmegaqwen_hip.so is not built: run `python -m megaqwen_amd.build`")
    return _lib.load()


def test_exports_match_header(lib):
    declared = header_functions()
    assert declared, "no functions parsed from the header"
    assert sorted(_lib.EXPORTED) == declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.mq_abi_version() == _lib.ABI_VERSION


def _desc(num_layers=28, vocab=151936, max_seq=4096, max_prefill=512, hidden=1024):
    fake = 1 << 20                                   # 16-byte aligned non-null placeholder
    layers = (_lib.LayerWeights * num_layers)()
    for l in range(num_layers):
        layers[l] = _lib.LayerWeights(*[fake] * 11)
    d = _lib.ModelDesc(hidden_size=hidden, intermediate_size=3072, num_q_heads=16, num_kv_heads=8,
                       head_dim=128, num_layers=num_layers, vocab_size=vocab,
                       max_seq_len=max_seq, max_prefill_len=max_prefill, embed=fake,
                       final_norm=fake, lm_head=fake, cos_table=fake, sin_table=fake,
                       layers=layers)
    d._keep = layers
    return d


def test_sizes(lib):
    d = _desc()
    assert lib.mq_kv_cache_bytes(ctypes.byref(d)) == 28 * 8 * 4096 * 128 * 2
    ws = lib.mq_workspace_bytes(ctypes.byref(d))
    d0 = _desc(max_prefill=0)
    ws0 = lib.mq_workspace_bytes(ctypes.byref(d0))
    assert 0 < ws0 < ws and ws % 256 == 0
    # prefill buffers: h, xn [n,1024], qkv [n,4096], att [n,2048], m [n,3072] in bf16
    assert ws - ws0 >= 512 * (1024 * 2 + 4096 + 2048 + 3072) * 2


def test_rejects_bad_shapes_and_args(lib):
    bad = _desc(hidden=2048)
    assert lib.mq_workspace_bytes(ctypes.byref(bad)) == 0
    assert b"compiled Qwen3-0.6B shape" in lib.mq_last_error()
    d = _desc(max_prefill=5000, max_seq=4096)
    assert lib.mq_workspace_bytes(ctypes.byref(d)) == 0
    d = _desc()
    d.embed = 3                                      # misaligned
    assert lib.mq_workspace_bytes(ctypes.byref(d)) == 0
    out = ctypes.c_void_p()
    assert lib.mq_decoder_create(ctypes.byref(_desc()), None, None, None, 0,
                                 ctypes.byref(out)) == _lib.MQ_ERR_INVALID_ARG
    assert out.value is None
    assert lib.mq_decode_step(None, None, None, None, None) == _lib.MQ_ERR_INVALID_ARG
    assert lib.mq_prefill(None, None, 0, None, None, None) == _lib.MQ_ERR_INVALID_ARG
    assert lib.mq_prefill_fused(None, None, 4, None, 0, 0, None, None, None) == \
        _lib.MQ_ERR_INVALID_ARG
    assert lib.mq_decoder_position(None) == -1
    with pytest.raises(_lib.MegaQwenError):
        _lib.check(lib.mq_decoder_reset(None, None))


def test_decoder_requires_cuda_tensors():
    import torch
    from megaqwen_amd.decoder import MegakernelDecoder
    t = torch.zeros(4, dtype=torch.bfloat16)
    with pytest.raises((TypeError, ValueError)):
        MegakernelDecoder(t, [t] * 11, t, t, t, t, 1, 16)


def test_decode_kernels_do_not_spill():
    """The decode kernels' register budget (two waves per SIMD for the 512-thread persistent
    kernel) is nearly full; a spill to scratch compiles silently and slows every decode step
    (a merge that held 16 64-bit words per thread spilled 99 VGPRs and cost ~15%).  The build records the
    compiler's per-kernel resource usage; every decode kernel must show no spill and no scratch."""
    from megaqwen_amd.build import RESOURCE_REPORT, parse_resource_usage
    if not os.path.exists(RESOURCE_REPORT):
        pytest.skip("no resource report: build with `python -m megaqwen_amd.build`")
    usage = parse_resource_usage(open(RESOURCE_REPORT).read())
    persistent = [k for k in usage if "mq_decode_persistent_kernel" in k]
    assert len(persistent) == 2, sorted(usage)
    for name, u in usage.items():
        assert u.get("VGPRs Spill", -1) == 0, (name, u)
        assert u.get("ScratchSize", -1) == 0, (name, u)
    for name in persistent:
        assert usage[name]["VGPRs"] + usage[name].get("AGPRs", 0) <= 256, usage[name]


def test_exchange_epoch_arithmetic(lib):
    """The persistent decode kernel hands values between workgroups as words carrying the epoch
    of the layer that wrote them (64-bit words) or a 2-bit tag of it (4-byte words); a reader
    must never take a stale word for a fresh one.  Checked here on the library's own epoch
    functions (the ones the kernels evaluate) at bases around the wrap of the epoch count:
    an epoch is never 0 (0 means "take the word without waiting" and is what cleared buffers and
    the one-kernel-per-phase mode hold), consecutive layers get cyclically consecutive epochs,
    the tags of any three consecutive epochs differ (a buffer alternates by layer parity, so the
    word a reader may still see was written one or two epochs earlier), and the base a launch
    leaves behind continues the sequence exactly."""
    P = lib.mq_exchange_epoch_period()
    assert P % 3 == 0 and P >= 1 << 31
    L, steps = 28, 64                    # layers per step, steps per chained launch
    bases = [0, 1, 2, 12345, P // 2, P - 3, P - 2, P - 1, P - L * steps, P - L * steps - 1]
    for b in bases:
        prev = []
        for k in range(2 * L * steps):
            e = lib.mq_exchange_epoch(b, k)
            assert 1 <= e <= P, (b, k, e)
            if prev:
                assert e == prev[-1] % P + 1, (b, k, e, prev[-1])
            window = [e] + prev[-2:]
            tags = [lib.mq_exchange_tag(x) for x in window]
            assert all(1 <= t <= 3 for t in tags) and len(set(tags)) == len(tags), (b, k, window)
            prev.append(e)
    for b in bases:
        for n in (0, 1, L, L * steps, P - 1, P, 2 * P + 5, (1 << 40) + 7):
            nb = lib.mq_exchange_epoch_advance(b, n)
            assert 0 <= nb < P
            for k in (0, 1, 2 * L):
                assert lib.mq_exchange_epoch(nb, k) == lib.mq_exchange_epoch(b, n + k), (b, n, k)
    # far past one period (a decoder never reset for years): still never 0
    for k in (P - 1, P, 2 * P - 1, 1 << 33, (1 << 40) + 3):
        for b in (0, P - 1):
            assert lib.mq_exchange_epoch(b, k) != 0
