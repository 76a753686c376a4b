"""Batch-1 bf16 Qwen3-0.6B decode benchmark on one MI355X (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload: Qwen3-0.6B architecture (28 layers, hidden 1024, 16/8 heads x 128, MLP 3072, vocab
151936, tied LM head), seeded N(0, 0.02) bf16 weights (megaqwen_amd.synthetic, seed 0), batch 1,
greedy decode.  A step is one decoded token.  Exactly K steps are timed at each position bucket:
positions 1..K, 128..127+K (the headline `value`) and 4096..4095+K; each bucket starts from an
untimed prefill of that many uniform-random tokens (seed 1), as BASELINE config 5 does for 4096.
Inputs are resident in HBM; the timed region is a device-side token chain (`mq_decode_steps`: the
persistent kernel decodes up to 64 chained tokens per launch, no host round trip per token).  The
rate with one launch per token is reported too (`tok_s_one_launch_per_token`, pos 128).

Prefill: a 512-token uniform-random prompt (seed 1) through the MFMA prefill,
reported as tokens/s and MFMA utilisation = 481.4 GFLOP (linear 450.97 + causal attention 30.12 +
last-token LM head 0.31) / time / 2.5 PFLOP/s dense bf16; the 4096-token prefill time is
reported too.

Roofline: algorithmic bytes per token = bf16 weights streamed (1,192,101,888 B) + KV read
(114,688 B x (pos + 1)) + KV write (114,688 B), times the tokens of a launch, over the per-launch
duration measured with HIP events on the launch stream, against 8 TB/s.  `traffic` is the HBM
bytes per launch: the bytes per token measured by two rocprofv3 counter passes (FETCH_SIZE,
WRITE_SIZE over `--pmc-workload`, scaled by what the same counters read for a 256 MiB copy),
taken from the committed profile summary, times the tokens of a launch; reported only while the
decode kernel sources still hash to the measured version (else null).

cpu_baseline: the CPU oracle (oracle/ref_cpu.py, PyTorch fp32 restatement of the reference decode
path) on BASELINE config 1 (16-token prompt fed through decode, then 32 greedy tokens), timed on
this host with all its cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12
WEIGHT_BYTES = 1_192_101_888
KV_BYTES_PER_POS = 28 * 8 * 128 * 2 * 2     # K + V, all layers, bf16


DECODE_SOURCES = ("decode.hip", "mq_device.h", "mq_decode.h", "mq_config.h")
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_persistent_qwen3_0.6b.md")


def decode_source_sha() -> str:
    import hashlib
    d = os.path.join(ROOT, "megaqwen_amd", "csrc")
    return hashlib.sha256(b"".join(open(os.path.join(d, f), "rb").read()
                                   for f in DECODE_SOURCES)).hexdigest()[:16]


def measured_traffic():
    """HBM bytes per decoded token from the committed FETCH_SIZE / WRITE_SIZE counter passes
    (copy-calibrated), or None when the decode sources changed since they were measured."""
    try:
        kv = dict(line.strip().split(": ", 1) for line in open(TRAFFIC_PROFILE)
                  if line.startswith("    ") and ": " in line)
    except OSError:
        return None
    if kv.get("source_sha") != decode_source_sha():
        return None
    return int(kv["traffic_bytes_per_token"])


def bytes_per_token(pos: int) -> int:
    return WEIGHT_BYTES + KV_BYTES_PER_POS * (pos + 1) + KV_BYTES_PER_POS


MFMA_BF16_PEAK = 2.5e15
LINEAR_PARAMS_PER_LAYER = 4096 * 1024 + 1024 * 2048 + 2 * 3072 * 1024 + 1024 * 3072


def prefill_flops(n: int) -> float:
    linear = 2.0 * n * LINEAR_PARAMS_PER_LAYER * 28
    attention = 28 * 16 * (n * (n + 1) / 2) * 128 * 4
    lm_head = 2.0 * 151936 * 1024
    return linear + attention + lm_head


def build_decoder(max_seq: int, max_prefill: int = 0):
    import torch
    from megaqwen_amd.decoder import MegakernelPrefillDecoder
    from megaqwen_amd.rope import build_rope_tables
    from megaqwen_amd.spec import _DEFAULT_MODEL_SPEC
    from megaqwen_amd.synthetic import make_weights

    spec = dict(_DEFAULT_MODEL_SPEC)
    w = make_weights(spec, seed=0)
    cos, sin = build_rope_tables(max_seq, 1e6, 128)
    emb = w["embed_weight"].cuda()
    layers = [t.cuda() for t in w["layer_weights"]]
    dec = MegakernelPrefillDecoder(emb, layers, w["final_norm_weight"].cuda(), emb, cos.cuda(),
                                   sin.cuda(), spec["num_layers"], max_seq,
                                   max_prefill_len=max_prefill)
    return dec, spec


STEPS_PER_LAUNCH = 64     # tokens the persistent kernel chains in one launch (MQ_STEPS_PER_LAUNCH)


def time_bucket(dec, start_pos: int, steps: int, per_launch_steps: int = STEPS_PER_LAUNCH):
    """Prefills `start_pos` random tokens, then times `steps` decode steps as a device-side chain
    of launches of up to `per_launch_steps` tokens, with an event pair around each launch (launch
    duration) inside one region bracketed by synchronize (wall time).  Returns (wall seconds,
    mean seconds per launch, mean tokens per launch)."""
    import torch
    from megaqwen_amd.synthetic import make_tokens
    dec.reset()
    tok = dec.prefill_step(make_tokens(start_pos, 151936, seed=1))
    assert dec.position() == start_pos
    buf = torch.empty(steps + 1, dtype=torch.int32, device="cuda")
    buf[0] = tok
    chunks = [(i, min(per_launch_steps, steps - i)) for i in range(0, steps, per_launch_steps)]
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in chunks]
    lib, h = dec._lib, dec._h
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for (i, n), (a, b) in zip(chunks, ev):
        a.record(stream)
        rc = lib.mq_decode_steps(h, buf.data_ptr() + 4 * i, n, sp)
        b.record(stream)
        if rc != 0:
            raise RuntimeError(lib.mq_last_error().decode())
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch = sum(a.elapsed_time(b) for a, b in ev) / len(ev) / 1e3
    dec.check()
    return wall, per_launch, steps / len(chunks)


def time_prefill_fused(dec, n: int, reps: int):
    """Best event-timed `mq_prefill_fused` call over `reps` (the fused short-prompt prefill of
    MegakernelFusedPrefillDecoder, n <= 64), after one warm-up call."""
    import torch
    from megaqwen_amd.synthetic import make_tokens
    d = make_tokens(n, 151936, seed=1).cuda()
    times = []
    for r in range(reps + 1):
        dec.reset()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        rc = dec._lib.mq_prefill_fused(dec._h, d.data_ptr(), n, None, 0, 0,
                                       dec._tok.data_ptr() + 4, None,
                                       torch.cuda.current_stream().cuda_stream)
        b.record()
        if rc != 0:
            raise RuntimeError(dec._lib.mq_last_error().decode())
        torch.cuda.synchronize()
        if r > 0:
            times.append(a.elapsed_time(b) / 1e3)
    dec.check()
    return min(times)


def time_prefill(dec, n: int, reps: int):
    import torch
    from megaqwen_amd.synthetic import make_tokens
    toks = make_tokens(n, 151936, seed=1)
    dec.reset()
    dec.prefill_step(toks)                       # warm-up
    times = []
    for _ in range(reps):
        dec.reset()
        d = toks.cuda()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        rc = dec._lib.mq_prefill(dec._h, d.data_ptr(), n, dec._tok.data_ptr() + 4, None,
                                 torch.cuda.current_stream().cuda_stream)
        b.record()
        if rc != 0:
            raise RuntimeError(dec._lib.mq_last_error().decode())
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / 1e3)
    dec.check()
    return min(times), sum(times) / len(times)


QKV_BYTES = 4096 * 1024 * 2 + 1024 * 2 + 2 * 128 * 2        # q|k|v rows, input norm, q/k norms
MLP_BYTES = 3 * 3072 * 1024 * 2 + 1024 * 2                  # gate, up, down, post-attention norm
LM_HEAD_BYTES = 151936 * 1024 * 2 + 1024 * 2                # tied LM head, final norm
ATT_LENGTHS = (1, 128, 1024, 8192, 32768)


def time_op(fn, reps: int):
    """Mean seconds per call of fn() over `reps` calls, and how it was timed.  The calls are
    captured into one HIP graph and replayed between HIP events, so the figure is device time
    (kernels and the gaps between them), not the Python/ctypes cost of issuing each call; if
    capture fails, the calls are issued eagerly between the events instead ("eager")."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / 1e3 / reps, "graph"
    except RuntimeError:
        torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / reps, "eager"


def time_ops(dec):
    """each decode op of the Qwen3-0.6B shapes through its C-ABI entry point,
    as GB/s of its algorithmic bytes against the 8 TB/s HBM peak; plus flash_attn_bhwd (the audio
    tower's attention, B=1, 14 heads, T=1500) as TFLOP/s against the dense MFMA peak."""
    import torch
    from megaqwen_amd.flash_attn import flash_attn_bhwd
    g = torch.Generator(device="cuda").manual_seed(3)
    x = (torch.randn(1024, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    a = torch.randn(1024, device="cuda", generator=g)
    q = torch.randn(16 * 128, device="cuda", generator=g)
    qo = torch.empty(16 * 128, device="cuda")
    xo = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    ops = {}

    def entry(name, timed, nbytes):
        sec, how = timed
        ops[name] = {"us": round(sec * 1e6, 2), "bytes": int(nbytes),
                     "gb_s": round(nbytes / sec / 1e9, 1), "frac": round(nbytes / sec / HBM_PEAK, 4),
                     "timing": how}

    dec.reset()
    entry("qkv_norm_rope", time_op(lambda: dec.op_qkv_rope(0, x, 100, qo), 200), QKV_BYTES)
    entry("mlp_swiglu", time_op(lambda: dec.op_mlp(0, a, xo), 200), MLP_BYTES)
    entry("lm_head_argmax", time_op(lambda: dec.op_lm_head(x, tok), 50), LM_HEAD_BYTES)
    # K/V ~ N(0, 1) in layer 0's cache rows [0, max(L))
    n = max(ATT_LENGTHS)
    dec.k_cache[0, :, :n].normal_(generator=g)
    dec.v_cache[0, :, :n].normal_(generator=g)
    for L in ATT_LENGTHS:
        entry(f"attention_L{L}", time_op(lambda: dec.op_attention(0, q, L, qo), 100),
              L * 8 * 128 * 2 * 2 + 16 * 128 * 4)
    qf, kf, vf = (torch.randn(1, 14, 1500, 64, device="cuda", generator=g).to(torch.bfloat16)
                  for _ in range(3))
    sec, how = time_op(lambda: flash_attn_bhwd(qf, kf, vf), 50)
    flops = 4.0 * 14 * 1500 * 1500 * 64
    ops["flash_attn_bhwd_T1500"] = {"us": round(sec * 1e6, 2), "tflops": round(flops / sec / 1e12, 1),
                                    "frac_mfma_peak": round(flops / sec / MFMA_BF16_PEAK, 4),
                                    "timing": how}
    dec.reset()
    return ops


def time_buckets(dec):
    """16-token random prompt, greedy decode from position 16 to 256 as one
    device-side token chain, one persistent launch per bucket (16-63, 64-127, 128-191, 192-255)
    with an event pair around each.  Returns {bucket: tok/s} and the whole run's wall tok/s."""
    import torch
    from megaqwen_amd.synthetic import make_tokens
    dec.reset()
    first = dec.prefill_step(make_tokens(16, 151936, seed=0))
    buckets = [(16, 64), (64, 128), (128, 192), (192, 256)]
    buf = torch.empty(257, dtype=torch.int32, device="cuda")
    buf[16] = first
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in buckets]
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for (lo, hi), (a, b) in zip(buckets, ev):
        a.record(stream)
        rc = dec._lib.mq_decode_steps(dec._h, buf.data_ptr() + 4 * lo, hi - lo, stream.cuda_stream)
        b.record(stream)
        if rc != 0:
            raise RuntimeError(dec._lib.mq_last_error().decode())
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dec.check()
    out = {}
    for (lo, hi), (a, b) in zip(buckets, ev):
        sec = a.elapsed_time(b) / 1e3
        mid = (lo + hi - 1) // 2
        out[f"{lo}-{hi - 1}"] = {"tok_s": round((hi - lo) / sec, 1),
                                 "roofline_frac": round(bytes_per_token(mid) * (hi - lo) / sec / HBM_PEAK, 4)}
    return out, round(240 / wall, 1)


def write_maps(path: str):
    """Copies /proc/self/maps (which file is mapped at which address) to `path`."""
    with open("/proc/self/maps") as src, open(path, "w") as dst:
        dst.write(src.read())


def teardown(*objs):
    """Ends the run's GPU work before the interpreter exits: waits for the device, drops the
    decoders and device tensors, and returns the caching allocator's blocks, so nothing of this
    program is left to be torn down by exit handlers after a profiler tool has finalized."""
    import gc
    import torch
    torch.cuda.synchronize()
    for o in objs:
        del o
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.synchronize()


def pmc_workload():
    """Fixed short run for counter passes (rocprofv3 --pmc ...): every dispatch is profiled, so
    it stays small.  The 256 MiB copy is the calibration kernel for the traffic counters."""
    import torch
    from megaqwen_amd.synthetic import make_tokens
    a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    dec, _ = build_decoder(256, max_prefill=128)
    tok = dec.prefill_step(make_tokens(128, 151936, seed=1))
    toks = dec.decode_steps_cuda(tok, 16)          # one persistent launch of 16 chained tokens
    torch.cuda.synchronize()
    dec.check()
    last = toks[-1].item()
    del a, b, toks, dec
    teardown()
    print(f"pmc workload done: 256 MiB copy, prefill 128, decode 16 -> {last}")


def prefill_workload(n: int):
    """One n-token prefill (after one warm-up call) for counter runs of the prefill kernels."""
    import torch
    from megaqwen_amd.synthetic import make_tokens
    dec, _ = build_decoder(n + 8, max_prefill=n)
    toks = make_tokens(n, 151936, seed=1)
    dec.prefill_step(toks)
    dec.reset()
    tok = dec.prefill_step(toks)
    torch.cuda.synchronize()
    dec.check()
    del dec
    teardown()
    print(f"prefill workload done: 2 x prefill {n} -> {tok}")


def flash_workload():
    """For counter runs of flash_attn_bhwd: B = 1, 14 heads, T = 1500, bf16, 10 calls."""
    import torch
    from megaqwen_amd.flash_attn import flash_attn_bhwd
    g = torch.Generator(device="cuda").manual_seed(3)
    q, k, v = (torch.randn(1, 14, 1500, 64, device="cuda", generator=g).to(torch.bfloat16)
               for _ in range(3))
    for _ in range(10):
        out = flash_attn_bhwd(q, k, v)
    torch.cuda.synchronize()
    checksum = float(out.float().abs().sum())
    del q, k, v, out
    teardown()
    print(f"flash workload done: 10 x flash_attn_bhwd [1, 14, 1500, 64] bf16 -> {checksum:.3f}")


def cpu_baseline(prompt_len: int = 16, gen: int = 32):
    import torch
    from megaqwen_amd.rope import build_rope_tables
    from megaqwen_amd.spec import _DEFAULT_MODEL_SPEC
    from megaqwen_amd.synthetic import make_tokens, make_weights
    from oracle.ref_cpu import OracleModel

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    spec = dict(_DEFAULT_MODEL_SPEC)
    w = make_weights(spec, seed=0, dtype=torch.float32)
    cos, sin = build_rope_tables(prompt_len + gen + 2, 1e6, 128)
    m = OracleModel(w, spec, cos, sin, prompt_len + gen + 2, round_bf16=True)
    prompt = make_tokens(prompt_len, spec["vocab_size"], seed=0).tolist()
    for t in prompt[:-1]:
        m.decode_step(t, return_logits=False)
    tok = m.decode_step(prompt[-1], return_logits=False)          # warm-up token
    t0 = time.perf_counter()
    for _ in range(gen):
        tok = m.decode_step(tok, return_logits=False)
    dt = time.perf_counter() - t0
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": gen / dt, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config 1: 28-layer fp32 CPU oracle, {prompt_len}-token prompt fed through "
                      f"decode, {gen} greedy tokens timed ({dt:.1f} s); os.cpu_count()={threads}; "
                      f"{cpu_model}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", default="persistent", choices=["persistent", "multi_kernel"])
    ap.add_argument("--pmc-workload", action="store_true",
                    help="short fixed workload for hardware-counter runs: a 256 MiB device copy "
                         "(calibration of FETCH_SIZE / WRITE_SIZE), a 128-token prefill, then one "
                         "decode launch of 16 chained steps at positions 128..143")
    ap.add_argument("--prefill-workload", type=int, default=0, metavar="N",
                    help="for counter runs of the prefill kernels: two N-token prefills, nothing else")
    ap.add_argument("--flash-workload", action="store_true",
                    help="for counter runs of flash_attn_bhwd: 10 calls at [1, 14, 1500, 64] bf16")
    ap.add_argument("--maps-out", default="", metavar="PATH",
                    help="write this process's /proc/self/maps to PATH when the run is done (to "
                         "attribute addresses in a crash report printed at exit)")
    args = ap.parse_args()
    if args.maps_out:
        import atexit
        atexit.register(write_maps, args.maps_out)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (--gpus {args.gpus} requested): the decode and prefill "
              "kernels here are single-GPU; there is no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.pmc_workload:
        pmc_workload()
        return
    if args.prefill_workload > 0:
        prefill_workload(args.prefill_workload)
        return
    if args.flash_workload:
        flash_workload()
        return
    K, W = int(args.steps), int(args.warmup)
    positions = (1, 128, 4096)
    max_seq = max(positions[-1] + K + 8, max(ATT_LENGTHS))
    dec, spec = build_decoder(max_seq, max_prefill=4096)
    dec.set_mode(args.mode)
    print(f"[bench] decoder ready: mode={dec.mode} grid={dec.grid} max_seq={max_seq}", file=sys.stderr,
          flush=True)
    # warm-up (untimed)
    dec.reset()
    dec.decode_steps_cuda(9707, W)
    torch.cuda.synchronize()
    res = {}
    for p in positions:
        wall, per_launch, tpl = time_bucket(dec, p, K)
        tok_s = K / wall
        mid = p + (K - 1) / 2
        res[p] = {"tok_s": tok_s, "ms_per_token": 1e3 * wall / K,
                  "launch_us": per_launch * 1e6, "tokens_per_launch": tpl,
                  "kernel_us_per_token": per_launch / tpl * 1e6,
                  "bytes_per_token": bytes_per_token(int(mid)),
                  "roofline_frac_wall": bytes_per_token(int(mid)) * tok_s / HBM_PEAK,
                  "roofline_frac_kernel": bytes_per_token(int(mid)) * tpl / per_launch / HBM_PEAK}
        print(f"[bench] pos {p}: {tok_s:.1f} tok/s, kernel {per_launch / tpl * 1e6:.1f} us/token "
              f"({tpl:.0f} tokens per launch), roofline {res[p]['roofline_frac_wall'] * 100:.1f}% "
              f"(wall) {res[p]['roofline_frac_kernel'] * 100:.1f}% (kernel)", file=sys.stderr,
              flush=True)
    # the reference's pattern, one launch per token (bindings_prefill.cpp:1045-1120)
    wall1, per_launch1, _ = time_bucket(dec, 128, K, per_launch_steps=1)
    one_launch = {"tok_s": round(K / wall1, 2), "kernel_us": round(per_launch1 * 1e6, 1)}
    print(f"[bench] pos 128, one launch per token: {one_launch['tok_s']} tok/s, kernel "
          f"{one_launch['kernel_us']} us", file=sys.stderr, flush=True)

    buckets, buckets_wall = time_buckets(dec)
    print(f"[bench] positions 16..255 by bucket: {buckets} (wall {buckets_wall} tok/s)",
          file=sys.stderr, flush=True)
    ops = time_ops(dec)
    print(f"[bench] ops: {ops}", file=sys.stderr, flush=True)

    pf_best, pf_mean = time_prefill(dec, 512, 5)
    pf4_best, _ = time_prefill(dec, 4096, 2)
    pf16_best, _ = time_prefill(dec, 16, 5)
    pf64_best, _ = time_prefill(dec, 64, 5)
    prefill = {"tokens": 512, "ms": round(pf_mean * 1e3, 3), "tok_s": round(512 / pf_mean, 1),
               "mfma_util": round(prefill_flops(512) / pf_mean / MFMA_BF16_PEAK, 4),
               "tflops": round(prefill_flops(512) / pf_mean / 1e12, 1),
               "ms_4096": round(pf4_best * 1e3, 2),
               "mfma_util_4096": round(prefill_flops(4096) / pf4_best / MFMA_BF16_PEAK, 4),
               "ms_16": round(pf16_best * 1e3, 3), "ms_64": round(pf64_best * 1e3, 3),
               "fused_ms_16": round(time_prefill_fused(dec, 16, 5) * 1e3, 3),
               "fused_ms_64": round(time_prefill_fused(dec, 64, 5) * 1e3, 3)}
    print(f"[bench] prefill 512: {prefill['ms']} ms, {prefill['tok_s']} tok/s, "
          f"{prefill['tflops']} TFLOP/s = {prefill['mfma_util'] * 100:.1f}% of dense bf16 peak; "
          f"4096: {prefill['ms_4096']} ms ({prefill['mfma_util_4096'] * 100:.1f}%); 16: "
          f"{prefill['ms_16']} ms; 64: {prefill['ms_64']} ms; fused prefill 16: "
          f"{prefill['fused_ms_16']} ms, 64: {prefill['fused_ms_64']} ms",
          file=sys.stderr, flush=True)
    head = res[128]
    achieved = head["bytes_per_token"] * head["tokens_per_launch"] / (head["launch_us"] * 1e-6)
    traffic = measured_traffic() if args.mode == "persistent" else None
    cpu = None
    del dec
    teardown()
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        print(f"[bench] cpu baseline {cpu['value']:.2f} tok/s on {cpu['cores']} threads",
              file=sys.stderr, flush=True)
    line = {
        "metric": "batch-1 decode tok/s at pos 1/128/4096 + % HBM roofline, Qwen3-0.6B bf16",
        "value": round(head["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(head["ms_per_token"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) random-init weights, greedy token chain)",
        "config": {"workload": "Qwen3-0.6B-architecture batch-1 greedy decode; value = positions "
                               f"128..{127 + K}", "layers": 28, "hidden": 1024, "vocab": 151936,
                   "kv_heads": 8, "head_dim": 128, "decode_mode": args.mode,
                   "tok_s_by_position": {str(p): round(r["tok_s"], 2) for p, r in res.items()},
                   "roofline_frac_by_position": {str(p): round(r["roofline_frac_wall"], 4)
                                                 for p, r in res.items()},
                   "tokens_per_launch": head["tokens_per_launch"],
                   "tok_s_one_launch_per_token": one_launch,
                   "tok_s_by_bucket_16_256": buckets, "tok_s_16_256_wall": buckets_wall,
                   "ops": ops,
                   "prefill": prefill},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 2), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": (int(traffic * head["tokens_per_launch"])
                                 if traffic is not None else None),
                     "kernel": "mq_decode_persistent_kernel" if args.mode == "persistent"
                     else "mq_decode_phase_kernel (all phases)",
                     "kernel_us": round(head["launch_us"], 2),
                     "kernel_us_per_token": round(head["kernel_us_per_token"], 2),
                     "bytes_per_launch": int(head["bytes_per_token"] * head["tokens_per_launch"])},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
