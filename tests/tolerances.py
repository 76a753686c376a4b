"""Logit tolerances of the GPU parity tests, and the oracle measurements they rest on.

The north-star bar is 2e-2 max-abs on per-step logits.  Where a test holds a looser bound, the
bound is at most twice the spread between the CPU oracle's own fp32 and fp64 evaluations of the
same case (same weights, tokens and bf16 rounding points): how far fp32 summation order alone
moves the result.  The GPU sums in fp32 in yet another order, so its distance from the fp32
oracle is expected at the same scale.  tests/test_oracle_spread.py recomputes every spread
below on the CPU and fails if a bound exceeds twice its measurement.
"""

# north star: per-step logits, 2-layer decode (also against the unrounded fp32 oracle)
DECODE_LOGITS = 2e-2

# 28-layer free-running decode (tests/test_gpu_decode.py: seed 0, 8 tokens of seed 0): the
# oracle's fp32-vs-fp64 spread is 2.76e-2 (steps 1-7; step 0 is 8.8e-7), so the bound is 5.5e-2
DECODE_28L_SPREAD = 2.76e-2
DECODE_28L = 5.5e-2

# prefill logits, 2 layers (tests/test_gpu_prefill.py `small`: seed 2, norm jitter 0.1,
# n in {1, 7, 64, 100, 512}, tokens of seed n): spread 1.69e-2 .. 2.03e-2 (n = 100)
PREFILL_2L_SPREAD = 2.03e-2
PREFILL_2L = 4e-2

# prefill logits, 28 layers, 512 tokens (seed 0 weights, tokens of seed 1): spread 3.66e-2
PREFILL_28L_SPREAD = 3.66e-2
PREFILL_28L = 7e-2

# the multi-kernel prefill's bf16 rounding points (bf16 after every op, as launch_prefill_float)
# against the unrounded fp32 model that the HF fixtures pin, on the CPU oracle (2 layers, seed 2,
# norm jitter 0.1, n in {1, 7, 64, 100, 512}, tokens of seed n): 1.85e-2 .. 2.90e-2 (n = 64).
# tests/test_oracle_spread.py holds the oracle between these two bounds: the rounding points
# must move the logits (a lost rounding point shrinks the distance) but only by bf16 noise.
PREFILL_ROUNDING_2L_MIN = 1.0e-2
PREFILL_ROUNDING_2L = 3.0e-2
# GPU multi-kernel prefill against the unrounded fp32 oracle, same 2-layer cases (n in {7, 64,
# 512}): the rounding above plus the GPU's own fp32 summation order (PREFILL_2L_SPREAD)
PREFILL_VS_FP32_2L = 5e-2

# fused short-prompt prefill (tests/test_gpu_fused_prefill.py) against the oracle's restatement
# of the prefill megakernel (fp32 activations, bf16 weights): measured 2.6e-6 .. 4.4e-6 at n in
# {1, 7, 16, 20, 24, 33, 64} with 2 and 28 layers; held at 2e-5.  On the CPU oracle, activations
# kept to 16 significant bits (the three-part bf16 split without its lo part) move the logits by
# 3.4e-5 .. 6.5e-5, bf16 norm outputs by 8.7e-3 .. 1.7e-2 (tests/test_oracle_spread.py).
FUSED_PREFILL = 2e-5

# flash_attn_bhwd (tests/test_gpu_flash_attn.py): the output is the 16-bit rounding of an fp32
# evaluation, so it must lie within half a unit in the last place of the float64 oracle plus the
# fp32 evaluation's own error.  That error is bounded by the P hi + lo split (2^-18 of max|v| for
# bf16, 2^-22 for fp16) plus fp32 accumulation over <= 1500 keys (~2^-24 * sqrt(T)): ~5e-6 of
# max|v|, held here at 2e-5 of max|v|.  (The reference's Triton kernel evaluates q k^T and P V
# with TF32 dots, ~1e-3 relative; this bound is tighter than the reference's own accuracy.)
FLASH_ATTN_ABS = 2e-5
