"""Text-level generators with the reference's API (csrc/megakernel/megakernel_generators.py:12-128).

- `MegakernelGenerator(model_name, max_seq_len)` feeds the prompt through decode steps, then
  decodes greedily (:12-64).
- `MegakernelPrefillGenerator(model_name, max_seq_len, max_prefill_len)` runs the prompt through
  the MFMA prefill, then decodes (:67-128). It adds `prefill_only(prompt) -> (next_token,
  position)`.
- `MegakernelFusedPrefillGenerator` is the reference's small-prompt generator (default
  `max_prefill_len=64`, megakernel_generators.py:131-190). Its decoder,
  `MegakernelFusedPrefillDecoder`, runs prompts of up to 64 tokens through the fused prefill
  (`mq_prefill_fused`: one cooperative launch with the reference prefill megakernel's fp32
  activations) and longer ones, when max_prefill_len allows them, through the multi-kernel MFMA
  prefill.

Generation stops at a stop token (the tokenizer's EOS by default), after `max_new_tokens`, or
when the position reaches `max_seq_len - 1`, as the reference's loops do. `temperature` is
accepted and ignored: the reference decodes greedily too.

`model_name` is resolved by `megaqwen_amd.weights.load_qwen3_weights`: a local checkpoint
directory, or "random[:seed]" for seeded random-init weights.
"""
from __future__ import annotations

import torch

from .decoder import MegakernelDecoder, MegakernelFusedPrefillDecoder, MegakernelPrefillDecoder
from .spec import get_active_model_spec
from .weights import load_qwen3_weights


def _decoder_args(weights: dict, max_seq_len: int) -> tuple:
    return (weights["embed_weight"], weights["layer_weights"], weights["final_norm_weight"],
            weights["lm_head_weight"], weights["cos_table"], weights["sin_table"],
            int(get_active_model_spec()["num_layers"]), int(max_seq_len))


class MegakernelGenerator:
    """Prompt through decode steps, then greedy decode (megakernel_generators.py:12-64)."""

    def __init__(self, model_name="Qwen/Qwen3-0.6B", max_seq_len=2048):
        weights = load_qwen3_weights(model_name, max_seq_len=max_seq_len)
        self.decoder = MegakernelDecoder(*_decoder_args(weights, max_seq_len))
        self.tokenizer = weights["tokenizer"]
        self.max_seq_len = int(max_seq_len)

    def _stops(self, stop_tokens):
        return set(stop_tokens) if stop_tokens else {self.tokenizer.eos_token_id}

    def _tokens(self, prompt, max_new_tokens, stop_tokens):
        self.decoder.reset()
        ids = self.tokenizer.encode(prompt, add_special_tokens=True)
        for t in ids[:-1]:
            self.decoder.decode_step(t)
        stops = self._stops(stop_tokens)
        cur = ids[-1]
        for _ in range(int(max_new_tokens)):
            nxt = self.decoder.decode_step(cur)
            if nxt in stops:
                return
            yield nxt
            cur = nxt
            if self.decoder.position() >= self.max_seq_len - 1:
                return

    def generate(self, prompt, max_new_tokens=100, temperature=1.0, stop_tokens=None):
        out = list(self._tokens(prompt, max_new_tokens, stop_tokens))
        return self.tokenizer.decode(out, skip_special_tokens=True)

    def generate_stream(self, prompt, max_new_tokens=100, stop_tokens=None):
        for t in self._tokens(prompt, max_new_tokens, stop_tokens):
            yield self.tokenizer.decode([t])


class MegakernelPrefillGenerator:
    """Prefill the prompt, then greedy decode (megakernel_generators.py:67-128)."""

    _decoder_cls = MegakernelPrefillDecoder

    def __init__(self, model_name="Qwen/Qwen3-0.6B", max_seq_len=2048, max_prefill_len=512):
        weights = load_qwen3_weights(model_name, max_seq_len=max_seq_len)
        self.decoder = self._decoder_cls(*_decoder_args(weights, max_seq_len), max_prefill_len)
        self.tokenizer = weights["tokenizer"]
        self.max_seq_len = int(max_seq_len)
        self.max_prefill_len = int(max_prefill_len)

    def _tokenize(self, prompt):
        ids = self.tokenizer.encode(prompt, add_special_tokens=True)
        if len(ids) > self.max_prefill_len:
            raise ValueError(f"Prompt length {len(ids)} exceeds max prefill length "
                             f"{self.max_prefill_len}")
        return ids

    def _tokens(self, prompt, max_new_tokens, stop_tokens):
        self.decoder.reset()
        nxt = self.decoder.prefill_step(torch.tensor(self._tokenize(prompt), dtype=torch.int32))
        stops = set(stop_tokens) if stop_tokens else {self.tokenizer.eos_token_id}
        for _ in range(int(max_new_tokens)):
            if nxt in stops:
                return
            yield nxt
            if self.decoder.position() >= self.max_seq_len - 1:
                return
            nxt = self.decoder.decode_step(nxt)

    def generate(self, prompt, max_new_tokens=100, stop_tokens=None):
        out = list(self._tokens(prompt, max_new_tokens, stop_tokens))
        return self.tokenizer.decode(out, skip_special_tokens=True)

    def generate_stream(self, prompt, max_new_tokens=100, stop_tokens=None):
        for t in self._tokens(prompt, max_new_tokens, stop_tokens):
            yield self.tokenizer.decode([t])

    def prefill_only(self, prompt):
        self.decoder.reset()
        nxt = self.decoder.prefill_step(torch.tensor(self._tokenize(prompt), dtype=torch.int32))
        return nxt, self.decoder.position()


class MegakernelFusedPrefillGenerator(MegakernelPrefillGenerator):
    """The reference's small-prompt generator (megakernel_generators.py:131-190): prompts of up
    to 64 tokens run the fused prefill (`mq_prefill_fused`) of MegakernelFusedPrefillDecoder."""

    _decoder_cls = MegakernelFusedPrefillDecoder

    def __init__(self, model_name="Qwen/Qwen3-0.6B", max_seq_len=2048, max_prefill_len=64):
        super().__init__(model_name, max_seq_len=max_seq_len, max_prefill_len=max_prefill_len)
