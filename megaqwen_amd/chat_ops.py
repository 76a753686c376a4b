"""The two function-style binding surfaces of the reference, on libmegaqwen_hip.so.

`compile_kernel()` gives chat.py's inline extension (chat.py:123-321):
- `init_ldg_layer_weights(input_ln, q, k, v, q_norm, k_norm, o, post_ln, gate, up, down)`:
  eleven per-layer lists;
- `init_ldg_embed_weight(embed)`;
- `decode_ldg(token, final_norm, lm_head, cos, sin, k_cache, v_cache, <11 scratch tensors>,
  num_layers, position, cache_len, max_seq_len) -> int`;
- `decode_ldg_with_logits(...)`, with the same arguments, `-> (int, fp32[vocab])`.

The caller owns the KV caches `[layers, 8, max_seq_len, 128]` bf16, as in chat.py:409-421. The
decoder writes KV row `position` and attends over rows [0, position]. The eleven scratch tensors
(hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate,
g_normalized, block_max_vals, block_max_idxs) are accepted for signature compatibility and not
used. The decoder keeps its own workspace, whose layout the HIP kernels define.

`compile_kernels()` gives generate.py's per-layer extension (generate.py:78-143):
- `decode_layer(h, input_ln, q, k, v, q_norm, k_norm, o, post_ln, gate, up, down, cos, sin,
  k_cache, v_cache, position, cache_len, max_seq_len) -> h'`: bf16 [1024] in and out, with
  per-layer caches `[8, max_seq_len, 128]`;
- `lm_head_last(h, norm_weight, lm_weight) -> bf16 logits[vocab]` of the last row of `h`.

Both keep one library decoder per distinct set of device tensors (keyed by data pointers), so
repeated calls with the same tensors reuse it.
"""
from __future__ import annotations

import torch

from .decoder import MegakernelDecoder

_LAYER_LISTS = ("input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
                "post_attn_layernorm", "gate_proj", "up_proj", "down_proj")


def _ptrs(*ts) -> tuple:
    return tuple(int(t.data_ptr()) for t in ts)


class _ChatKernel:
    """chat.py's `ldg_kernel_chat` module (chat.py:123-321)."""

    def __init__(self):
        self._layers: list[torch.Tensor] | None = None
        self._embed: torch.Tensor | None = None
        self._dec: MegakernelDecoder | None = None
        self._key = None

    def init_ldg_layer_weights(self, *lists):
        if len(lists) != 11:
            raise TypeError("init_ldg_layer_weights takes 11 per-layer lists")
        n = len(lists[0])
        if any(len(x) != n for x in lists):
            raise ValueError("all 11 weight lists must have one tensor per layer")
        self._layers = [lists[j][i].contiguous() for i in range(n) for j in range(11)]
        self._dec = None

    def init_ldg_embed_weight(self, embed_weight: torch.Tensor):
        self._embed = embed_weight.contiguous()
        self._dec = None

    def _decoder(self, final_norm, lm_head, cos, sin, k_cache, v_cache, num_layers, max_seq_len):
        if self._layers is None or self._embed is None:
            raise RuntimeError("call init_ldg_layer_weights and init_ldg_embed_weight first")
        if len(self._layers) != 11 * int(num_layers):
            raise ValueError(f"num_layers {num_layers} != {len(self._layers) // 11} initialised layers")
        key = _ptrs(final_norm, lm_head, cos, sin, k_cache, v_cache) + (int(num_layers), int(max_seq_len))
        if self._dec is None or self._key != key:
            self._dec = MegakernelDecoder(self._embed, self._layers, final_norm, lm_head, cos, sin,
                                          num_layers, max_seq_len, k_cache=k_cache, v_cache=v_cache)
            self._key = key
        return self._dec

    def _prepare(self, args):
        (tok, final_norm, lm_head, cos, sin, k_cache, v_cache, *scratch) = args[:18]
        num_layers, position, cache_len, max_seq_len = (int(a) for a in args[18:22])
        if len(args) != 22:
            raise TypeError(f"decode_ldg takes 22 arguments ({len(args)} given)")
        if cache_len != position + 1:
            raise ValueError(f"cache_len {cache_len} must equal position + 1 = {position + 1}")
        dec = self._decoder(final_norm, lm_head, cos, sin, k_cache, v_cache, num_layers, max_seq_len)
        if dec.position() != position:
            dec.set_position(position)
        return dec, int(tok)

    def decode_ldg(self, *args) -> int:
        dec, tok = self._prepare(args)
        return dec.decode_step(tok)

    def decode_ldg_with_logits(self, *args):
        dec, tok = self._prepare(args)
        return dec.decode_step_with_logits(tok)


class _LayerKernels:
    """generate.py's `compile_kernels()` module (generate.py:78-143)."""

    def __init__(self):
        self._layer_decs: dict[tuple, MegakernelDecoder] = {}
        self._head_decs: dict[tuple, MegakernelDecoder] = {}

    @staticmethod
    def _dummies(device, max_seq_len=1):
        z = torch.zeros(1, 1024, dtype=torch.bfloat16, device=device)
        one = torch.ones(1024, dtype=torch.bfloat16, device=device)
        return z, one

    def decode_layer(self, hidden_states, input_layernorm_weight, q_proj_weight, k_proj_weight,
                     v_proj_weight, q_norm_weight, k_norm_weight, o_proj_weight,
                     post_attn_layernorm_weight, gate_proj_weight, up_proj_weight,
                     down_proj_weight, cos_table, sin_table, k_cache, v_cache, position,
                     cache_len, max_seq_len):
        ws = [input_layernorm_weight, q_proj_weight, k_proj_weight, v_proj_weight, q_norm_weight,
              k_norm_weight, o_proj_weight, post_attn_layernorm_weight, gate_proj_weight,
              up_proj_weight, down_proj_weight]
        if int(cache_len) != int(position) + 1:
            raise ValueError(f"cache_len {cache_len} must equal position + 1")
        key = _ptrs(*ws, cos_table, sin_table, k_cache, v_cache) + (int(max_seq_len),)
        dec = self._layer_decs.get(key)
        if dec is None:
            z, one = self._dummies(hidden_states.device)
            dec = MegakernelDecoder(z, [w.contiguous() for w in ws], one, z, cos_table, sin_table,
                                    1, int(max_seq_len), k_cache=k_cache, v_cache=v_cache)
            self._layer_decs[key] = dec
        return dec.op_decode_layer(0, hidden_states.reshape(-1), int(position))

    def lm_head_last(self, hidden_states, norm_weight, lm_weight):
        key = _ptrs(norm_weight, lm_weight)
        dec = self._head_decs.get(key)
        dev = lm_weight.device
        if dec is None:
            kv = torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16, device=dev)
            rope = torch.zeros(1, 128, dtype=torch.bfloat16, device=dev)
            dec = MegakernelDecoder(lm_weight, [], norm_weight, lm_weight, rope, rope, 0, 1,
                                    k_cache=kv, v_cache=kv.clone())
            self._head_decs[key] = dec
        h = hidden_states.reshape(-1, 1024)[-1].contiguous()
        logits = torch.empty(lm_weight.shape[0], dtype=torch.float32, device=dev)
        dec.op_lm_head(h, logits=logits)
        return logits.to(torch.bfloat16)


def compile_kernel() -> _ChatKernel:
    """chat.py:23-340 `compile_kernel()`; nothing is compiled at run time, the HIP library is
    prebuilt."""
    return _ChatKernel()


def compile_kernels() -> _LayerKernels:
    """generate.py:17-156 `compile_kernels()`."""
    return _LayerKernels()
