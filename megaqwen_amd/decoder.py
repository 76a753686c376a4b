"""Decoder objects with the reference's binding surface, running on libmegaqwen_hip.so.

* `MegakernelDecoder` mirrors the pybind class of csrc/megakernel/bindings_decode.cpp:80-280:
  constructor `(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table,
  sin_table, num_layers, max_seq_len)`, `decode_step(int) -> int` (synchronous), `reset()`,
  `position()`.
* `MegakernelPrefillDecoder` mirrors csrc/megakernel/bindings_prefill.cpp:302-1701:
  `prefill_step(int32 tensor) -> int`, `decode_step`, `decode_steps(first, n) -> cpu int32[n]`,
  `decode_steps_cuda(first, n) -> device int32[n]`, `decode_steps_cuda_graph(first, n)`,
  `decode_greedy_cuda(first, max_new_tokens, eos_ids, chunk=32) -> (int32[k], k, stop_code)`,
  `reset()`, `position()`, `get_k_cache()`, `get_v_cache()`.

Both also expose `decode_step_with_logits(int) -> (int, fp32[vocab])`, the per-step logits hook
of chat.py's `decode_ldg_with_logits` (chat.py:241-314).

The KV caches and the workspace are torch tensors owned by the Python object (the reference's
C++ object owns its caches, bindings_decode.cpp:127-158); the library handle only points at
them.  Weights must be contiguous bf16 CUDA tensors; references to them are kept alive.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .spec import COMPILED_LAYER_SHAPE

_NKV, _D = COMPILED_LAYER_SHAPE["num_kv_heads"], COMPILED_LAYER_SHAPE["head_dim"]


def _stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


class _PrefillLimit(int):
    """An int that can also be called: `dec.max_prefill_len` reads it as an attribute and
    `dec.max_prefill_len()` as the method of the reference's fused-prefill decoder
    (bindings_fused_prefill.cpp:536)."""

    def __call__(self) -> int:
        return int(self)


def _bf16_cuda(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA tensor")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")
    return t.contiguous()


class MegakernelDecoder:
    """Batch-1 greedy decoder (bindings_decode.cpp:80-280) over the HIP decode kernels."""

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight,
                 cos_table, sin_table, num_layers, max_seq_len, max_prefill_len=0, *,
                 k_cache=None, v_cache=None):
        lib = _lib.load()
        self._lib = lib
        num_layers, max_seq_len = int(num_layers), int(max_seq_len)
        if len(layer_weights_flat) != 11 * num_layers:
            raise ValueError(f"expected {11 * num_layers} layer tensors, got {len(layer_weights_flat)}")
        self.embed_weight = _bf16_cuda(embed_weight, "embed_weight")
        self.final_norm_weight = _bf16_cuda(final_norm_weight, "final_norm_weight")
        self.lm_head_weight = _bf16_cuda(lm_head_weight, "lm_head_weight")
        self.cos_table = _bf16_cuda(cos_table, "cos_table")
        self.sin_table = _bf16_cuda(sin_table, "sin_table")
        self.layer_weights = [_bf16_cuda(t, f"layer_weights[{i}]") for i, t in enumerate(layer_weights_flat)]
        vocab, hidden = self.embed_weight.shape
        if self.cos_table.shape[0] < max_seq_len or self.sin_table.shape[0] < max_seq_len:
            raise ValueError("RoPE tables must cover max_seq_len positions")
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.max_prefill_len = _PrefillLimit(int(max_prefill_len))
        self.vocab_size = int(vocab)
        device = self.embed_weight.device

        layers = (_lib.LayerWeights * num_layers)()
        for l in range(num_layers):
            ptrs = [t.data_ptr() for t in self.layer_weights[11 * l:11 * (l + 1)]]
            layers[l] = _lib.LayerWeights(*ptrs)
        w = self.layer_weights
        if num_layers > 0:
            shape = dict(intermediate_size=int(w[8].shape[0]),
                         num_q_heads=int(w[1].shape[0]) // int(w[4].shape[0]),
                         num_kv_heads=int(w[2].shape[0]) // int(w[5].shape[0]),
                         head_dim=int(w[4].shape[0]))
        else:
            shape = {k: COMPILED_LAYER_SHAPE[k] for k in
                     ("intermediate_size", "num_q_heads", "num_kv_heads", "head_dim")}
        self._desc = _lib.ModelDesc(
            hidden_size=int(hidden), **shape,
            num_layers=num_layers, vocab_size=int(vocab), max_seq_len=max_seq_len,
            max_prefill_len=self.max_prefill_len, embed=self.embed_weight.data_ptr(),
            final_norm=self.final_norm_weight.data_ptr(), lm_head=self.lm_head_weight.data_ptr(),
            cos_table=self.cos_table.data_ptr(), sin_table=self.sin_table.data_ptr(),
            layers=layers)
        self._layers_keepalive = layers
        ws_bytes = lib.mq_workspace_bytes(ctypes.byref(self._desc))
        if ws_bytes == 0:
            raise _lib.MegaQwenError(_lib.MQ_ERR_INVALID_ARG, lib.mq_last_error().decode())
        cache_shape = (max(num_layers, 1), _NKV, max_seq_len, _D)
        if (k_cache is None) != (v_cache is None):
            raise ValueError("pass both k_cache and v_cache, or neither")
        if k_cache is None:
            self.k_cache = torch.zeros(cache_shape, dtype=torch.bfloat16, device=device)
            self.v_cache = torch.zeros_like(self.k_cache)
        else:
            # caller-owned caches (chat.py:409-421): [layers, kv_heads, max_seq_len, head_dim]
            for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
                if (not isinstance(c, torch.Tensor) or not c.is_cuda or c.dtype != torch.bfloat16
                        or not c.is_contiguous() or c.numel() < num_layers * _NKV * max_seq_len * _D
                        or c.shape[-2:] != (max_seq_len, _D)):
                    raise ValueError(f"{name} must be a contiguous bf16 CUDA tensor of shape "
                                     f"[{num_layers}, {_NKV}, {max_seq_len}, {_D}]")
            self.k_cache, self.v_cache = k_cache, v_cache
        self._workspace = torch.zeros((ws_bytes + 255) // 256 * 64, dtype=torch.int32, device=device)
        assert self._workspace.data_ptr() % 256 == 0
        self._tok = torch.zeros(2, dtype=torch.int32, device=device)
        self._logits = None
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        _lib.check(lib.mq_decoder_create(ctypes.byref(self._desc), self.k_cache.data_ptr(),
                                         self.v_cache.data_ptr(), self._workspace.data_ptr(),
                                         ws_bytes, ctypes.byref(handle)))
        self._h = handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.mq_decoder_destroy(h)
            self._h = None

    # ------------------------------------------------------------------ reference surface
    def _check_token(self, token_id: int) -> int:
        t = int(token_id)
        if not 0 <= t < self.vocab_size:
            raise ValueError(f"token id {t} outside [0, {self.vocab_size})")
        return t

    def decode_step(self, input_token_id: int) -> int:
        """One greedy step; returns the next token id (bindings_decode.cpp:193-234)."""
        self._tok[0].fill_(self._check_token(input_token_id))
        _lib.check(self._lib.mq_decode_step(self._h, self._tok.data_ptr(), self._tok.data_ptr() + 4,
                                            None, _stream_ptr()))
        return int(self._tok[1].item())

    def decode_step_with_logits(self, input_token_id: int):
        """(next token, fp32 logits [vocab]) — chat.py's decode_ldg_with_logits (:241-314)."""
        if self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        self._tok[0].fill_(self._check_token(input_token_id))
        _lib.check(self._lib.mq_decode_step(self._h, self._tok.data_ptr(), self._tok.data_ptr() + 4,
                                            self._logits.data_ptr(), _stream_ptr()))
        return int(self._tok[1].item()), self._logits.clone()

    def debug_decode_step_layers(self, input_token_id: int):
        """(next token, fp32 logits [vocab], hidden state after every layer [num_layers, H]);
        the per-layer counterpart of the reference's debug_ldg_decode_cycles hook."""
        if self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        trace = torch.empty(self.num_layers, self.embed_weight.shape[1], dtype=torch.float32,
                            device=self._tok.device)
        self._tok[0].fill_(self._check_token(input_token_id))
        _lib.check(self._lib.mq_debug_decode_step_layers(
            self._h, self._tok.data_ptr(), self._tok.data_ptr() + 4, self._logits.data_ptr(),
            trace.data_ptr(), _stream_ptr()))
        return int(self._tok[1].item()), self._logits.clone(), trace

    def debug_decode_step_timing(self, input_token_id: int):
        """(next token, int64 [grid, num_layers, 11] 100 MHz stage timestamps) of one persistent
        decode step — the counterpart of the reference's debug_ldg_decode_cycles."""
        stamps = torch.zeros(self.grid, self.num_layers, 11, dtype=torch.int64,
                             device=self._tok.device)
        self._tok[0].fill_(self._check_token(input_token_id))
        _lib.check(self._lib.mq_debug_decode_step_timing(
            self._h, self._tok.data_ptr(), self._tok.data_ptr() + 4, stamps.data_ptr(),
            _stream_ptr()))
        return int(self._tok[1].item()), stamps

    # stage columns of the reference's debug_ldg_decode_cycles (fused_decode_ldg_common.inl:51-69)
    # filled from this kernel's phases; the stages it fuses (the input RMSNorm into the q|k|v
    # GEMV, the q/k norm + RoPE into attention, the post norm into gate|up) read 0
    _CYCLE_COLUMNS = (2, 3, 6, 7, 8, 9, 12, 13, 14, 15)

    def debug_ldg_decode_cycles(self, input_token_id: int) -> torch.Tensor:
        """One persistent decode step with stage timing, as the reference's
        debug_ldg_decode_cycles (bindings_prefill.cpp:980-1043): an int64 CUDA tensor
        [grid, num_layers, 16] of per-workgroup stage durations in the reference's stage columns
        (MATVEC_QKV, MATVEC_SYNC2, ATTN, ATTN_SYNC, OPROJ_RESID, OPROJ_SYNC, GATE_UP,
        GATE_UP_SYNC, DOWNPROJ, DOWNPROJ_SYNC).  Durations are in ticks of the 100 MHz
        constant-rate clock (10 ns), not shader cycles."""
        _, stamps = self.debug_decode_step_timing(input_token_id)
        d = stamps[..., 1:] - stamps[..., :-1]
        out = torch.zeros(stamps.shape[0], stamps.shape[1], 16, dtype=torch.int64,
                          device=stamps.device)
        out[..., list(self._CYCLE_COLUMNS)] = d
        return out

    def debug_set_exchange_epoch(self, xep: int) -> None:
        """Sets the exchange-epoch base of the persistent kernel's cross-workgroup words (in
        stream order), e.g. just below the wrap of the epoch count; results do not depend on it."""
        _lib.check(self._lib.mq_debug_set_exchange_epoch(self._h, int(xep), _stream_ptr()))

    def debug_exchange_epoch(self) -> int:
        """The current exchange-epoch base (synchronises the stream)."""
        v = ctypes.c_uint32()
        _lib.check(self._lib.mq_debug_get_exchange_epoch(self._h, ctypes.byref(v), _stream_ptr()))
        return int(v.value)

    def set_position(self, position: int) -> None:
        """Moves the decode position (host and device) without touching the KV cache; the
        chat.py binding passes the position with every call (chat.py:448-470)."""
        _lib.check(self._lib.mq_decoder_set_position(self._h, int(position), _stream_ptr()))

    def reset(self) -> None:
        """Zeroes the KV cache and sets the position to 0 (bindings_decode.cpp:236-240)."""
        _lib.check(self._lib.mq_decoder_reset(self._h, _stream_ptr()))

    def position(self) -> int:
        return int(self._lib.mq_decoder_position(self._h))

    # ------------------------------------------------------------------ extras
    def check(self) -> None:
        """Synchronises and raises if a kernel flagged an error (barrier time-out, bad input)."""
        _lib.check(self._lib.mq_decoder_check(self._h, _stream_ptr()))

    def set_mode(self, mode: str) -> None:
        """'persistent' (one cooperative kernel per token) or 'multi_kernel'."""
        m = {"persistent": _lib.MQ_MODE_PERSISTENT, "multi_kernel": _lib.MQ_MODE_MULTI_KERNEL}[mode]
        _lib.check(self._lib.mq_decoder_set_mode(self._h, m))

    @property
    def mode(self) -> str:
        return {0: "persistent", 1: "multi_kernel"}.get(self._lib.mq_decoder_get_mode(self._h), "?")

    @property
    def grid(self) -> int:
        return int(self._lib.mq_decoder_grid(self._h))

    def get_k_cache(self) -> torch.Tensor:
        return self.k_cache

    def get_v_cache(self) -> torch.Tensor:
        return self.v_cache

    # -------------------------------------------- op-level entry points (per-op microbenchmarks)
    def op_qkv_rope(self, layer: int, x: torch.Tensor, pos: int, q_out: torch.Tensor | None = None):
        """RMSNorm + q|k|v GEMV + q/k norm + RoPE at `pos`; K/V rows land in the cache."""
        x = _bf16_cuda(x, "x")
        if q_out is None:
            q_out = torch.empty(16 * _D, dtype=torch.float32, device=x.device)
        _lib.check(self._lib.mq_op_qkv_rope(self._h, int(layer), x.data_ptr(), int(pos),
                                            q_out.data_ptr(), _stream_ptr()))
        return q_out

    def op_attention(self, layer: int, q: torch.Tensor, cache_len: int,
                     out: torch.Tensor | None = None):
        """GQA attention of rotated queries over cache rows [0, cache_len)."""
        assert q.dtype == torch.float32 and q.is_cuda and q.numel() == 16 * _D
        if out is None:
            out = torch.empty(16 * _D, dtype=torch.float32, device=q.device)
        _lib.check(self._lib.mq_op_attention(self._h, int(layer), q.contiguous().data_ptr(),
                                             int(cache_len), out.data_ptr(), _stream_ptr()))
        return out

    def op_mlp(self, layer: int, a: torch.Tensor, x_out: torch.Tensor | None = None):
        """bf16(W_down(silu(W_gate n) * W_up n) + a), n = RMSNorm(a)."""
        assert a.dtype == torch.float32 and a.is_cuda
        if x_out is None:
            x_out = torch.empty(a.numel(), dtype=torch.bfloat16, device=a.device)
        _lib.check(self._lib.mq_op_mlp(self._h, int(layer), a.contiguous().data_ptr(),
                                       x_out.data_ptr(), _stream_ptr()))
        return x_out

    def op_decode_layer(self, layer: int, x: torch.Tensor, pos: int,
                        x_out: torch.Tensor | None = None) -> torch.Tensor:
        """One decoder layer at `pos` (generate.py:78-110): bf16 [1024] in -> bf16 [1024] out;
        writes KV row `pos` of `layer`, attends over rows [0, pos]."""
        x = _bf16_cuda(x, "x").reshape(-1)
        if x.numel() != 1024:
            raise ValueError("x must hold 1024 elements")
        if x_out is None:
            x_out = torch.empty_like(x)
        _lib.check(self._lib.mq_op_decode_layer(self._h, int(layer), x.data_ptr(), int(pos),
                                                x_out.data_ptr(), _stream_ptr()))
        return x_out

    def op_lm_head(self, x: torch.Tensor, tok_out: torch.Tensor | None = None,
                   logits: torch.Tensor | None = None):
        """Final RMSNorm + LM head (+ logits) + argmax of a bf16 hidden state."""
        x = _bf16_cuda(x, "x")
        if tok_out is None:
            tok_out = torch.empty(1, dtype=torch.int32, device=x.device)
        _lib.check(self._lib.mq_op_lm_head(self._h, x.data_ptr(), tok_out.data_ptr(),
                                           None if logits is None else logits.data_ptr(),
                                           _stream_ptr()))
        return tok_out


class MegakernelPrefillDecoder(MegakernelDecoder):
    """Prefill + decode object of bindings_prefill.cpp:302-1701 (coop decode backend)."""

    _W4_ARGS = tuple(f"split_{m}_w4_{k}" for m in ("q", "k", "v", "o", "gateup", "down")
                     for k in ("packed", "scales", "codebook"))

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight,
                 cos_table, sin_table, num_layers, max_seq_len, max_prefill_len=512, **kwargs):
        for k, v in kwargs.items():
            if k not in self._W4_ARGS:
                raise TypeError(f"unexpected argument {k!r}")
            if v:
                raise NotImplementedError("W4 split-GEMM weights are not supported")
        super().__init__(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight,
                         cos_table, sin_table, num_layers, max_seq_len,
                         max_prefill_len=max_prefill_len)
        self._graph = None
        self._graph_steps = 0
        self._graph_tokens = None
        self._graph_failed = set()     # step counts whose capture failed (not retried)

    def prefill_step(self, input_token_ids) -> int:
        """Prefill positions 0..n-1, return the greedy next token, set position = n
        (bindings_prefill.cpp:731-833; errors as :734-739)."""
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_prefill_len:
            raise RuntimeError(f"Prefill sequence length {n} exceeds maximum {self.max_prefill_len}")
        if int(toks.min()) < 0 or int(toks.max()) >= self.vocab_size:
            raise ValueError("token id outside the vocabulary")
        d = toks.to(device=self._tok.device, dtype=torch.int32).contiguous()
        _lib.check(self._lib.mq_prefill(self._h, d.data_ptr(), n, self._tok.data_ptr() + 4, None,
                                        _stream_ptr()))
        return int(self._tok[1].item())

    def prefill_asr(self, input_token_ids, audio_embeds, audio_start_idx: int, *,
                    return_logits: bool = False):
        """Prefill whose embedding rows [audio_start_idx, audio_start_idx + audio_len) are the
        caller's bf16 `audio_embeds` [audio_len, 1024] (bindings_prefill.cpp:835-955); returns
        the greedy next token (with the last position's fp32 logits if return_logits) and sets
        position = n.  Errors as the reference's checks."""
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if n > self.max_prefill_len:
            raise RuntimeError("Prefill sequence length exceeds maximum")
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if (not isinstance(audio_embeds, torch.Tensor) or not audio_embeds.is_cuda
                or audio_embeds.dtype != torch.bfloat16 or audio_embeds.dim() != 2):
            raise RuntimeError("audio_embeds must be a CUDA bfloat16 2D tensor [audio_len, hidden_size]")
        audio_len, hidden = int(audio_embeds.shape[0]), int(audio_embeds.shape[1])
        if hidden != 1024:
            raise RuntimeError("audio_embeds hidden_size mismatch with compiled megakernel spec: "
                               f"expected=1024, got={hidden}")
        if audio_len <= 0:
            raise RuntimeError("audio_embeds must have audio_len > 0")
        start = int(audio_start_idx)
        if start < 0 or start + audio_len > n:
            raise RuntimeError("Invalid audio_start_idx/audio_len for the given seq_len")
        if int(toks.min()) < 0 or int(toks.max()) >= self.vocab_size:
            raise ValueError("token id outside the vocabulary")
        d = toks.to(device=self._tok.device, dtype=torch.int32).contiguous()
        emb = audio_embeds.contiguous()
        if return_logits and self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        lg = self._logits.data_ptr() if return_logits else None
        _lib.check(self._lib.mq_prefill_embeds(self._h, d.data_ptr(), n, emb.data_ptr(), start,
                                               audio_len, self._tok.data_ptr() + 4, lg,
                                               _stream_ptr()))
        tok = int(self._tok[1].item())
        return (tok, self._logits.clone()) if return_logits else tok

    def prefill_step_with_logits(self, input_token_ids):
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        if self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        d = toks.to(device=self._tok.device, dtype=torch.int32).contiguous()
        n = int(d.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        _lib.check(self._lib.mq_prefill(self._h, d.data_ptr(), n, self._tok.data_ptr() + 4,
                                        self._logits.data_ptr(), _stream_ptr()))
        return int(self._tok[1].item()), self._logits.clone()

    def debug_prefill_layers(self, input_token_ids):
        """prefill_step that also returns the residual stream after every layer:
        (next token, fp32 logits [vocab], bf16 [num_layers, n, hidden])."""
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_prefill_len:
            raise RuntimeError(f"Prefill sequence length {n} exceeds maximum {self.max_prefill_len}")
        if self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        d = toks.to(device=self._tok.device, dtype=torch.int32).contiguous()
        trace = torch.empty(max(self.num_layers, 1), n, self.embed_weight.shape[1],
                            dtype=torch.bfloat16, device=self._tok.device)
        _lib.check(self._lib.mq_debug_prefill_layers(self._h, d.data_ptr(), n,
                                                     self._tok.data_ptr() + 4,
                                                     self._logits.data_ptr(), trace.data_ptr(),
                                                     _stream_ptr()))
        return int(self._tok[1].item()), self._logits.clone(), trace[:self.num_layers]

    def debug_prefill_buffers(self, n: int) -> dict:
        """Views (bf16) of the prefill buffers after a prefill of n tokens: h, xn, qkv, att, mlp
        (the last layer's values)."""
        ptrs = (ctypes.c_void_p * 5)()
        _lib.check(self._lib.mq_debug_prefill_buffers(self._h, ptrs))
        base = self._workspace.data_ptr()
        raw = self._workspace.view(torch.uint8)
        widths = {"h": 1024, "xn": 1024, "qkv": 4096, "att": 2048, "mlp": 3072}
        out = {}
        for (name, width), ptr in zip(widths.items(), ptrs):
            off = int(ptr) - base
            out[name] = raw[off:off + n * width * 2].view(torch.bfloat16).view(n, width)
        return out

    def _chain(self, first_token_id: int, num_steps: int) -> torch.Tensor:
        if self.position() + num_steps >= self.max_seq_len:
            raise RuntimeError("decode_steps would exceed max_seq_len")
        toks = torch.empty(num_steps + 1, dtype=torch.int32, device=self._tok.device)
        toks[0] = self._check_token(first_token_id)
        _lib.check(self._lib.mq_decode_steps(self._h, toks.data_ptr(), num_steps, _stream_ptr()))
        return toks

    def decode_steps_cuda(self, first_token_id: int, num_steps: int) -> torch.Tensor:
        """Chained decode on the device; returns the generated tokens (bindings_prefill.cpp
        :1045-1075)."""
        if num_steps <= 0:
            return torch.empty(0, dtype=torch.int32, device=self._tok.device)
        return self._chain(first_token_id, int(num_steps))[1:]

    def decode_steps(self, first_token_id: int, num_steps: int) -> torch.Tensor:
        return self.decode_steps_cuda(first_token_id, num_steps).cpu()

    @property
    def graph_captured(self) -> bool:
        """Whether the last decode_steps_cuda_graph call replayed a captured graph."""
        return self._graph is not None

    def decode_steps_cuda_graph(self, first_token_id: int, num_steps: int) -> torch.Tensor:
        """decode_steps_cuda replayed from a captured HIP graph (rebuilt when num_steps changes;
        bindings_prefill.cpp:1082-1150).  Falls back to the eager chain if capture fails; a step
        count whose capture failed is not captured again (graph_captured tells which ran)."""
        num_steps = int(num_steps)
        if num_steps <= 0:
            return torch.empty(0, dtype=torch.int32, device=self._tok.device)
        if self.position() + num_steps >= self.max_seq_len:
            raise RuntimeError("decode_steps_cuda_graph would exceed max_seq_len")
        if self._graph is None or self._graph_steps != num_steps:
            if num_steps in self._graph_failed or not self._capture(num_steps):
                self._graph_failed.add(num_steps)
                self._graph = None
                return self.decode_steps_cuda(first_token_id, num_steps)
        self._graph_tokens[0] = self._check_token(first_token_id)
        self._graph.replay()
        self._advance_host_position(num_steps)
        return self._graph_tokens[1:].clone()

    def _capture(self, num_steps: int) -> bool:
        dev = self._tok.device
        toks = torch.zeros(num_steps + 1, dtype=torch.int32, device=dev)
        g = torch.cuda.CUDAGraph()
        pos0 = self.position()
        try:
            torch.cuda.synchronize(dev)
            with torch.cuda.graph(g):
                rc = self._lib.mq_decode_steps(self._h, toks.data_ptr(), num_steps, _stream_ptr())
            _lib.check(rc)
        except Exception:
            self._graph = None
            self._set_host_position(pos0)
            return False
        # capture advanced the host position counter without running anything
        self._set_host_position(pos0)
        self._graph, self._graph_steps, self._graph_tokens = g, num_steps, toks
        return True

    def _set_host_position(self, pos: int) -> None:
        _lib.check(self._lib.mq_decoder_set_host_position(self._h, int(pos)))

    def _advance_host_position(self, n: int) -> None:
        self._set_host_position(self.position() + int(n))

    def decode_greedy_cuda(self, first_token_id: int, max_new_tokens: int, eos_ids, chunk: int = 32,
                           *, scan_chunk_tail: bool = False):
        """GPU-resident greedy loop with a chunked EOS scan (bindings_prefill.cpp:1159-1349,
        its default coop backend).  Returns (tokens int32[k] on the device, k, stop_code) where
        tokens[0] is the first token and tokens[i] the token fed to step i.

        Each chunk of `steps` decode steps feeds toks[0] (the previous chunk's last output, or
        the first token) and produces toks[1..steps]; toks[0..steps-1] are appended to the
        result.  As in the reference, only toks[1..steps-1] are scanned for an EOS id (none when
        steps == 1): the chunk's tail token toks[steps] becomes the next chunk's toks[0], which
        is emitted but never scanned, so an EOS produced as a chunk's last step does not stop
        generation, and on the final chunk the tail is not emitted at all.  On the first scanned
        EOS the result ends just before it (stop_code 1); otherwise after max_new_tokens entries
        (stop_code 0).  The position advances by every decoded step, as in the reference.

        scan_chunk_tail=True (not in the reference) also scans toks[steps], so the result is
        exactly the greedy sequence up to, not including, its first EOS after the first token."""
        max_new = int(max_new_tokens)
        if max_new <= 0:
            return torch.empty(0, dtype=torch.int32, device=self._tok.device), 0, 0
        if chunk <= 0:
            chunk = 32
        eos = torch.as_tensor(eos_ids, dtype=torch.int32).reshape(-1)
        if eos.numel() == 0:
            raise RuntimeError("eos_ids must be a non-empty int32 tensor")
        eos = eos.to(self._tok.device)
        out = torch.empty(max_new, dtype=torch.int32, device=self._tok.device)
        nxt = self._check_token(first_token_id)
        gen = 0
        while gen < max_new:
            steps = min(chunk, max_new - gen)
            toks = self._chain(nxt, steps)
            out[gen:gen + steps] = toks[:steps]
            end = steps + 1 if scan_chunk_tail else steps     # scanned: toks[1:end]
            hit = torch.isin(toks[1:end], eos).nonzero() if end > 1 else None
            gen += steps
            if hit is not None and hit.numel() > 0:
                first = int(hit[0, 0]) + 1          # index in toks of the EOS token
                kept = gen - steps + first
                return out[:kept], kept, 1
            nxt = int(toks[steps].item())
        return out[:gen], gen, 0


class MegakernelFusedPrefillDecoder(MegakernelPrefillDecoder):
    """The reference's short-prompt decoder class (bindings_fused_prefill.cpp:286-545; default
    max_prefill_len 64, `max_prefill_len()` a method).  Prompts of up to 64 tokens run the fused
    prefill (`mq_prefill_fused`: one cooperative launch with the prefill megakernel's fp32
    arithmetic, fused_prefill_megakernel_core.inl:658-745); a longer prompt, possible only with
    max_prefill_len > 64, runs the multi-kernel bf16 prefill of MegakernelPrefillDecoder."""

    FUSED_MAX = 64

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight,
                 cos_table, sin_table, num_layers, max_seq_len, max_prefill_len=64, **kwargs):
        super().__init__(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight,
                         cos_table, sin_table, num_layers, max_seq_len,
                         max_prefill_len=max_prefill_len, **kwargs)

    def _fused(self, toks, emb=None, start: int = 0, return_logits: bool = False):
        n = int(toks.numel())
        if return_logits and self._logits is None:
            self._logits = torch.empty(self.vocab_size, dtype=torch.float32, device=self._tok.device)
        d = toks.to(device=self._tok.device, dtype=torch.int32).contiguous()
        lg = self._logits.data_ptr() if return_logits else None
        _lib.check(self._lib.mq_prefill_fused(
            self._h, d.data_ptr(), n, emb.data_ptr() if emb is not None else None, start,
            int(emb.shape[0]) if emb is not None else 0, self._tok.data_ptr() + 4, lg,
            _stream_ptr()))
        tok = int(self._tok[1].item())
        return (tok, self._logits.clone()) if return_logits else tok

    def prefill_step(self, input_token_ids) -> int:
        """bindings_fused_prefill.cpp:235-283 (errors as :236-243)."""
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if n == 0 or n > min(self.FUSED_MAX, int(self.max_prefill_len)):
            return super().prefill_step(input_token_ids)
        if int(toks.min()) < 0 or int(toks.max()) >= self.vocab_size:
            raise ValueError("token id outside the vocabulary")
        return self._fused(toks)

    def prefill_step_with_logits(self, input_token_ids):
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if n == 0 or n > min(self.FUSED_MAX, int(self.max_prefill_len)):
            return super().prefill_step_with_logits(input_token_ids)
        return self._fused(toks, return_logits=True)

    def prefill_asr(self, input_token_ids, audio_embeds, audio_start_idx: int, *,
                    return_logits: bool = False):
        """bindings_fused_prefill.cpp:286-330; argument checks as the multi-kernel prefill_asr."""
        toks = torch.as_tensor(input_token_ids).reshape(-1)
        n = int(toks.numel())
        if (n == 0 or n > min(self.FUSED_MAX, int(self.max_prefill_len))
                or not isinstance(audio_embeds, torch.Tensor) or not audio_embeds.is_cuda
                or audio_embeds.dtype != torch.bfloat16 or audio_embeds.dim() != 2
                or int(audio_embeds.shape[1]) != 1024 or int(audio_embeds.shape[0]) <= 0
                or int(audio_start_idx) < 0
                or int(audio_start_idx) + int(audio_embeds.shape[0]) > n):
            # the multi-kernel path raises the reference's errors for bad arguments
            return super().prefill_asr(input_token_ids, audio_embeds, audio_start_idx,
                                       return_logits=return_logits)
        if int(toks.min()) < 0 or int(toks.max()) >= self.vocab_size:
            raise ValueError("token id outside the vocabulary")
        return self._fused(toks, audio_embeds.contiguous(), int(audio_start_idx), return_logits)
