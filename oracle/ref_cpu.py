"""CPU oracle for the Qwen3-0.6B decode/prefill hot path.  TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import this
module, and only as the checker / the timed CPU baseline.  The product path (`megaqwen_amd`)
never imports it.

It restates, in PyTorch-CPU fp32 (or fp64 with the same rounding points, to measure the fp32
evaluation's own spread), what the reference computes:

* decode step (`mode="decode"`): the persistent decode kernel of the reference,
  csrc/megakernel/fused_decode_ldg_kernel.inl:43-137 driving the phases in
  fused_decode_ldg_common.inl:131-262 (input RMSNorm + QKV GEMV),
  :268-394 (per-head q/k RMSNorm, rotate-half RoPE, bf16 K/V cache write),
  :417-602 (GQA attention over the bf16 cache, kv_head = qh / 2, scale 1/sqrt(D)),
  fused_decode_ldg_mlp.inl:5-218 (O GEMV + residual, post RMSNorm, SwiGLU, down GEMV +
  residual rounded to bf16) and fused_decode_ldg_lm.inl:47-163 (LM head argmax).
  Intermediates are fp32; rounding points are: the hidden state to bf16 at every layer end
  (fused_decode_ldg_mlp.inl:200), K and V to bf16 on the cache write
  (fused_decode_ldg_common.inl:376-377), cos/sin tables in bf16 (megakernel_weights.py:131-137).
* prefill (`prefill`): csrc/megakernel/fused_prefill_launch.inl:245-657 with the kernels in
  fused_prefill_kernels.inl:3-342,619-824: every GEMM output and every elementwise result is
  rounded to bf16 (normalized input, q/k/v, q/k after norm+RoPE, attention output, O, residual
  sums, post-norm, gate, up, silu*up, down); the last token's final norm is bf16 and the LM head
  argmax reads that bf16 vector.

`round_bf16=False` removes every rounding point (pure fp32 model): with fp32 RoPE tables this is
the model HuggingFace's `Qwen3ForCausalLM` computes in fp32, which is what the golden fixtures
under tests/golden pin (see tests/golden/make_golden.py).

Argmax ties resolve to the lowest index (torch.argmax on CPU returns the first maximal index).
The reference resolves ties by lowest block then lowest warp (fused_decode_ldg_lm.inl:86-121,
138-158), which coincides except for exact fp32 ties across interleaved rows.
"""
from __future__ import annotations

import math

import torch

EPS = 1e-6


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even to bf16, returned in x's dtype (as __float2bfloat16 then widening)."""
    return x.to(torch.bfloat16).to(x.dtype)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * w over the last dim, fp32.
    (fused_decode_ldg_common.inl:150-191; fused_prefill_kernels.inl:52-105)"""
    ms = (x * x).mean(dim=-1, keepdim=True)
    return x * torch.rsqrt(ms + eps) * w


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE on the last dim (fused_decode_ldg_common.inl:321-330,364-373):
    o_i = x_i c_i - x_{i+D/2} s_i for i < D/2, o_i = x_{i-D/2} s_i + x_i c_i otherwise."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2 = cos[..., :half], cos[..., half:]
    s1, s2 = sin[..., :half], sin[..., half:]
    return torch.cat([x1 * c1 - x2 * s1, x1 * s2 + x2 * c2], dim=-1)


def silu(x: torch.Tensor) -> torch.Tensor:
    """x / (1 + exp(-x)) (fused_decode_ldg_common.inl:123-125)."""
    return x / (1.0 + torch.exp(-x))


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Softmax attention of one query block against keys/values (fp32).
    q [Hq, n, D], k/v [Hq, L, D] (already expanded for GQA) -> [Hq, n, D].  No mask."""
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v)


class OracleModel:
    """CPU model over bf16-representable weights, in fp32 (the reference's arithmetic) or, with
    `dtype=torch.float64`, in fp64 with the same bf16 rounding points.  The fp64 evaluation
    measures how far the fp32 oracle's own rounding of sums moves its results (the spread the
    GPU tests' tolerances are set against); it is not a different model.

    weights: dict from megaqwen_amd.synthetic.make_weights (any float dtype; converted to `dtype`).
    cos/sin: [max_seq, D] tables (bf16 values as in the reference, or fp32 for the HF pin).
    """

    def __init__(self, weights: dict, spec: dict, cos: torch.Tensor, sin: torch.Tensor,
                 max_seq_len: int, round_bf16: bool = True, threads: int | None = None,
                 dtype: torch.dtype = torch.float32):
        if threads is not None:
            torch.set_num_threads(int(threads))
        if dtype not in (torch.float32, torch.float64):
            raise ValueError("dtype must be torch.float32 or torch.float64")
        self.dtype = dtype
        f = lambda t: t.to(dtype).contiguous()
        self.spec = dict(spec)
        self.H = int(spec["hidden_size"])
        self.I = int(spec["intermediate_size"])
        self.nq = int(spec["num_q_heads"])
        self.nkv = int(spec["num_kv_heads"])
        self.D = int(spec["head_dim"])
        self.L = int(spec["num_layers"])
        self.V = int(spec["vocab_size"])
        self.group = self.nq // self.nkv
        self.scale = 1.0 / math.sqrt(self.D)
        self.embed = f(weights["embed_weight"])
        self.lm_head = f(weights["lm_head_weight"])
        self.final_norm = f(weights["final_norm_weight"])
        flat = weights["layer_weights"]
        keys = ("input_ln", "q", "k", "v", "q_norm", "k_norm", "o", "post_ln", "gate", "up", "down")
        self.layers = [dict(zip(keys, [f(t) for t in flat[i * 11:(i + 1) * 11]])) for i in range(self.L)]
        self.cos = f(cos)
        self.sin = f(sin)
        self.max_seq_len = int(max_seq_len)
        self.round = bool(round_bf16)
        self.k_cache = torch.zeros(self.L, self.nkv, self.max_seq_len, self.D, dtype=dtype)
        self.v_cache = torch.zeros(self.L, self.nkv, self.max_seq_len, self.D, dtype=dtype)
        self.position = 0

    def _r(self, x: torch.Tensor) -> torch.Tensor:
        return bf16(x) if self.round else x

    def reset(self) -> None:
        """bindings_decode.cpp:236-240: zero the KV cache and set position 0."""
        self.k_cache.zero_()
        self.v_cache.zero_()
        self.position = 0

    # ------------------------------------------------------------------ decode
    def decode_layer(self, li: int, x: torch.Tensor, pos: int, write_kv: bool = True) -> torch.Tensor:
        """One decoder layer at position `pos` on the fp32 hidden state x [H] (bf16-valued):
        writes K/V row `pos` of layer li (unless `write_kv` is False, in which case the row
        already in the cache is used) and returns the layer output (rounded to bf16)."""
        w = self.layers[li]
        c, s = self.cos[pos], self.sin[pos]
        cache_len = pos + 1
        r = x
        n = rms_norm(r, w["input_ln"])
        q = w["q"] @ n
        k = w["k"] @ n
        v = w["v"] @ n
        q = rope(rms_norm(q.view(self.nq, self.D), w["q_norm"]), c, s)      # kept fp32
        k = rope(rms_norm(k.view(self.nkv, self.D), w["k_norm"]), c, s)
        if write_kv:
            self.k_cache[li, :, pos] = self._r(k)
            self.v_cache[li, :, pos] = self._r(v.view(self.nkv, self.D))
        K = self.k_cache[li, :, :cache_len].repeat_interleave(self.group, dim=0)
        Vv = self.v_cache[li, :, :cache_len].repeat_interleave(self.group, dim=0)
        att = attend(q.unsqueeze(1), K, Vv, self.scale).reshape(-1)
        a = w["o"] @ att + r
        n2 = rms_norm(a, w["post_ln"])
        m = silu(w["gate"] @ n2) * (w["up"] @ n2)
        return self._r(w["down"] @ m + a)

    def lm_head_logits(self, x: torch.Tensor) -> torch.Tensor:
        """Final RMSNorm (fp32) + tied LM head (fused_decode_ldg_kernel.inl:103-137,
        fused_decode_ldg_lm.inl:47-122)."""
        return self.lm_head @ rms_norm(x, self.final_norm)

    def decode_step(self, token: int, return_logits: bool = True):
        """One decode step at the current position; returns (next_token, logits fp32 [V])."""
        pos = self.position
        if pos >= self.max_seq_len:
            raise RuntimeError("decode position exceeds max_seq_len")
        x = self.embed[int(token)].clone()                  # bf16 row widened (kernel.inl:47-52)
        for li in range(self.L):
            x = self.decode_layer(li, x, pos)
        logits = self.lm_head_logits(x)
        self.position += 1
        tok = int(torch.argmax(logits).item())
        return (tok, logits) if return_logits else tok

    # ----------------------------------------------------------------- prefill
    def prefill(self, tokens, return_logits: bool = True, embeds=None, embeds_start: int = 0):
        """Prefill of `tokens` at positions 0..n-1 (fused_prefill_launch.inl:245-657).
        Writes K/V rows 0..n-1 and sets position = n (bindings_prefill.cpp:731-833).
        `embeds` [m, H] (bf16 values) replace the embedding rows [embeds_start, embeds_start + m)
        (prefill_asr, bindings_prefill.cpp:835-955; prefill_patch_audio_kernel,
        fused_prefill_kernels.inl:28-45)."""
        toks = torch.as_tensor(tokens, dtype=torch.long).reshape(-1)
        n = int(toks.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_seq_len:
            raise RuntimeError("Prefill sequence length exceeds maximum")
        R = self._r
        h = self.embed[toks].clone()                          # [n, H]
        if embeds is not None:
            e = torch.as_tensor(embeds).to(self.dtype).reshape(-1, h.shape[1])
            if e.shape[0] <= 0 or embeds_start < 0 or embeds_start + e.shape[0] > n:
                raise RuntimeError("Invalid audio_start_idx/audio_len for the given seq_len")
            h[embeds_start:embeds_start + e.shape[0]] = e
        for li in range(self.L):
            h = self.prefill_layer(li, h)
        hf = R(rms_norm(h[-1], self.final_norm))
        logits = self.lm_head @ hf
        self.position = n
        tok = int(torch.argmax(logits).item())
        return (tok, logits) if return_logits else tok

    def prefill_layer(self, li: int, h: torch.Tensor, fused: bool = False) -> torch.Tensor:
        """Prefill layer li on the residual stream h [n, H] (bf16 values) at positions 0..n-1
        (fused_prefill_launch.inl:245-657): writes K/V rows 0..n-1 of layer li and returns the
        layer output [n, H].  Every GEMM output and elementwise result is rounded to bf16.
        With `fused`, the prefill megakernel's arithmetic instead
        (fused_prefill_megakernel_core.inl:35-599): fp32 throughout, attention over the fp32
        normalised keys and values, and only the K/V cache rows rounded to bf16 (:313-315)."""
        R = (lambda x: x) if fused else self._r
        w = self.layers[li]
        n = int(h.shape[0])
        c, s = self.cos[:n].unsqueeze(1), self.sin[:n].unsqueeze(1)
        causal = torch.ones(n, n, dtype=torch.bool).tril()
        resid = h
        nrm = R(rms_norm(h, w["input_ln"]))
        q = R(nrm @ w["q"].T).view(n, self.nq, self.D)
        k = R(nrm @ w["k"].T).view(n, self.nkv, self.D)
        v = R(nrm @ w["v"].T).view(n, self.nkv, self.D)
        q = R(rope(rms_norm(q, w["q_norm"]), c, s))
        k = R(rope(rms_norm(k, w["k_norm"]), c, s))
        self.k_cache[li, :, :n] = bf16(k.transpose(0, 1)) if fused else k.transpose(0, 1)
        self.v_cache[li, :, :n] = bf16(v.transpose(0, 1)) if fused else v.transpose(0, 1)
        qh = q.transpose(0, 1)                                          # [nq, n, D]
        kh = k.transpose(0, 1).repeat_interleave(self.group, dim=0)     # [nq, n, D]
        vh = v.transpose(0, 1).repeat_interleave(self.group, dim=0)
        sc = torch.matmul(qh, kh.transpose(-1, -2)) * self.scale
        sc = sc.masked_fill(~causal, float("-inf"))
        att = torch.matmul(torch.softmax(sc, dim=-1), vh)               # [nq, n, D]
        att = R(att.transpose(0, 1).reshape(n, self.nq * self.D))
        o = R(att @ w["o"].T)
        h = R(o + resid)
        resid = h
        n2 = R(rms_norm(h, w["post_ln"]))
        g = R(n2 @ w["gate"].T)
        u = R(n2 @ w["up"].T)
        m = R(silu(g) * u)
        d = R(m @ w["down"].T)
        return R(d + resid)

    def prefill_fused(self, tokens, return_logits: bool = True, embeds=None,
                      embeds_start: int = 0):
        """The reference's prefill megakernel (prefill_megakernel,
        fused_prefill_megakernel_core.inl:658-745, MegakernelFusedPrefillDecoder.prefill_step /
        prefill_asr, bindings_fused_prefill.cpp:235-330): fp32 activations from the bf16
        embedding rows (:3-33, audio rows :693-703), prefill_layer(fused=True) per layer, then
        the fp32 final RMSNorm of the last position (:601-650) and the LM head.  Writes the
        bf16 K/V rows 0..n-1 and sets position = n."""
        toks = torch.as_tensor(tokens, dtype=torch.long).reshape(-1)
        n = int(toks.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_seq_len:
            raise RuntimeError("Prefill sequence length exceeds maximum")
        h = self.embed[toks].clone()
        if embeds is not None:
            e = torch.as_tensor(embeds).to(self.dtype).reshape(-1, h.shape[1])
            if e.shape[0] <= 0 or embeds_start < 0 or embeds_start + e.shape[0] > n:
                raise RuntimeError("Invalid audio_start_idx/audio_len for the given seq_len")
            h[embeds_start:embeds_start + e.shape[0]] = e
        for li in range(self.L):
            h = self.prefill_layer(li, h, fused=True)
        logits = self.lm_head @ rms_norm(h[-1], self.final_norm)
        self.position = n
        tok = int(torch.argmax(logits).item())
        return (tok, logits) if return_logits else tok

    def prefill_hidden_all(self, tokens):
        """fp32 logits for EVERY prompt position (no mutation of position semantics beyond
        prefill); used only to compare the pure-fp32 model with HuggingFace's full forward."""
        toks = torch.as_tensor(tokens, dtype=torch.long).reshape(-1)
        n = int(toks.numel())
        saved = self.round
        R = self._r
        h = self.embed[toks].clone()
        c, s = self.cos[:n].unsqueeze(1), self.sin[:n].unsqueeze(1)
        causal = torch.ones(n, n, dtype=torch.bool).tril()
        for w in self.layers:
            resid = h
            nrm = R(rms_norm(h, w["input_ln"]))
            q = R(nrm @ w["q"].T).view(n, self.nq, self.D)
            k = R(nrm @ w["k"].T).view(n, self.nkv, self.D)
            v = R(nrm @ w["v"].T).view(n, self.nkv, self.D)
            q = R(rope(rms_norm(q, w["q_norm"]), c, s))
            k = R(rope(rms_norm(k, w["k_norm"]), c, s))
            qh = q.transpose(0, 1)
            kh = k.transpose(0, 1).repeat_interleave(self.group, dim=0)
            vh = v.transpose(0, 1).repeat_interleave(self.group, dim=0)
            sc = torch.matmul(qh, kh.transpose(-1, -2)) * self.scale
            sc = sc.masked_fill(~causal, float("-inf"))
            att = R(torch.matmul(torch.softmax(sc, dim=-1), vh).transpose(0, 1).reshape(n, -1))
            h = R(R(att @ w["o"].T) + resid)
            resid = h
            n2 = R(rms_norm(h, w["post_ln"]))
            m = R(silu(R(n2 @ w["gate"].T)) * R(n2 @ w["up"].T))
            h = R(R(m @ w["down"].T) + resid)
        self.round = saved
        return R(rms_norm(h, self.final_norm)) @ self.lm_head.T
