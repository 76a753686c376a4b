/* megaqwen_hip.h — C ABI of libmegaqwen_hip.so, the MI355X (gfx950) batch-1 Qwen3-0.6B
 * decode / prefill library.
 *
 * Plain C: device pointers are `void*` / typed pointers to device memory, streams are the
 * `hipStream_t` value passed as `void*` (NULL = default stream).  Every function returns
 * MQ_OK (0) or a negative MQ_ERR_* code; mq_last_error() describes the last failure of the
 * calling thread.  No function takes ownership of caller memory.
 *
 * Reference interfaces replaced (baicai-1145/MegaQwen, paths relative to its root):
 *   struct LDGLayerWeights ............ csrc/megakernel/fused_decode_ldg_common.inl:97-109
 *   MegakernelDecoder (ctor, decode_step, reset, position)
 *                                       csrc/megakernel/bindings_decode.cpp:80-280
 *   launch_ldg_decode / launch_ldg_decode_with_logits
 *                                       csrc/megakernel/fused_decode_ldg_launch.inl:55-364
 *   MegakernelPrefillDecoder.prefill_step / decode_steps_cuda
 *                                       csrc/megakernel/bindings_prefill.cpp:731-833,1045-1075
 *   launch_prefill_float .............. csrc/megakernel/fused_prefill_launch.inl:71-731
 *   launch_ldg_fill_iota / launch_ldg_find_first_eos (device token chain of decode_greedy_cuda)
 *                                       csrc/megakernel/fused_decode_ldg_launch.inl:5-53
 *   chat.py decode_ldg (caller-owned caches, host position per call) ... chat.py:123-321
 *   generate.py decode_layer / lm_head_last .............. generate.py:78-138
 */
#ifndef MEGAQWEN_HIP_H
#define MEGAQWEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_ABI_VERSION 1

#define MQ_OK 0
#define MQ_ERR_INVALID_ARG -1     /* null pointer, bad size, unsupported shape */
#define MQ_ERR_HIP -2             /* a HIP runtime call failed */
#define MQ_ERR_POSITION -3        /* position would exceed max_seq_len */
#define MQ_ERR_DEVICE -4          /* the kernel reported an error (wait time-out, bad input) */
#define MQ_ERR_UNSUPPORTED -5     /* e.g. cooperative launch not available for persistent mode */

/* Decode kernel organisation. */
#define MQ_MODE_PERSISTENT 0      /* one cooperative kernel per token (or chain of tokens); its phases
                                     hand values over as epoch- or tag-carrying words */
#define MQ_MODE_MULTI_KERNEL 1    /* one kernel launch per phase (launch boundaries order them) */

/* One layer's bf16 weights (row-major, contiguous), same order and meaning as the reference's
 * LDGLayerWeights (fused_decode_ldg_common.inl:97-109) and its 11-per-layer flat list
 * (megakernel_weights.py:109-128). */
typedef struct mq_layer_weights {
  const void* input_layernorm;     /* [H]            */
  const void* q_proj;              /* [Hq*D, H]      */
  const void* k_proj;              /* [Hkv*D, H]     */
  const void* v_proj;              /* [Hkv*D, H]     */
  const void* q_norm;              /* [D]            */
  const void* k_norm;              /* [D]            */
  const void* o_proj;              /* [H, Hq*D]      */
  const void* post_attn_layernorm; /* [H]            */
  const void* gate_proj;           /* [I, H]         */
  const void* up_proj;             /* [I, H]         */
  const void* down_proj;           /* [H, I]         */
} mq_layer_weights;

/* Model description: the constructor arguments of MegakernelDecoder /
 * MegakernelPrefillDecoder (bindings_decode.cpp:82-191, bindings_prefill.cpp:1639-1674). */
typedef struct mq_model_desc {
  int hidden_size;        /* must be 1024 (compiled layer shape) */
  int intermediate_size;  /* 3072 */
  int num_q_heads;        /* 16 */
  int num_kv_heads;       /* 8 */
  int head_dim;           /* 128 */
  int num_layers;         /* >= 0 (0: embedding -> final norm -> LM head only) */
  int vocab_size;         /* >= 1 */
  int max_seq_len;        /* KV-cache capacity in positions */
  int max_prefill_len;    /* 0 = decode only */
  const void* embed;      /* bf16 [vocab, H] */
  const void* final_norm; /* bf16 [H] */
  const void* lm_head;    /* bf16 [vocab, H] (may equal embed: tied) */
  const void* cos_table;  /* bf16 [max_seq_len, D] */
  const void* sin_table;  /* bf16 [max_seq_len, D] */
  const mq_layer_weights* layers; /* host array [num_layers] of device pointers */
} mq_model_desc;

typedef struct mq_decoder mq_decoder;

int mq_abi_version(void);
const char* mq_last_error(void);

/* Bytes of the zero-initialised device workspace a decoder needs (sync state, layer table,
 * activations, attention partials and, when max_prefill_len > 0, prefill buffers). */
size_t mq_workspace_bytes(const mq_model_desc* desc);

/* Bytes of ONE of the two KV caches: num_layers * num_kv_heads * max_seq_len * head_dim * 2.
 * Layout [num_layers][num_kv_heads][max_seq_len][head_dim] bf16, as the reference
 * (bindings_decode.cpp:127-130). */
size_t mq_kv_cache_bytes(const mq_model_desc* desc);

/* MegakernelDecoder(...) constructor.  k_cache, v_cache and workspace are caller-owned device
 * buffers of the sizes above; the workspace must be zero-filled.  Position starts at 0. */
int mq_decoder_create(const mq_model_desc* desc, void* k_cache, void* v_cache, void* workspace,
                      size_t workspace_bytes, mq_decoder** out);
int mq_decoder_destroy(mq_decoder* dec);

/* reset(): zeroes both KV caches and sets the position to 0 (bindings_decode.cpp:236-240); also
 * clears the device error flag (see mq_decoder_check). */
int mq_decoder_reset(mq_decoder* dec, void* stream);
/* position() (bindings_decode.cpp:273-280).  Returns the host-side position counter. */
int mq_decoder_position(const mq_decoder* dec);
/* Sets the host-side position counter only (0 <= pos <= max_seq_len).  For callers that replay
 * captured mq_decode_steps launches: the device-side position advances inside the kernels, the
 * host counter (used for bounds checks and position()) does not. */
int mq_decoder_set_host_position(mq_decoder* dec, int pos);
/* Moves the decode position to `pos` (0 <= pos <= max_seq_len) on the host and, in stream order,
 * on the device; KV rows [0, pos) are kept as they are.  Replaces the host-side position that
 * chat.py passes to every decode_ldg call (chat.py:448-470, bindings copy it to the device per
 * launch, fused_decode_ldg_launch.inl:55-87). */
int mq_decoder_set_position(mq_decoder* dec, int pos, void* stream);
/* Selects MQ_MODE_PERSISTENT or MQ_MODE_MULTI_KERNEL; returns MQ_ERR_UNSUPPORTED if the device
 * cannot co-schedule the persistent grid. */
int mq_decoder_set_mode(mq_decoder* dec, int mode);
int mq_decoder_get_mode(const mq_decoder* dec);
/* Workgroups per decode launch (one per compute unit). */
int mq_decoder_grid(const mq_decoder* dec);

/* One decode step (launch_ldg_decode / launch_ldg_decode_with_logits): consumes the token at
 * d_token_in, writes the greedy next token to d_token_out and, if d_logits is non-NULL, the
 * fp32 logits [vocab].  Asynchronous on `stream`; advances the position by one.  Fails with
 * MQ_ERR_POSITION when position >= max_seq_len. */
int mq_decode_step(mq_decoder* dec, const int32_t* d_token_in, int32_t* d_token_out,
                   float* d_logits, void* stream);

/* decode_steps_cuda (bindings_prefill.cpp:1045-1075): d_tokens[0] holds the first token;
 * step i reads d_tokens[i] and writes d_tokens[i+1], i < n.  The chain stays on the device, so
 * it also replaces the reference's fill_iota + first-EOS helpers
 * (fused_decode_ldg_launch.inl:5-53) that decode_greedy_cuda builds on.  In the persistent mode
 * one kernel launch decodes up to 64 chained tokens (the reference launches once per token). */
int mq_decode_steps(mq_decoder* dec, int32_t* d_tokens, int n, void* stream);

/* Debug hook (the reference's counterpart is debug_ldg_decode_cycles,
 * bindings_prefill.cpp:980-1043): mq_decode_step that also writes the hidden state after every
 * layer (bf16-rounded values as fp32) to d_hidden_trace [num_layers][hidden_size]. */
int mq_debug_decode_step_layers(mq_decoder* dec, const int32_t* d_token_in,
                                int32_t* d_token_out, float* d_logits, float* d_hidden_trace,
                                void* stream);

/* Debug hook, the counterpart of debug_ldg_decode_cycles (bindings_prefill.cpp:980-1043) and
 * its per-block stage clock (fused_decode_ldg_common.inl:15-69): one persistent-mode decode step
 * that records 100 MHz timestamps to d_stamps [grid][num_layers][11]: per layer, the start, then
 * for each of the 5 phases "compute done" and "barrier passed". */
int mq_debug_decode_step_timing(mq_decoder* dec, const int32_t* d_token_in,
                                int32_t* d_token_out, uint64_t* d_stamps, void* stream);

/* Synchronises `stream` and returns MQ_ERR_DEVICE if a kernel flagged an error (a wait that hit
 * its spin limit, bad position or token id).  The flag stays set until mq_decoder_reset; while it
 * is set the kernels end their waits early, so results are not meaningful. */
int mq_decoder_check(mq_decoder* dec, void* stream);

/* Exchange epochs of the persistent decode kernel.  No counterpart in the reference, whose
 * cooperative grid.sync() needs none; they exist for tests and for callers that audit long runs.
 * The persistent kernel hands values between workgroups as words that carry the epoch of the
 * layer that wrote them.  The decoder state holds a base xep in [0, mq_exchange_epoch_period());
 * the k-th layer run after it (k = step * num_layers + layer) uses epoch
 * mq_exchange_epoch(xep, k), which is never 0 and runs through [1, period] cyclically, and a
 * decode step of either mode advances the base to mq_exchange_epoch_advance(xep, num_layers).
 * mq_exchange_tag(e) is the 2-bit tag the tagged (4-byte) exchange words carry for epoch e; the
 * period is a multiple of 3, so consecutive epochs keep distinct tags across the wrap.  These four
 * are pure host arithmetic (the same functions the kernels evaluate) and need no GPU. */
uint32_t mq_exchange_epoch(uint32_t xep, uint64_t k);
uint32_t mq_exchange_epoch_advance(uint32_t xep, uint64_t layers);
uint32_t mq_exchange_tag(uint32_t epoch);
uint32_t mq_exchange_epoch_period(void);
/* Debug hooks: set (in stream order; MQ_ERR_INVALID_ARG unless xep < period) or read
 * (synchronising `stream`) the decoder's exchange-epoch base, e.g. to run decode across the
 * wrap of the epoch count without decoding ~10^8 tokens first.  Creation and mq_decoder_reset
 * set it to 0. */
int mq_debug_set_exchange_epoch(mq_decoder* dec, uint32_t xep, void* stream);
int mq_debug_get_exchange_epoch(mq_decoder* dec, uint32_t* xep_out, void* stream);

/* prefill_step (bindings_prefill.cpp:731-833) over launch_prefill_float
 * (fused_prefill_launch.inl:71-731): runs tokens d_tokens[0..n) at positions 0..n-1, fills the
 * KV cache, writes the greedy next token to d_token_out (and the last position's fp32 logits to
 * d_logits if non-NULL) and sets the position to n.  1 <= n <= max_prefill_len.  A token id
 * outside [0, vocab_size) is read as id 0 and sets the device error flag that
 * mq_decoder_check reports (the ids stay on the device, so they are not checked on the host). */
int mq_prefill(mq_decoder* dec, const int32_t* d_tokens, int n, int32_t* d_token_out,
               float* d_logits, void* stream);

/* Prefill with caller-supplied embedding rows: as mq_prefill, but rows
 * [embeds_start, embeds_start + embeds_len) of the input take d_embeds (bf16
 * [embeds_len, 1024], e.g. audio-tower outputs) instead of the token embeddings.
 * Replaces prefill_asr (bindings_prefill.cpp:835-955, bindings_fused_prefill.cpp:286-330) and
 * prefill_patch_audio_kernel (fused_prefill_kernels.inl:28-45); errors as bindings_prefill.cpp:
 * 838-859 (embeds_len > 0, 0 <= embeds_start, embeds_start + embeds_len <= n). */
int mq_prefill_embeds(mq_decoder* dec, const int32_t* d_tokens, int n, const void* d_embeds,
                      int embeds_start, int embeds_len, int32_t* d_token_out, float* d_logits,
                      void* stream);

/* prefill_step / prefill_asr of MegakernelFusedPrefillDecoder (bindings_fused_prefill.cpp:235-330)
 * over the reference's prefill megakernel (prefill_megakernel, fused_prefill_megakernel_core.inl:
 * 658-745, launched by fused_prefill_megakernel_launch.inl): one cooperative launch runs all
 * layers over the n prompt positions with fp32 activations (bf16 weights and K/V cache rows, no
 * bf16 rounding of the residual stream), then the final norm and LM head of the last position.
 * 1 <= n <= min(64, max_prefill_len).  d_embeds (bf16 [embeds_len, 1024]) may be NULL, then
 * embeds_len must be 0; otherwise rows [embeds_start, embeds_start + embeds_len) take it, with
 * the checks of mq_prefill_embeds.  Writes the greedy next token (and the fp32 logits if
 * d_logits is non-NULL) and sets the position to n.  MQ_ERR_UNSUPPORTED on a device that cannot
 * hold 256 co-resident 512-thread workgroups. */
int mq_prefill_fused(mq_decoder* dec, const int32_t* d_tokens, int n, const void* d_embeds,
                     int embeds_start, int embeds_len, int32_t* d_token_out, float* d_logits,
                     void* stream);

/* Debug hook: mq_prefill that also writes the residual stream after every layer to d_trace
 * (bf16 [num_layers][n][hidden_size]), for layer-by-layer parity checks of the prefill path
 * (launch_prefill_float's per-layer hidden_bf16, fused_prefill_launch.inl:245-657). */
int mq_debug_prefill_layers(mq_decoder* dec, const int32_t* d_tokens, int n,
                            int32_t* d_token_out, float* d_logits, void* d_trace, void* stream);

/* Debug hook: device addresses (inside the workspace) of the prefill buffers of the last
 * prefill: out5 = {h [n,H], xn [n,H], qkv [n,Hq*D+2*Hkv*D], att [n,Hq*D], mlp [n,I]}, bf16. */
int mq_debug_prefill_buffers(const mq_decoder* dec, void** out5);

/* ---- op-level entry points (per-op microbenchmarks; layer `layer` of the decoder's model) ----
 * (a) RMSNorm + q|k|v GEMV + q/k RMSNorm + RoPE at `pos`; writes rotated q (fp32 [Hq*D]) and the
 *     K/V cache rows at `pos` (fused_decode_ldg_common.inl:131-394). */
int mq_op_qkv_rope(mq_decoder* dec, int layer, const void* d_x_bf16, int pos, float* d_q_out,
                   void* stream);
/* (b) GQA attention of rotated queries (fp32 [Hq*D]) over cache rows [0, cache_len) of `layer`
 *     -> fp32 [Hq*D] (fused_decode_ldg_common.inl:417-794). */
int mq_op_attention(mq_decoder* dec, int layer, const float* d_q, int cache_len, float* d_out,
                    void* stream);
/* (b') Allocation-free variant of mq_op_attention.  No counterpart in the reference: it is for
 *     callers that cannot allocate device memory (code under HIP graph capture, tight serving
 *     loops, harnesses that forbid hipMalloc).  Same inputs, outputs and kernels as
 *     mq_op_attention, but the split-K partials live in a static device array of the library
 *     (640 KiB on each GPU it runs on, held until the process ends) instead of the decoder's
 *     workspace, and the call allocates nothing.  Calls that overlap on one GPU share that array
 *     and race.  The array's size does not depend on the input: the split is capped at 64
 *     position chunks per kv head, and the array holds that many partials, so every cache
 *     length mq_op_attention accepts fits; cache_len outside [1, max_seq_len] (and a bad layer)
 *     is rejected with MQ_ERR_INVALID_ARG before anything runs. */
int mq_op_attention_noalloc(mq_decoder* dec, int layer, const float* d_q, int cache_len,
                            float* d_out, void* stream);
/* (c) x_out = bf16(W_down(silu(W_gate n) * W_up n) + a), n = RMSNorm(a) * post_ln
 *     (fused_decode_ldg_mlp.inl:70-217).  a: fp32 [H]. */
int mq_op_mlp(mq_decoder* dec, int layer, const float* d_a, void* d_x_out_bf16, void* stream);
/* One whole decoder layer at position `pos` (generate.py:78-110 decode_layer): bf16 hidden in ->
 * bf16 hidden out, writing K/V cache row `pos` of `layer` and attending over rows [0, pos].
 * Uses the decoder's workspace; does not change the decode position.  Input and output must
 * not alias. */
int mq_op_decode_layer(mq_decoder* dec, int layer, const void* d_x_bf16, int pos,
                       void* d_x_out_bf16, void* stream);
/* (d) final RMSNorm + LM head + argmax of a bf16 hidden state (fused_decode_ldg_lm.inl:6-163);
 *     d_logits may be NULL. */
int mq_op_lm_head(mq_decoder* dec, const void* d_x_bf16, int32_t* d_token_out, float* d_logits,
                  void* stream);

/* ---- Unmasked multi-head attention over [B, H, T, 64] (the ASR audio tower's self-attention).
 * Replaces flash_attn_bhwd (megaqwen/triton_flash_attn.py:27-171); that function's argument
 * checks (:38-50) are made by its Python front end (megaqwen_amd/flash_attn.py).
 * out = softmax(scale * q k^T) v for every (batch, head), no mask.  q, k, v, out: contiguous
 * [batch, heads, seq_len, head_dim] tensors of one 16-bit type `dtype`; head_dim must be 64.
 * fp32 arithmetic, output rounded to nearest-even in `dtype`.  Needs no decoder.
 * seq_len == 0 (or batch or heads 0) is a no-op; batch * heads must be <= 65535; out must not
 * overlap k or v (it may be q).  d_workspace: device memory of at least
 * mq_flash_attn_workspace_bytes() bytes, 16-byte aligned (K and V^T copies in MFMA-operand
 * order, written and read within the call). */
#define MQ_DTYPE_BF16 0
#define MQ_DTYPE_F16 1
size_t mq_flash_attn_workspace_bytes(int batch, int heads, int seq_len, int head_dim);
int mq_flash_attn_bhwd(const void* d_q, const void* d_k, const void* d_v, void* d_out,
                       int batch, int heads, int seq_len, int head_dim, int dtype, float scale,
                       void* d_workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEGAQWEN_HIP_H */
