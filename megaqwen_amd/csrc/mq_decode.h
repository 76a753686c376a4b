// Shared host/device declarations of the decode path: device-side weight table, per-step
// scratch, kernel parameters and the host launchers implemented in decode.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mq_config.h"
#include "mq_device.h"

// Device copy of one layer's weight pointers, in the order of the reference's LDGLayerWeights
// (csrc/megakernel/fused_decode_ldg_common.inl:97-109) and of the public mq_layer_weights.
struct MqLayerW {
  const bf16_t* in_ln;
  const bf16_t* wq;
  const bf16_t* wk;
  const bf16_t* wv;
  const bf16_t* q_norm;
  const bf16_t* k_norm;
  const bf16_t* wo;
  const bf16_t* post_ln;
  const bf16_t* wg;
  const bf16_t* wu;
  const bf16_t* wd;
};

// fp32 activations of the op-level entry points and the attention split-K partials (in the
// caller's workspace).  Every array here is written and read across workgroups with the coherent
// (sc1) accessors of mq_device.h.
struct MqScratch {
  float qkv[MQ_QKV];           // raw q | k | v projections (before q/k RMSNorm and RoPE)
  float att[MQ_QDIM];          // merged attention output
  float a[MQ_H];               // residual stream after attention: W_o att + x
  float mlp[MQ_I];             // silu(gate) * up
  float part[MQ_NKV * MQ_MAX_CHUNKS * MQ_GQA * MQ_PART_STRIDE];  // attention split-K partials
};

// Exchange buffers of the decode kernels (in the caller's workspace).  Values that cross
// workgroups travel without any barrier.  The q|k|v rows and the layer output are 64-bit
// (value, epoch) words: the low 32 bits are
// the fp32 value, the high 32 bits the exchange epoch of the step and layer that wrote it.  A
// reader polls the words it needs until every one carries the epoch it expects: one store and one
// load per value, no acknowledgement wait before an arrival and no atomic.  The buffers
// alternate by layer parity.  Values every workgroup reads are written once per kv-head group
// (copy g is read by the workgroups wg % 8 == g), so each cache line has 32 readers instead of
// 256; on MI355X that took a 1024-value exchange among 256 workgroups from 3.4 to 1.6 us.
// The one-kernel-per-phase mode writes these with epoch 0 (never expected: epochs start at 1)
// and reads the values only.  The larger exchanges (the O partials, 8192 values, silu(gate) * up,
// 3072, and the split-mode attention partials) keep 4-byte words: a tag derived from the epoch
// replaces the two lowest mantissa bits of each fp32 value (tag_bits in decode.hip), and every
// thread of the reader polls its share; both modes write them with the same epochs.  Against a
// counter barrier (stores, acknowledgement wait, arrival atomics, poll, then the data load) that
// took a token at pos 128 from 572 to 536 us, and the tagged attention partials a token at 1024
// positions from 620 to 579 us.
struct MqExchange {
  uint64_t q[2][MQ_NKV][4 * MQ_D];       // q|k|v rows of each kv-head group (read by the group)
  uint64_t h[2][MQ_GROUPS][MQ_H / 2];    // layer output: a bf16 row pair per word (bits 0-15
                                         // row 2k, 16-31 row 2k + 1), epoch in bits 32-63
  // tagged fp32 words (the two low mantissa bits hold the epoch's low bits), by layer parity,
  // one copy per group (XCD):
  float opart[2][MQ_GROUPS][MQ_NKV][MQ_H];  // per-kv-head O-projection partials W_o[:, head h] att_h
  float m[2][MQ_GROUPS][MQ_I];              // silu(gate) * up
  // split-mode attention partials (m, l, o[128] per query head and chunk, part_ptr layout), tagged
  // words by layer parity; every member of a group rewrites its slot in every split-mode layer.
  // Cleared whenever the position is set: a sequence that starts in local mode and reaches split
  // mode later must not find an earlier sequence's words there, whose tags may match.
  float part[2][MQ_NKV * MQ_MAX_CHUNKS * MQ_GQA * MQ_PART_STRIDE];
};
MQ_DEV uint64_t xword(float v, uint32_t e) { return ((uint64_t)e << 32) | __float_as_uint(v); }
MQ_DEV float xvalue(uint64_t w) { return __uint_as_float((uint32_t)w); }
MQ_DEV uint32_t xepoch(uint64_t w) { return (uint32_t)(w >> 32); }

// Exchange epochs.  Layer k (k = step * num_layers + l, counted from the launch's first layer)
// of a launch whose state holds base xep (0 <= xep < MQ_XEP_PERIOD) exchanges its values under
// epoch 1 + (xep + k) mod MQ_XEP_PERIOD, and the launch leaves (xep + layers run) mod
// MQ_XEP_PERIOD behind for the next one.  So an epoch is never 0 (the value the one-kernel-per-
// phase mode writes into its epoch words, and a cleared buffer holds), and the epochs of
// consecutive layers run 1, 2, ..., MQ_XEP_PERIOD, 1, 2, ... without a break: MQ_XEP_PERIOD is a
// multiple of 3, so the tags 1 + e mod 3 of the tagged words also stay distinct for e, e - 1 and
// e - 2 across the wrap.  (A 32-bit count that simply wrapped would give epoch 0 after 2^32
// layers, about 153 M tokens at 28 layers, and two equal tags in a row there.)
#define MQ_XEP_PERIOD 3221225472u      // 3 * 2^30
__host__ __device__ inline uint32_t mq_xep_epoch(uint32_t xep, uint64_t k) {
  return 1u + (uint32_t)(((uint64_t)xep + k) % MQ_XEP_PERIOD);
}
__host__ __device__ inline uint32_t mq_xep_advance(uint32_t xep, uint64_t layers) {
  return (uint32_t)(((uint64_t)xep + layers) % MQ_XEP_PERIOD);
}
__host__ __device__ inline uint32_t mq_xtag(uint32_t e) { return 1u + e % 3u; }

struct MqState {
  MqSync sync;
  MqLine pos;                  // device-side decode position (read at step start, +1 at step end)
  MqLine steps;                // completed steps of multi-step launches (the step-done epoch)
  MqLine xep;                  // exchange-epoch base in [0, MQ_XEP_PERIOD): advanced by
                               // mq_xep_advance(xep, num_layers) per decode step of either mode;
                               // creation and reset, which clear MqExchange, zero it
  MqLine place[MQ_GROUPS];     // persistent launches: workgroups claimed on each XCD so far in
                               // this launch (reset by its last step, and by every state fill)
};

struct MqDecodeParams {
  const MqLayerW* layers;      // device array [num_layers]
  int num_layers;
  int vocab;
  int max_seq;
  const bf16_t* embed;         // [vocab, H]
  const bf16_t* final_norm;    // [H]
  const bf16_t* lm_head;       // [vocab, H] (tied to embed for Qwen3-0.6B)
  const bf16_t* cos;           // [max_seq, D] bf16
  const bf16_t* sin;
  bf16_t* kc;                  // [num_layers, NKV, max_seq, D]
  bf16_t* vc;
  const int* tok_in;           // device token id consumed by this step
  int* tok_out;                // device argmax token written at the end of the step
  float* logits;               // optional fp32 [vocab]
  float* trace;                // optional fp32 [num_layers, H]: hidden state after every layer
  uint64_t* stamps;            // optional [grid][num_layers][MQ_NSTAMP] 100 MHz timestamps
  MqScratch* s;
  MqExchange* x;
  MqState* st;
  float scale_log2;            // log2(e) / sqrt(D): scores are kept in the log2 domain
  int attn_local_max;          // cache lengths up to this are attended over all positions by
                               // every workgroup of a kv-head group (no split-K partials, no
                               // merge); longer ones are split into position chunks
  int early_kv;                // persistent mode: launch the long-context variant that issues
                               // each layer's K rows with its q|k|v weights (host-chosen per
                               // launch, mq_decode_early_kv; correct at any position)
  int nsteps;                  // persistent mode: tokens decoded by one launch.  Step i reads
                               // tok_in (i = 0) or tok_out[i - 1] and writes tok_out[i]; logits
                               // are written for nsteps == 1 only
};

// Per-layer timestamps of the persistent kernel's debug mode (s_memrealtime, 100 MHz):
// 0 layer start, then for each of the 5 phases k: 2k+1 compute done, 2k+2 input received.
#define MQ_NSTAMP 11

// Attention work split: number of position chunks per kv head for a given cache length and
// grid size, chosen so that every chunk is non-empty.  Shared by host and device.
#define MQ_ATT_MIN_CHUNK MQ_ATT_BLOCK
__host__ __device__ inline int mq_attn_nchunks(int cache_len, int grid) {
  int maxc = grid / MQ_NKV;
  if (maxc > MQ_MAX_CHUNKS) maxc = MQ_MAX_CHUNKS;
  if (maxc < 1) maxc = 1;
  int want = (cache_len + MQ_ATT_MIN_CHUNK - 1) / MQ_ATT_MIN_CHUNK;
  if (want < 1) want = 1;
  if (want > maxc) want = maxc;
  int clen = (cache_len + want - 1) / want;
  return (cache_len + clen - 1) / clen;
}
__host__ __device__ inline int mq_attn_chunk_len(int cache_len, int nch) {
  return (cache_len + nch - 1) / nch;
}

// ---------------------------------------------------------------- host launchers (decode.hip)
// Decode kernel organisation (values match MQ_MODE_* of include/megaqwen_hip.h).
#ifndef MQ_MODE_PERSISTENT
#define MQ_MODE_PERSISTENT 0
#define MQ_MODE_MULTI_KERNEL 1
#endif

int mq_launch_decode(const MqDecodeParams& p, int mode, int grid, hipStream_t stream);

// Fused short-prompt prefill (mq_prefill_fused_kernel): fp32 buffers for up to
// MQ_FUSED_MAX_N positions, in the decoder workspace (mq_fused_workspace_bytes).  Every
// activation of a launch has a buffer of its own (one per layer and stage), written once, as
// tagged words (the launch's tag in the two lowest mantissa bits) that their readers poll with
// device-scope loads: h, att and m with device-scope stores (they cross XCDs), q|k|v, which one
// XCD both writes and reads, with plain stores into that XCD's L2.
#define MQ_FUSED_MAX_N 64
struct MqFusedArgs {
  float* h;                    // [2 L + 1][MQ_FUSED_MAX_N][H] residual stream: the embeddings,
                               // then per layer l the stream after attention (2 l + 1) and
                               // after the MLP (2 l + 2)
  float* qkv;                  // [L][MQ_FUSED_MAX_N][4096] raw q | k | v projections
  float* att;                  // [L][MQ_FUSED_MAX_N][2048] attention output
  float* m;                    // [L][MQ_FUSED_MAX_N][I] silu(gate) * up
  uint32_t* bar;               // sync area, zeroed per launch: per-XCD role-claim counters (8
                               // lines of 128 bytes)
  const int32_t* tokens;       // device token ids [n]
  int n;
  const bf16_t* patch;         // optional bf16 rows replacing the embeddings [patch_start, +len)
  int patch_start;
  int patch_len;
  int* tok_out;                // greedy next token
  float* logits;               // optional fp32 [vocab] of the last position
  int tag;                     // 1..3: the tag of this launch's activation words (no row < n of
                               // h, qkv, att or m holds it from an earlier launch)
};
size_t mq_fused_workspace_bytes(int num_layers);
// Bytes of the tagged activation buffers (h, qkv, att, m: one region from f.h), which must hold
// zeros (no tag) before the first launch.
size_t mq_fused_activation_bytes(int num_layers);
void mq_fused_bind(MqFusedArgs* f, char* base, int num_layers);
// One cooperative launch over `grid` (>= 256) workgroups; 1 <= f.n <= MQ_FUSED_MAX_N.
int mq_launch_prefill_fused(const MqDecodeParams& p, const MqFusedArgs& f, int grid,
                            hipStream_t stream);
// Smallest split-mode attention chunk (positions) of a kv-head group for a cache length: each
// chunk is a partial the whole group polls and merges, so below a few thousand positions fewer,
// longer chunks pay (per token, A/B on one box, against chunks of at least 28: 1024 positions
// 525.8 against 536.9 us with 56, 2048 positions 550.6 against 554.2 with 112; 300 positions
// unchanged with 56, slower with 112).  Every chunk is at least one register slot per compute
// wave (MQ_ATT_SLOT).
__host__ __device__ inline int mq_attn_min_chunk(int cache_len) {
  return cache_len < 1536 ? 2 * MQ_ATT_SLOT : 4 * MQ_ATT_SLOT;
}
// Whether a persistent launch starting at `pos` should use the long-context variant: every
// workgroup of a group then holds an attention chunk in every step of the launch (positions
// only grow within a launch), and the short-context local mode no longer applies.
__host__ __device__ inline int mq_decode_early_kv(int pos, int grid, int local_max) {
  const int cache_len = pos + 1;
  return cache_len >= (grid / MQ_GROUPS) * mq_attn_min_chunk(cache_len) && cache_len > local_max
             ? 1 : 0;
}
// Clears the completion state and sets the device position; the error flag is kept
// (sticky until mq_decoder_reset or creation, so mq_decoder_check still reports it) unless
// `clear_err`.
int mq_launch_fill_state(MqState* st, int pos, hipStream_t stream, bool clear_err = false);
// A new position for the next decode step (after a prefill or a caller's seek): clears the
// split-mode attention partials, then sets the state as mq_launch_fill_state does.
int mq_launch_set_position(MqState* st, MqExchange* x, int pos, hipStream_t stream);
// Creation / reset: the state as above with the error flag and the exchange epoch zeroed, and the
// exchange buffers cleared (no stale word can carry an epoch a later step expects).
int mq_launch_clear_state(MqState* st, MqExchange* x, hipStream_t stream);
int mq_launch_zero(void* ptr, size_t bytes, hipStream_t stream);
int mq_decode_grid(int mode, int* grid_out);
int mq_read_error(MqState* st, hipStream_t stream, uint32_t* err_out);
// Debug: sets / reads the exchange-epoch base MqState.xep (set: xep < MQ_XEP_PERIOD, else -3).
int mq_launch_set_xep(MqState* st, uint32_t xep, hipStream_t stream);
int mq_read_xep(MqState* st, hipStream_t stream, uint32_t* xep_out);

// op-level launchers (per-op microbenchmarks and parity tests)
int mq_launch_op_qkv_rope(const MqDecodeParams& p, int layer, const bf16_t* x, int pos,
                          float* q_out, int grid, hipStream_t stream);
int mq_launch_op_attention(const MqDecodeParams& p, int layer, const float* q_hat, int cache_len,
                           float* att_out, int grid, hipStream_t stream);
// mq_launch_op_attention with p.s replaced by the library's static device scratch (no
// allocation, no workspace).  Calls that overlap on one GPU share that scratch and race.
#define MQ_NOALLOC_SCRATCH_BYTES (640u * 1024u)
int mq_launch_op_attention_noalloc(const MqDecodeParams& p, int layer, const float* q_hat,
                                   int cache_len, float* att_out, int grid, hipStream_t stream);
int mq_launch_op_mlp(const MqDecodeParams& p, int layer, const float* a_in, bf16_t* x_out,
                     int grid, hipStream_t stream);
int mq_launch_op_layer(const MqDecodeParams& p, int layer, const bf16_t* x, int pos,
                       bf16_t* x_out, int grid, hipStream_t stream);
int mq_launch_op_lm_head(const MqDecodeParams& p, const bf16_t* x, int* tok_out, float* logits,
                         int grid, hipStream_t stream);
// LM head over bf16(RMSNorm(x) * w_final) (the prefill path's last-token head).
int mq_launch_lm_head_bf16norm(const MqDecodeParams& p, const bf16_t* x, int* tok_out,
                               float* logits, int grid, hipStream_t stream);
