// C ABI of libmegaqwen_hip.so (declared in include/megaqwen_hip.h).
//
// The decoder handle is a small host object: it owns no device memory.  KV caches and the
// workspace (sync state, device layer-pointer table, activations, attention partials, prefill
// buffers) are caller-owned, so a Python caller can keep them as torch tensors, as the
// reference's chat.py keeps its caches (chat.py:409-421).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <new>
#include <string>
#include <vector>

#include "../../include/megaqwen_hip.h"
#include "mq_decode.h"
#include "mq_flash.h"
#include "mq_prefill.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Layout {
  size_t state, layers, scratch, xch, prefill, fused, total;
};

Layout layout_of(const mq_model_desc* d) {
  Layout L;
  L.state = 0;
  L.layers = align_up(L.state + sizeof(MqState), 256);
  L.scratch = align_up(L.layers + sizeof(MqLayerW) * (size_t)d->num_layers, 256);
  L.xch = align_up(L.scratch + sizeof(MqScratch), 256);
  L.prefill = align_up(L.xch + sizeof(MqExchange), 256);
  L.fused = align_up(L.prefill + mq_prefill_workspace_bytes(d->max_prefill_len), 256);
  // the fused short-prompt prefill's fp32 buffers (only for decoders that can prefill)
  L.total = align_up(L.fused + (d->max_prefill_len > 0 ? mq_fused_workspace_bytes(d->num_layers) : 0), 256);
  return L;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Integer tuning knob from the environment (the reference reads its kernel switches the same
// way, e.g. MEGAQWEN_FUSE_LM_HEAD); out-of-range or malformed values fall back to `dflt`.
int env_int(const char* name, int dflt, int lo, int hi) {
  const char* v = getenv(name);
  if (v == nullptr || *v == 0) return dflt;
  char* end = nullptr;
  const long x = strtol(v, &end, 10);
  if (end == v || *end != 0 || x < lo || x > hi) return dflt;
  return (int)x;
}

int check_desc(const mq_model_desc* d) {
  if (d == nullptr) return fail(MQ_ERR_INVALID_ARG, "model description is NULL");
  if (d->hidden_size != MQ_H || d->intermediate_size != MQ_I || d->num_q_heads != MQ_NQ ||
      d->num_kv_heads != MQ_NKV || d->head_dim != MQ_D)
    return fail(MQ_ERR_INVALID_ARG,
                "layer shape (hidden %d, intermediate %d, heads %d/%d, head_dim %d) differs from "
                "the compiled Qwen3-0.6B shape (1024, 3072, 16/8, 128)",
                d->hidden_size, d->intermediate_size, d->num_q_heads, d->num_kv_heads,
                d->head_dim);
  if (d->num_layers < 0 || d->num_layers > MQ_MAX_LAYERS)
    return fail(MQ_ERR_INVALID_ARG, "num_layers %d out of range", d->num_layers);
  if (d->vocab_size < 1) return fail(MQ_ERR_INVALID_ARG, "vocab_size %d < 1", d->vocab_size);
  if (d->max_seq_len < 1) return fail(MQ_ERR_INVALID_ARG, "max_seq_len %d < 1", d->max_seq_len);
  if (d->max_prefill_len < 0 || d->max_prefill_len > d->max_seq_len)
    return fail(MQ_ERR_INVALID_ARG, "max_prefill_len %d must be in [0, max_seq_len=%d]",
                d->max_prefill_len, d->max_seq_len);
  const void* top[] = {d->embed, d->final_norm, d->lm_head, d->cos_table, d->sin_table};
  for (const void* t : top)
    if (t == nullptr || !aligned16(t))
      return fail(MQ_ERR_INVALID_ARG, "model tensors must be non-NULL and 16-byte aligned");
  if (d->layers == nullptr && d->num_layers > 0)
    return fail(MQ_ERR_INVALID_ARG, "layers array is NULL");
  for (int l = 0; l < d->num_layers; ++l) {
    const void* const* f = reinterpret_cast<const void* const*>(&d->layers[l]);
    for (int i = 0; i < 11; ++i)
      if (f[i] == nullptr || !aligned16(f[i]))
        return fail(MQ_ERR_INVALID_ARG,
                    "layer %d weight %d is NULL or not 16-byte aligned", l, i);
  }
  return MQ_OK;
}

}  // namespace

struct mq_decoder {
  MqDecodeParams p;
  Layout lay;
  int mode;
  int grid;
  int pos;
  int max_prefill;
  int early_kv_mode;       // -1: long-context variant chosen by position; 0 never (default); 1 always
  size_t kv_bytes;
  char* ws;
  MqPrefillBuffers pf;
  MqFusedArgs fused;
  // tag of the last fused-prefill launch that wrote each row of the tagged activation buffers
  // (0: zeros since creation or reset)
  uint8_t fused_tag[MQ_FUSED_MAX_N];
  std::vector<MqLayerW> host_layers;
};

// Zeroes the fused prefill's tagged activation buffers and forgets their tags.
static int clear_fused_tags(mq_decoder* dec, hipStream_t s) {
  memset(dec->fused_tag, 0, sizeof(dec->fused_tag));
  if (dec->max_prefill <= 0) return 0;
  return mq_launch_zero(dec->fused.h, mq_fused_activation_bytes(dec->p.num_layers), s);
}

extern "C" {

// Kernel variant of the next persistent launch (MEGAQWEN_EARLY_KV forces it either way; both
// variants give the same results at every position).
static int early_kv(const mq_decoder* dec) {
  if (dec->early_kv_mode >= 0) return dec->early_kv_mode;
  return mq_decode_early_kv(dec->pos, dec->grid, dec->p.attn_local_max);
}

int mq_abi_version(void) { return MQ_ABI_VERSION; }

const char* mq_last_error(void) { return g_err.c_str(); }

size_t mq_workspace_bytes(const mq_model_desc* desc) {
  if (check_desc(desc) != MQ_OK) return 0;
  return layout_of(desc).total;
}

size_t mq_kv_cache_bytes(const mq_model_desc* desc) {
  if (check_desc(desc) != MQ_OK) return 0;
  return (size_t)desc->num_layers * MQ_NKV * (size_t)desc->max_seq_len * MQ_D * sizeof(bf16_t);
}

int mq_decoder_create(const mq_model_desc* desc, void* k_cache, void* v_cache, void* workspace,
                      size_t workspace_bytes, mq_decoder** out) {
  if (out == nullptr) return fail(MQ_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  int rc = check_desc(desc);
  if (rc != MQ_OK) return rc;
  const Layout lay = layout_of(desc);
  if (workspace == nullptr || workspace_bytes < lay.total || (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(MQ_ERR_INVALID_ARG, "workspace must be 256-byte aligned and >= %zu bytes",
                lay.total);
  if (k_cache == nullptr || v_cache == nullptr || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(MQ_ERR_INVALID_ARG, "KV caches must be non-NULL and 16-byte aligned");

  int grid = 0, mode = MQ_MODE_PERSISTENT;
  if (mq_decode_grid(MQ_MODE_PERSISTENT, &grid) != 0) {
    mode = MQ_MODE_MULTI_KERNEL;
    if (mq_decode_grid(MQ_MODE_MULTI_KERNEL, &grid) != 0)
      return fail(MQ_ERR_HIP, "cannot query the HIP device");
  }
  if (grid < 64)
    return fail(MQ_ERR_UNSUPPORTED, "device has %d compute units; at least 64 are required",
                grid);

  char* ws = static_cast<char*>(workspace);
  // Device copy of the layer-pointer table (LDGLayerWeights[] of bindings_decode.cpp:119-122).
  MqLayerW* host_layers = new (std::nothrow) MqLayerW[desc->num_layers];
  if (host_layers == nullptr) return fail(MQ_ERR_INVALID_ARG, "out of host memory");
  for (int l = 0; l < desc->num_layers; ++l) {
    const mq_layer_weights& s = desc->layers[l];
    MqLayerW& d = host_layers[l];
    d.in_ln = static_cast<const bf16_t*>(s.input_layernorm);
    d.wq = static_cast<const bf16_t*>(s.q_proj);
    d.wk = static_cast<const bf16_t*>(s.k_proj);
    d.wv = static_cast<const bf16_t*>(s.v_proj);
    d.q_norm = static_cast<const bf16_t*>(s.q_norm);
    d.k_norm = static_cast<const bf16_t*>(s.k_norm);
    d.wo = static_cast<const bf16_t*>(s.o_proj);
    d.post_ln = static_cast<const bf16_t*>(s.post_attn_layernorm);
    d.wg = static_cast<const bf16_t*>(s.gate_proj);
    d.wu = static_cast<const bf16_t*>(s.up_proj);
    d.wd = static_cast<const bf16_t*>(s.down_proj);
  }
  hipError_t e = hipMemcpy(ws + lay.layers, host_layers, sizeof(MqLayerW) * desc->num_layers,
                           hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    delete[] host_layers;
    return fail(MQ_ERR_HIP, "hipMemcpy(layer table): %s", hipGetErrorString(e));
  }
  mq_decoder* dec = new (std::nothrow) mq_decoder();
  if (dec == nullptr) {
    delete[] host_layers;
    return fail(MQ_ERR_INVALID_ARG, "out of host memory");
  }
  dec->host_layers.assign(host_layers, host_layers + desc->num_layers);
  delete[] host_layers;
  MqDecodeParams& p = dec->p;
  memset(&p, 0, sizeof(p));
  p.layers = reinterpret_cast<const MqLayerW*>(ws + lay.layers);
  p.num_layers = desc->num_layers;
  p.vocab = desc->vocab_size;
  p.max_seq = desc->max_seq_len;
  p.embed = static_cast<const bf16_t*>(desc->embed);
  p.final_norm = static_cast<const bf16_t*>(desc->final_norm);
  p.lm_head = static_cast<const bf16_t*>(desc->lm_head);
  p.cos = static_cast<const bf16_t*>(desc->cos_table);
  p.sin = static_cast<const bf16_t*>(desc->sin_table);
  p.kc = static_cast<bf16_t*>(k_cache);
  p.vc = static_cast<bf16_t*>(v_cache);
  p.s = reinterpret_cast<MqScratch*>(ws + lay.scratch);
  p.x = reinterpret_cast<MqExchange*>(ws + lay.xch);
  p.st = reinterpret_cast<MqState*>(ws + lay.state);
  p.scale_log2 = (float)(1.4426950408889634 / sqrt((double)MQ_D));
  p.attn_local_max = env_int("MEGAQWEN_ATTN_LOCAL_MAX", MQ_ATT_LOCAL_DEFAULT, 0, 1 << 20);
  p.early_kv = 0;
  p.nsteps = 1;
  // the long-context variant (K rows issued a phase early) lost to the plain one once the
  // exchanges carried tagged words: 646 against 659 us per token at pos 4096, 570 against 580
  // at 1024 (A/B on one box), so it runs only when asked for
  dec->early_kv_mode = env_int("MEGAQWEN_EARLY_KV", 0, -1, 1);
  dec->lay = lay;
  dec->mode = mode;
  dec->grid = grid;
  dec->pos = 0;
  dec->max_prefill = desc->max_prefill_len;
  dec->kv_bytes = (size_t)desc->num_layers * MQ_NKV * (size_t)desc->max_seq_len * MQ_D * 2;
  dec->ws = ws;
  mq_prefill_bind(&dec->pf, ws + lay.prefill, desc->max_prefill_len);
  memset(&dec->fused, 0, sizeof(dec->fused));
  if (desc->max_prefill_len > 0) mq_fused_bind(&dec->fused, ws + lay.fused, desc->num_layers);
  if (mq_launch_clear_state(p.st, p.x, nullptr) != 0 || clear_fused_tags(dec, nullptr) != 0 ||
      (dec->pf.cnt != nullptr && mq_launch_zero(dec->pf.cnt, dec->pf.cnt_bytes, nullptr) != 0) ||
      hipStreamSynchronize(nullptr) != hipSuccess) {
    delete dec;
    return fail(MQ_ERR_HIP, "state initialisation failed");
  }
  *out = dec;
  return MQ_OK;
}

int mq_decoder_destroy(mq_decoder* dec) {
  delete dec;
  return MQ_OK;
}

int mq_decoder_reset(mq_decoder* dec, void* stream) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mq_launch_zero(dec->p.kc, dec->kv_bytes, s) != 0 ||
      mq_launch_zero(dec->p.vc, dec->kv_bytes, s) != 0 ||
      mq_launch_clear_state(dec->p.st, dec->p.x, s) != 0 || clear_fused_tags(dec, s) != 0 ||
      (dec->pf.cnt != nullptr && mq_launch_zero(dec->pf.cnt, dec->pf.cnt_bytes, s) != 0))
    return fail(MQ_ERR_HIP, "reset kernels failed to launch");
  dec->pos = 0;
  return MQ_OK;
}

int mq_decoder_position(const mq_decoder* dec) { return dec ? dec->pos : -1; }

int mq_decoder_set_host_position(mq_decoder* dec, int pos) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  if (pos < 0 || pos > dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "position %d outside [0, %d]", pos, dec->p.max_seq);
  dec->pos = pos;
  return MQ_OK;
}

int mq_decoder_set_position(mq_decoder* dec, int pos, void* stream) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  if (pos < 0 || pos > dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "position %d outside [0, %d]", pos, dec->p.max_seq);
  if (mq_launch_set_position(dec->p.st, dec->p.x, pos, static_cast<hipStream_t>(stream)) != 0)
    return fail(MQ_ERR_HIP, "state update failed");
  dec->pos = pos;
  return MQ_OK;
}

int mq_decoder_set_mode(mq_decoder* dec, int mode) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  if (mode != MQ_MODE_PERSISTENT && mode != MQ_MODE_MULTI_KERNEL)
    return fail(MQ_ERR_INVALID_ARG, "unknown mode %d", mode);
  int grid = 0;
  if (mq_decode_grid(mode, &grid) != 0)
    return fail(MQ_ERR_UNSUPPORTED, "mode %d is not available on this device", mode);
  dec->mode = mode;
  dec->grid = grid;
  return MQ_OK;
}

int mq_decoder_get_mode(const mq_decoder* dec) { return dec ? dec->mode : -1; }
int mq_decoder_grid(const mq_decoder* dec) { return dec ? dec->grid : -1; }

int mq_decode_step(mq_decoder* dec, const int32_t* d_token_in, int32_t* d_token_out,
                   float* d_logits, void* stream) {
  if (dec == nullptr || d_token_in == nullptr || d_token_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder and token pointers must be non-NULL");
  if (dec->pos >= dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "decode position %d reaches max_seq_len %d", dec->pos,
                dec->p.max_seq);
  MqDecodeParams p = dec->p;
  p.early_kv = early_kv(dec);
  p.tok_in = d_token_in;
  p.tok_out = d_token_out;
  p.logits = d_logits;
  int rc = mq_launch_decode(p, dec->mode, dec->grid, static_cast<hipStream_t>(stream));
  if (rc != 0) return fail(MQ_ERR_HIP, "decode launch failed (%d)", rc);
  dec->pos += 1;
  return MQ_OK;
}

int mq_debug_decode_step_layers(mq_decoder* dec, const int32_t* d_token_in,
                                int32_t* d_token_out, float* d_logits, float* d_hidden_trace,
                                void* stream) {
  if (dec == nullptr || d_token_in == nullptr || d_token_out == nullptr ||
      d_hidden_trace == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder, token and trace pointers must be non-NULL");
  if (dec->pos >= dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "decode position %d reaches max_seq_len %d", dec->pos,
                dec->p.max_seq);
  MqDecodeParams p = dec->p;
  p.early_kv = early_kv(dec);
  p.tok_in = d_token_in;
  p.tok_out = d_token_out;
  p.logits = d_logits;
  p.trace = d_hidden_trace;
  int rc = mq_launch_decode(p, dec->mode, dec->grid, static_cast<hipStream_t>(stream));
  if (rc != 0) return fail(MQ_ERR_HIP, "decode launch failed (%d)", rc);
  dec->pos += 1;
  return MQ_OK;
}

int mq_debug_decode_step_timing(mq_decoder* dec, const int32_t* d_token_in,
                                int32_t* d_token_out, uint64_t* d_stamps, void* stream) {
  if (dec == nullptr || d_token_in == nullptr || d_token_out == nullptr || d_stamps == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder, token and stamp pointers must be non-NULL");
  if (dec->mode != MQ_MODE_PERSISTENT)
    return fail(MQ_ERR_UNSUPPORTED, "stage timing needs the persistent mode");
  if (dec->pos >= dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "decode position %d reaches max_seq_len %d", dec->pos,
                dec->p.max_seq);
  MqDecodeParams p = dec->p;
  p.early_kv = early_kv(dec);
  p.tok_in = d_token_in;
  p.tok_out = d_token_out;
  p.stamps = d_stamps;
  int rc = mq_launch_decode(p, dec->mode, dec->grid, static_cast<hipStream_t>(stream));
  if (rc != 0) return fail(MQ_ERR_HIP, "decode launch failed (%d)", rc);
  dec->pos += 1;
  return MQ_OK;
}

int mq_decode_steps(mq_decoder* dec, int32_t* d_tokens, int n, void* stream) {
  if (dec == nullptr || d_tokens == nullptr || n < 0)
    return fail(MQ_ERR_INVALID_ARG, "bad decode_steps arguments");
  if ((long long)dec->pos + n > dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "decode_steps would exceed max_seq_len (%d + %d > %d)",
                dec->pos, n, dec->p.max_seq);
  // persistent mode: up to MQ_STEPS_PER_LAUNCH tokens per launch (the kernel chains them on the
  // device); the multi-kernel mode launches its phases per token
  const int per = dec->mode == MQ_MODE_PERSISTENT ? MQ_STEPS_PER_LAUNCH : 1;
  for (int i = 0; i < n; i += per) {
    MqDecodeParams p = dec->p;
    p.early_kv = early_kv(dec);
    p.nsteps = n - i < per ? n - i : per;
    p.tok_in = d_tokens + i;
    p.tok_out = d_tokens + i + 1;
    p.logits = nullptr;
    int rc = mq_launch_decode(p, dec->mode, dec->grid, static_cast<hipStream_t>(stream));
    if (rc != 0) return fail(MQ_ERR_HIP, "decode launch at step %d failed (%d)", i, rc);
    dec->pos += p.nsteps;
  }
  return MQ_OK;
}

int mq_decoder_check(mq_decoder* dec, void* stream) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  uint32_t err = 0;
  if (mq_read_error(dec->p.st, static_cast<hipStream_t>(stream), &err) != 0)
    return fail(MQ_ERR_HIP, "error-flag readback failed");
  if (err != 0) return fail(MQ_ERR_DEVICE, "device error flag %u (1 = exchange time-out, 2 = bad position/token, 4 = workgroup placement)", err);
  return MQ_OK;
}

uint32_t mq_exchange_epoch(uint32_t xep, uint64_t k) { return mq_xep_epoch(xep % MQ_XEP_PERIOD, k); }
uint32_t mq_exchange_epoch_advance(uint32_t xep, uint64_t layers) {
  return mq_xep_advance(xep % MQ_XEP_PERIOD, layers);
}
uint32_t mq_exchange_tag(uint32_t epoch) { return mq_xtag(epoch); }
uint32_t mq_exchange_epoch_period(void) { return MQ_XEP_PERIOD; }

int mq_debug_set_exchange_epoch(mq_decoder* dec, uint32_t xep, void* stream) {
  if (dec == nullptr) return fail(MQ_ERR_INVALID_ARG, "decoder is NULL");
  if (xep >= MQ_XEP_PERIOD)
    return fail(MQ_ERR_INVALID_ARG, "exchange epoch base %u outside [0, %u)", xep, MQ_XEP_PERIOD);
  if (mq_launch_set_xep(dec->p.st, xep, static_cast<hipStream_t>(stream)) != 0)
    return fail(MQ_ERR_HIP, "state update failed");
  return MQ_OK;
}

int mq_debug_get_exchange_epoch(mq_decoder* dec, uint32_t* xep_out, void* stream) {
  if (dec == nullptr || xep_out == nullptr) return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (mq_read_xep(dec->p.st, static_cast<hipStream_t>(stream), xep_out) != 0)
    return fail(MQ_ERR_HIP, "exchange-epoch readback failed");
  return MQ_OK;
}

int mq_prefill(mq_decoder* dec, const int32_t* d_tokens, int n, int32_t* d_token_out,
               float* d_logits, void* stream) {
  if (dec == nullptr || d_tokens == nullptr || d_token_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder and token pointers must be non-NULL");
  if (n <= 0) return fail(MQ_ERR_INVALID_ARG, "Empty input sequence");
  if (n > dec->max_prefill)
    return fail(MQ_ERR_INVALID_ARG, "Prefill sequence length %d exceeds maximum %d", n,
                dec->max_prefill);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = mq_launch_prefill(dec->p, dec->host_layers.data(), dec->pf, d_tokens, n, d_token_out,
                             d_logits, dec->grid, s);
  if (rc != 0) return fail(MQ_ERR_HIP, "prefill launch failed (%d)", rc);
  if (mq_launch_set_position(dec->p.st, dec->p.x, n, s) != 0) return fail(MQ_ERR_HIP, "state update failed");
  dec->pos = n;
  return MQ_OK;
}

int mq_prefill_embeds(mq_decoder* dec, const int32_t* d_tokens, int n, const void* d_embeds,
                      int embeds_start, int embeds_len, int32_t* d_token_out, float* d_logits,
                      void* stream) {
  if (dec == nullptr || d_tokens == nullptr || d_token_out == nullptr || d_embeds == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder, token and embedding pointers must be non-NULL");
  if (n > dec->max_prefill) return fail(MQ_ERR_INVALID_ARG, "Prefill sequence length exceeds maximum");
  if (n <= 0) return fail(MQ_ERR_INVALID_ARG, "Empty input sequence");
  if (embeds_len <= 0) return fail(MQ_ERR_INVALID_ARG, "audio_embeds must have audio_len > 0");
  if (embeds_start < 0 || embeds_start + embeds_len > n)
    return fail(MQ_ERR_INVALID_ARG, "Invalid audio_start_idx/audio_len for the given seq_len");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = mq_launch_prefill(dec->p, dec->host_layers.data(), dec->pf, d_tokens, n, d_token_out,
                             d_logits, dec->grid, s, static_cast<const bf16_t*>(d_embeds),
                             embeds_start, embeds_len);
  if (rc != 0) return fail(MQ_ERR_HIP, "prefill launch failed (%d)", rc);
  if (mq_launch_set_position(dec->p.st, dec->p.x, n, s) != 0) return fail(MQ_ERR_HIP, "state update failed");
  dec->pos = n;
  return MQ_OK;
}

int mq_prefill_fused(mq_decoder* dec, const int32_t* d_tokens, int n, const void* d_embeds,
                     int embeds_start, int embeds_len, int32_t* d_token_out, float* d_logits,
                     void* stream) {
  if (dec == nullptr || d_tokens == nullptr || d_token_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder and token pointers must be non-NULL");
  if (n <= 0) return fail(MQ_ERR_INVALID_ARG, "Empty input sequence");
  if (n > dec->max_prefill || n > MQ_FUSED_MAX_N)
    return fail(MQ_ERR_INVALID_ARG, "Prefill sequence length %d exceeds maximum %d", n,
                dec->max_prefill < MQ_FUSED_MAX_N ? dec->max_prefill : MQ_FUSED_MAX_N);
  if (d_embeds != nullptr) {
    if (embeds_len <= 0) return fail(MQ_ERR_INVALID_ARG, "audio_embeds must have audio_len > 0");
    if (embeds_start < 0 || embeds_start + embeds_len > n)
      return fail(MQ_ERR_INVALID_ARG, "Invalid audio_start_idx/audio_len for the given seq_len");
  } else if (embeds_len != 0) {
    return fail(MQ_ERR_INVALID_ARG, "embeds_len without embeddings");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  MqFusedArgs f = dec->fused;
  f.tokens = d_tokens;
  f.n = n;
  f.patch = static_cast<const bf16_t*>(d_embeds);
  f.patch_start = d_embeds != nullptr ? embeds_start : 0;
  f.patch_len = d_embeds != nullptr ? embeds_len : 0;
  f.tok_out = d_token_out;
  f.logits = d_logits;
  // a tag that no row < n holds from an earlier launch (rows hold at most the three tags; when
  // all three are present, the buffers are zeroed first)
  unsigned used = 0;
  for (int r = 0; r < n; ++r) used |= 1u << dec->fused_tag[r];
  int tag = 1;
  while (tag <= 3 && (used >> tag & 1u)) ++tag;
  if (tag > 3) {
    if (clear_fused_tags(dec, s) != 0) return fail(MQ_ERR_HIP, "fused buffer clear failed");
    tag = 1;
  }
  f.tag = tag;
  const int rc = mq_launch_prefill_fused(dec->p, f, dec->grid, s);
  if (rc == -2 || rc == -3)
    return fail(MQ_ERR_UNSUPPORTED, "the fused prefill needs 256 co-resident workgroups (%d)",
                dec->grid);
  if (rc != 0) return fail(MQ_ERR_HIP, "fused prefill launch failed (%d)", rc);
  memset(dec->fused_tag, tag, (size_t)n);
  if (mq_launch_set_position(dec->p.st, dec->p.x, n, s) != 0)
    return fail(MQ_ERR_HIP, "state update failed");
  dec->pos = n;
  return MQ_OK;
}

int mq_debug_prefill_layers(mq_decoder* dec, const int32_t* d_tokens, int n,
                            int32_t* d_token_out, float* d_logits, void* d_trace, void* stream) {
  if (dec == nullptr || d_tokens == nullptr || d_token_out == nullptr || d_trace == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "decoder, token and trace pointers must be non-NULL");
  if (n <= 0) return fail(MQ_ERR_INVALID_ARG, "Empty input sequence");
  if (n > dec->max_prefill)
    return fail(MQ_ERR_INVALID_ARG, "Prefill sequence length %d exceeds maximum %d", n,
                dec->max_prefill);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = mq_launch_prefill(dec->p, dec->host_layers.data(), dec->pf, d_tokens, n, d_token_out,
                             d_logits, dec->grid, s, nullptr, 0, 0, static_cast<bf16_t*>(d_trace));
  if (rc != 0) return fail(MQ_ERR_HIP, "prefill launch failed (%d)", rc);
  if (mq_launch_set_position(dec->p.st, dec->p.x, n, s) != 0) return fail(MQ_ERR_HIP, "state update failed");
  dec->pos = n;
  return MQ_OK;
}

int mq_debug_prefill_buffers(const mq_decoder* dec, void** out5) {
  if (dec == nullptr || out5 == nullptr) return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  out5[0] = dec->pf.h;
  out5[1] = dec->pf.xn;
  out5[2] = dec->pf.qkv;
  out5[3] = dec->pf.att;
  out5[4] = dec->pf.m;
  return MQ_OK;
}

int mq_op_qkv_rope(mq_decoder* dec, int layer, const void* d_x_bf16, int pos, float* d_q_out,
                   void* stream) {
  if (dec == nullptr || d_x_bf16 == nullptr || d_q_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (layer < 0 || layer >= dec->p.num_layers || pos < 0 || pos >= dec->p.max_seq)
    return fail(MQ_ERR_INVALID_ARG, "layer %d / pos %d out of range", layer, pos);
  int rc = mq_launch_op_qkv_rope(dec->p, layer, static_cast<const bf16_t*>(d_x_bf16), pos, d_q_out,
                                 dec->grid, static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

int mq_op_attention(mq_decoder* dec, int layer, const float* d_q, int cache_len, float* d_out,
                    void* stream) {
  if (dec == nullptr || d_q == nullptr || d_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (layer < 0 || layer >= dec->p.num_layers || cache_len < 1 || cache_len > dec->p.max_seq)
    return fail(MQ_ERR_INVALID_ARG, "layer %d / cache_len %d out of range", layer, cache_len);
  int rc = mq_launch_op_attention(dec->p, layer, d_q, cache_len, d_out, dec->grid,
                                  static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

int mq_op_attention_noalloc(mq_decoder* dec, int layer, const float* d_q, int cache_len,
                            float* d_out, void* stream) {
  if (dec == nullptr || d_q == nullptr || d_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (layer < 0 || layer >= dec->p.num_layers || cache_len < 1 || cache_len > dec->p.max_seq)
    return fail(MQ_ERR_INVALID_ARG, "layer %d / cache_len %d out of range", layer, cache_len);
  int rc = mq_launch_op_attention_noalloc(dec->p, layer, d_q, cache_len, d_out, dec->grid,
                                          static_cast<hipStream_t>(stream));
  if (rc == -1 || rc == -2)
    return fail(MQ_ERR_HIP, "device address of the static scratch unavailable (%d)", rc);
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

int mq_op_mlp(mq_decoder* dec, int layer, const float* d_a, void* d_x_out_bf16, void* stream) {
  if (dec == nullptr || d_a == nullptr || d_x_out_bf16 == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (layer < 0 || layer >= dec->p.num_layers)
    return fail(MQ_ERR_INVALID_ARG, "layer %d out of range", layer);
  int rc = mq_launch_op_mlp(dec->p, layer, d_a, static_cast<bf16_t*>(d_x_out_bf16), dec->grid,
                            static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

int mq_op_decode_layer(mq_decoder* dec, int layer, const void* d_x_bf16, int pos,
                       void* d_x_out_bf16, void* stream) {
  if (dec == nullptr || d_x_bf16 == nullptr || d_x_out_bf16 == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if (layer < 0 || layer >= dec->p.num_layers)
    return fail(MQ_ERR_INVALID_ARG, "layer %d out of range", layer);
  if (pos < 0 || pos >= dec->p.max_seq)
    return fail(MQ_ERR_POSITION, "position %d outside [0, max_seq_len=%d)", pos, dec->p.max_seq);
  if (d_x_bf16 == d_x_out_bf16)
    return fail(MQ_ERR_INVALID_ARG, "layer input and output must not alias");
  int rc = mq_launch_op_layer(dec->p, layer, static_cast<const bf16_t*>(d_x_bf16), pos,
                              static_cast<bf16_t*>(d_x_out_bf16), dec->grid,
                              static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

int mq_op_lm_head(mq_decoder* dec, const void* d_x_bf16, int32_t* d_token_out, float* d_logits,
                  void* stream) {
  if (dec == nullptr || d_x_bf16 == nullptr || d_token_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  int rc = mq_launch_op_lm_head(dec->p, static_cast<const bf16_t*>(d_x_bf16), d_token_out,
                                d_logits, dec->grid, static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%d)", rc);
}

size_t mq_flash_attn_workspace_bytes(int batch, int heads, int seq_len, int head_dim) {
  if (batch < 0 || heads < 0 || seq_len < 0 || head_dim != 64) {
    fail(MQ_ERR_INVALID_ARG, "bad shape (batch %d, heads %d, seq_len %d, head_dim %d)", batch,
         heads, seq_len, head_dim);
    return 0;
  }
  if ((long long)batch * heads > 65535) {
    fail(MQ_ERR_INVALID_ARG, "batch * heads = %lld exceeds 65535", (long long)batch * heads);
    return 0;
  }
  return mq_flash_attn_workspace(batch * heads, seq_len);
}

int mq_flash_attn_bhwd(const void* d_q, const void* d_k, const void* d_v, void* d_out,
                       int batch, int heads, int seq_len, int head_dim, int dtype, float scale,
                       void* d_workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || heads < 0 || seq_len < 0)
    return fail(MQ_ERR_INVALID_ARG, "negative size (batch %d, heads %d, seq_len %d)", batch,
                heads, seq_len);
  if (head_dim != 64) return fail(MQ_ERR_INVALID_ARG, "Only head_dim=64 supported, got %d", head_dim);
  if (dtype != MQ_DTYPE_BF16 && dtype != MQ_DTYPE_F16)
    return fail(MQ_ERR_INVALID_ARG, "dtype %d is neither MQ_DTYPE_BF16 nor MQ_DTYPE_F16", dtype);
  if (batch == 0 || heads == 0 || seq_len == 0) return MQ_OK;
  if (d_q == nullptr || d_k == nullptr || d_v == nullptr || d_out == nullptr)
    return fail(MQ_ERR_INVALID_ARG, "NULL argument");
  if ((long long)batch * heads > 65535)
    return fail(MQ_ERR_INVALID_ARG, "batch * heads = %lld exceeds 65535",
                (long long)batch * heads);
  const size_t bytes = (size_t)batch * heads * seq_len * head_dim * 2;
  auto overlaps = [&](const void* a, const void* b) {
    const char* x = static_cast<const char*>(a);
    const char* y = static_cast<const char*>(b);
    return x < y + bytes && y < x + bytes;
  };
  if (overlaps(d_out, d_k) || overlaps(d_out, d_v))
    return fail(MQ_ERR_INVALID_ARG, "out must not overlap k or v");
  const size_t ws = mq_flash_attn_workspace(batch * heads, seq_len);
  if (d_workspace == nullptr || workspace_bytes < ws || (reinterpret_cast<uintptr_t>(d_workspace) & 15) != 0)
    return fail(MQ_ERR_INVALID_ARG, "workspace needs %zu bytes, 16-byte aligned (got %zu)", ws,
                workspace_bytes);
  const float scale_log2 = (float)((double)scale * 1.4426950408889634);
  const int rc = mq_launch_flash_attn_bhwd(d_q, d_k, d_v, d_out, batch * heads, seq_len,
                                           dtype == MQ_DTYPE_F16, scale_log2, d_workspace,
                                           static_cast<hipStream_t>(stream));
  return rc == 0 ? MQ_OK : fail(MQ_ERR_HIP, "launch failed (%s)", hipGetErrorString(hipGetLastError()));
}

}  // extern "C"
