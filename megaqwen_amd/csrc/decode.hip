// Batch-1 bf16 decode for the Qwen3-0.6B layer shape on gfx950.
//
// One decode step = 28 layers x 5 phases + the LM head:
//   P1  RMSNorm(x) and the fused q|k|v GEMV (4096 rows x 1024)
//   P2  per-(kv head, position chunk) attention: q/k RMSNorm + RoPE prologue, K/V cache write of
//       the new position, two-pass softmax over the chunk; with several chunks per head each
//       publishes a split-K partial (m, l, o[128]) and the last chunk to finish merges them
//   P3  O GEMV (1024 x 2048) + residual
//   P4  RMSNorm(a) + gate/up GEMVs (2 x 3072 x 1024) + silu(g) * u
//   P5  down GEMV (1024 x 3072) + residual, rounded to bf16 (the layer output)
//   LM  final RMSNorm + LM-head GEMV (vocab x 1024) + argmax (packed 64-bit atomic max)
// The phases run either inside one persistent cooperative kernel separated by grid barriers
// (5 per layer = 140 per token, against 225 in the reference's ldg_decode_kernel,
// csrc/megakernel/fused_decode_ldg_kernel.inl:5-259), or as one kernel launch per phase.
//
// Workgroup organisation (512 threads): waves 0..6 are compute waves, wave 7 is the sync wave.
// Per phase the compute waves finish their dot products, publish outputs with coherent (sc1)
// stores, wait for them, then issue the NEXT phase's weight loads into registers; the sync wave
// meanwhile runs the grid barrier and, once it opens, loads the next phase's input vector into
// LDS.  Because gfx9 returns a wave's loads in order, keeping the prefetches out of the sync
// wave is what lets the barrier and the input broadcast proceed while weights stream in.
// Residuals stay in registers: a workgroup owns the same hidden rows in the O and down phases.
//
// Numerics follow the reference decode path: fp32 activations and accumulation, bf16 weights,
// bf16 K/V cache rows (fused_decode_ldg_common.inl:376-377), bf16 cos/sin tables, the residual
// stream rounded to bf16 at every layer end (fused_decode_ldg_mlp.inl:200), LM head on the fp32
// normalised hidden state (fused_decode_ldg_lm.inl:47-122).
#include "mq_decode.h"

#include <math.h>

#include <mutex>
#include <type_traits>

// Thread index hidden behind an empty asm so that per-lane address arithmetic is recomputed in
// every phase instead of being hoisted out of the 28-layer loop of the persistent kernel (where
// it would pin ~60 VGPRs for the whole kernel).
MQ_DEV int tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
MQ_DEV int wave_id() { return tid() >> 6; }
MQ_DEV int lane_id() { return tid() & 63; }

static_assert(MQ_THREADS * 2 == MQ_H, "the norm helpers assume two hidden elements per thread");
static_assert(MQ_GQA == 2, "attention items process the two query heads of a kv head");
static_assert(MQ_SYNC_WAVE == MQ_CWAVES && MQ_CWAVES + 1 == MQ_WAVES, "one sync wave");

// LDS carve (floats) of the GEMV phases.
#define LDS_IN 0          // [3072] phase input vector (filled by the sync wave)
#define LDS_XN 3072       // [1024] RMS-normalised input
#define LDS_PR 4096       // [256]  per-item partial dot products
#define LDS_RED 4352      // [16]   block reductions
#define LDS_KEYS 4368     // [16]   8 argmax keys (u64)
#define LDS_HID 4608      // [1024] the layer input (residual of the attention block)
#define LDS_A 5632        // [1024] a = layer input + attention block output (MLP residual)
#define LDS_ATTH 0        // [256]  merged attention output of the group's two query heads
#define LDS_AROW 6656     // [MQ_CWAVES][256] attention: unnormalised p.V of each compute wave
#define LDS_AL (LDS_AROW + MQ_CWAVES * 256)   // [MQ_CWAVES][2] sums of p of each compute wave
#define MQ_LDS_FLOATS (LDS_AL + MQ_CWAVES * 2)

// Balanced contiguous row range of workgroup `wg` out of `G` for an `n`-row matrix.
MQ_DEV void row_range(int n, int wg, int G, int& r0, int& nr) {
  r0 = (int)(((long long)n * wg) / G);
  nr = (int)(((long long)n * (wg + 1)) / G) - r0;
}

// ------------------------------------------------------------------ row GEMV with prefetch
// A workgroup owns `nr` rows (of one matrix, or of two stacked ones, see the row functions).
// A row of K bf16 elements is split into S segments; item it = (row it / S, segment it % S) is
// handled by compute wave it % 7 as 16-byte loads per lane over K/S/512 wave-wide chunks.
// `load` issues the first PF items of every compute wave into registers (in the persistent
// kernel, before the barrier that precedes the phase); `compute` finishes them against the fp32
// vector in LDS and streams any further items (only for grids smaller than 256 workgroups).
template <int K, int S, int PF>
struct RowSet {
  static constexpr int KS = K / S;
  static constexpr int NL = KS / 512;
  static_assert(KS % 512 == 0, "segments are whole 512-element wave loads");
  uint4 w[PF][NL];

  template <class RowPtr>
  MQ_DEV void load(RowPtr rowptr, int nr) {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int nitems = nr * S;
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int it = wave + j * MQ_CWAVES;
      if (it < nitems) {
        const bf16_t* r = rowptr(it / S) + (it % S) * KS + lane * 8;
#pragma unroll
        for (int l = 0; l < NL; ++l) w[j][l] = ld_nt16(r + l * 512);
      } else {
#pragma unroll
        for (int l = 0; l < NL; ++l) w[j][l] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  template <class RowPtr, class Out>
  MQ_DEV void compute(RowPtr rowptr, int nr, const float* __restrict__ x, Out out) const {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int nitems = nr * S;
    // all PF items as straight-line code (items past nitems hold zero weights), so the x reads
    // are shared and the four reductions run as one (sum4_rows: item j's total in lanes 16j..)
    static_assert(PF <= 4, "sum4_rows reduces four items");
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const float* xs = x + ((wave + j * MQ_CWAVES) % S) * KS + lane * 8;
#pragma unroll
      for (int l = 0; l < NL; ++l) acc[j] = dot8_lds(w[j][l], xs + l * 512, acc[j]);
    }
    {
      const float tot = sum4_rows(acc[0], acc[1], acc[2], acc[3]);
      const int j = lane >> 4, it = wave + j * MQ_CWAVES;
      if ((lane & 15) == 0 && j < PF && it < nitems) out(it, tot);
    }
    for (int it = wave + PF * MQ_CWAVES; it < nitems; it += MQ_CWAVES) {
      const bf16_t* r = rowptr(it / S) + (it % S) * KS + lane * 8;
      uint4 v[NL];
#pragma unroll
      for (int l = 0; l < NL; ++l) v[l] = ld_nt16(r + l * 512);
      const float* xs = x + (it % S) * KS + lane * 8;
      float acc = 0.f;
#pragma unroll
      for (int l = 0; l < NL; ++l) acc = dot8_lds(v[l], xs + l * 512, acc);
      acc = wave_sum(acc);
      if (lane == 0) out(it, acc);
    }
  }
};

typedef RowSet<MQ_H, 1, 3> QkvSet;      // 16 rows / workgroup at 256 workgroups
typedef RowSet<MQ_QDIM, 2, 2> OSet;     //  4 rows x 2 segments
typedef RowSet<MQ_H, 1, 4> GateUpSet;   // 12 gate + 12 up rows
typedef RowSet<MQ_I, 2, 2> DownSet;     //  4 rows x 2 segments

MQ_DEV const bf16_t* qkv_row(const MqLayerW& w, int r) {
  if (r < MQ_QDIM) return w.wq + (size_t)r * MQ_H;
  if (r < MQ_QDIM + MQ_KVDIM) return w.wk + (size_t)(r - MQ_QDIM) * MQ_H;
  return w.wv + (size_t)(r - MQ_QDIM - MQ_KVDIM) * MQ_H;
}

// --------------------------------------------------------------------- phase inputs (sync wave)
// Copies N coherent fp32 values (written by other workgroups) into LDS; all loads are issued
// before the first LDS store so the copy costs one memory round trip.
template <int N>
MQ_DEV void wave_copy_coh(float* dst, const float* src) {
  static_assert(N % 128 == 0, "whole float2 per lane");
  constexpr int P = N / 128;
  const int lane = lane_id();
  float2 v[P];
#pragma unroll
  for (int i = 0; i < P; ++i) v[i] = ld_coh2(src + 2 * (lane + 64 * i));
#pragma unroll
  for (int i = 0; i < P; ++i) reinterpret_cast<float2*>(dst)[lane + 64 * i] = v[i];
}
// The bf16 embedding row (read-only) -> fp32 LDS.
MQ_DEV void wave_copy_bf16_1024(float* dst, const bf16_t* src) {
  const int lane = lane_id();
  uint4 v[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = ld16(src + 8 * (lane + 64 * i));
#pragma unroll
  for (int i = 0; i < 2; ++i) unpack8(v[i], dst + 8 * (lane + 64 * i));
}

// Phase boundary.  Compute waves arrive with this phase's dot products in LDS and the next
// phase's weight prefetch in flight.  The sync wave then runs `epilogue()` (finishes this
// phase's outputs and publishes them with coherent stores), waits for those stores, runs the
// grid barrier (when `barrier`) and `input()` (the next phase's input vector into LDS).  The
// compute waves never wait for a store, so their prefetches are never waited on either.
template <class Epi, class Input>
MQ_DEV void phase_sync(MqSync* sy, uint32_t target, bool barrier, Epi epilogue, Input input) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) {
    epilogue();
    wait_all_memory();
    if (barrier) grid_barrier_wave(sy, target);
    input();
    wait_all_memory();
  }
  __syncthreads();
}
// End of a single-phase kernel: the sync wave publishes the phase's outputs.
template <class Epi>
MQ_DEV void phase_finish(Epi epilogue) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) epilogue();
}
#define MQ_NOTHING [] {}

// 2^x with the hardware v_exp_f32 (results below the normal range flush to zero, as the
// reference's fast-math __expf does); used for softmax weights, whose arguments are <= 0.
MQ_DEV float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------- RMSNorm
// xn = x * rsqrt(mean(x^2) + eps) * w over the 1024 values in LDS `x`, two per thread.
// fused_decode_ldg_common.inl:150-191 (input norm), fused_decode_ldg_mlp.inl:70-118 (post norm),
// fused_decode_ldg_kernel.inl:103-137 (final norm).
// With `round_out` the result is rounded to bf16 (the prefill path's final norm,
// prefill_final_norm_kernel, fused_prefill_kernels.inl:655-700).
MQ_DEV void norm_1024(const float* x, const bf16_t* __restrict__ w, float* xn, float* red,
                      bool round_out = false) {
  const int t = tid();
  const float2 v = reinterpret_cast<const float2*>(x)[t];
  const float ss = block_sum(v.x * v.x + v.y * v.y, red);
  const float r = rsqrtf(ss * (1.0f / MQ_H) + MQ_EPS);
  const uint32_t wv = ld32(w + 2 * t);
  float y0 = v.x * r * bf16_lo(wv), y1 = v.y * r * bf16_hi(wv);
  if (round_out) {
    y0 = round_bf16(y0);
    y1 = round_bf16(y1);
  }
  xn[2 * t] = y0;
  xn[2 * t + 1] = y1;
}

// ------------------------------------------------------------------------------ P1: q|k|v
MQ_DEV void qkv_load(QkvSet& ws, const MqLayerW& w, int wg, int G) {
  int r0, nr;
  row_range(MQ_QKV, wg, G, r0, nr);
  ws.load([&](int i) { return qkv_row(w, r0 + i); }, nr);
}
// Input: the layer input x in LDS_IN; dot products -> LDS_PR.
MQ_DEV void qkv_run(const QkvSet& ws, const MqLayerW& w, int wg, int G, float* lds) {
  norm_1024(lds + LDS_IN, w.in_ln, lds + LDS_XN, lds + LDS_RED);
  __syncthreads();
  int r0, nr;
  row_range(MQ_QKV, wg, G, r0, nr);
  ws.compute([&](int i) { return qkv_row(w, r0 + i); }, nr, lds + LDS_XN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: publish q|k|v rows.
MQ_DEV void qkv_publish(float* qkv, int wg, int G, const float* lds) {
  int r0, nr;
  row_range(MQ_QKV, wg, G, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) st_coh(qkv + r0 + t, lds[LDS_PR + t]);
}

// ------------------------------------------------------------------------- P2: attention
// LDS carve of the attention phase (floats).
#define ALDS_RAW 0        // [512] raw q(2 heads) | k | v of this kv head (sync wave input)
#define ALDS_QS 512       // [256] rotated q of the two query heads
#define ALDS_KN 768       // [128] new-position k-hat (bf16 values)
#define ALDS_VN 896       // [128] new-position v (bf16 values)
#define ALDS_PRM 1024     // [512] q_norm | k_norm | cos row | sin row of this step, as fp32
#define ALDS_WML 1536     // [MQ_CWAVES][4] per-wave m0, m1, l0, l1
#define ALDS_STAT 1568    // m[2], l[2] of the item
#define ALDS_ORED 1584    // [MQ_CWAVES][256] per-wave unnormalised outputs; the item's in [0, 256)
#define ALDS_WSC (ALDS_ORED + MQ_CWAVES * 256)   // [MQ_CWAVES][2][32] each wave's scores
// The merge of several chunks runs after this item's partial has been published and after the
// prologue's parameters have been used, so it reuses the parameter area.
#define ALDS_MW ALDS_PRM                         // merge: (m, l)[2][64] then weights [2][64]
#define ALDS_MSUM (ALDS_MW + 512)                // merge: [4][2][128] partial sums
static_assert(ALDS_WSC + MQ_CWAVES * 64 <= MQ_LDS_FLOATS, "attention LDS carve");
static_assert(ALDS_MSUM + 1024 <= MQ_LDS_FLOATS, "attention merge LDS carve");
static_assert(ALDS_MSUM + 1024 <= ALDS_ORED + MQ_CWAVES * 256, "merge stays in the phase carve");

// q/k RMSNorm over one head held as (lane, lane + 64) of one wave, then rotate-half RoPE with
// the bf16 table row (fused_decode_ldg_common.inl:268-394):
//   o_i = x_i c_i - x_{i+64} s_i,  o_{i+64} = x_i s_{i+64} + x_{i+64} c_{i+64}.
// nw, cs, sn: norm weight, cos row and sin row as fp32 in LDS.
MQ_DEV void head_norm_rope(float& lo, float& hi, const float* nw, const float* cs,
                           const float* sn) {
  const int lane = lane_id();
  const float ss = wave_sum(lo * lo + hi * hi);
  const float r = rsqrtf(ss * (1.0f / MQ_D) + MQ_EPS);
  const float a = lo * r * nw[lane];
  const float b = hi * r * nw[lane + 64];
  lo = a * cs[lane] - b * sn[lane];
  hi = a * sn[lane + 64] + b * cs[lane + 64];
}

MQ_DEV float* part_ptr(float* part, int h, int c, int j) {
  return part + ((size_t)(h * MQ_MAX_CHUNKS + c) * MQ_GQA + j) * MQ_PART_STRIDE;
}

// Sync-wave input of an attention item, one memory round trip: raw q of query heads 2h, 2h+1,
// k and v of kv head h (coherent loads of the q|k|v vector), plus the read-only parameters of the
// prologue (q_norm and k_norm weights of the layer, RoPE table rows of the position).
MQ_DEV void attn_input(const float* qkv, const bf16_t* qn, const bf16_t* kn, const bf16_t* cs,
                       const bf16_t* sn, int h, float* lds) {
  const int lane = lane_id();
  float2 v[4];
  v[0] = ld_coh2(qkv + 2 * h * MQ_D + 2 * lane);
  v[1] = ld_coh2(qkv + 2 * h * MQ_D + 128 + 2 * lane);
  v[2] = ld_coh2(qkv + MQ_QDIM + h * MQ_D + 2 * lane);
  v[3] = ld_coh2(qkv + MQ_QDIM + MQ_KVDIM + h * MQ_D + 2 * lane);
  uint32_t prm[4];
  prm[0] = ld32(qn + 2 * lane);
  prm[1] = ld32(kn + 2 * lane);
  prm[2] = ld32(cs + 2 * lane);
  prm[3] = ld32(sn + 2 * lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) reinterpret_cast<float2*>(lds + ALDS_RAW)[lane + 64 * i] = v[i];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    reinterpret_cast<float2*>(lds + ALDS_PRM)[64 * i + lane] =
        make_float2(bf16_lo(prm[i]), bf16_hi(prm[i]));
}

// Prologue of an attention item (inputs and parameters in LDS): q-hat of query heads 2h, 2h+1
// into ALDS_QS; k-hat and v of the new position rounded to bf16 (kept as fp32) into
// ALDS_KN / ALDS_VN.  Waves 0..3 each own one head.  The cache row itself is written later by
// the sync wave (attn_cache_row), so no compute wave ever waits for a store.
MQ_DEV void attn_prologue(float* lds) {
  const int lane = lane_id(), wave = wave_id();
  const float* raw = lds + ALDS_RAW;
  const float* prm = lds + ALDS_PRM;
  if (wave < 2) {
    float lo = raw[wave * MQ_D + lane], hi = raw[wave * MQ_D + 64 + lane];
    head_norm_rope(lo, hi, prm, prm + 256, prm + 384);
    lds[ALDS_QS + wave * MQ_D + lane] = lo;
    lds[ALDS_QS + wave * MQ_D + 64 + lane] = hi;
  } else if (wave == 2) {
    float lo = raw[256 + lane], hi = raw[256 + 64 + lane];
    head_norm_rope(lo, hi, prm + 128, prm + 256, prm + 384);
    lds[ALDS_KN + lane] = round_bf16(lo);
    lds[ALDS_KN + 64 + lane] = round_bf16(hi);
  } else if (wave == 3) {
    lds[ALDS_VN + lane] = round_bf16(raw[384 + lane]);
    lds[ALDS_VN + 64 + lane] = round_bf16(raw[384 + 64 + lane]);
  }
}

// Sync wave: the new position's K and V rows (bf16) into the cache of `layer`, kv head h.  The
// stores are device-scope (sc1): within a multi-step launch a workgroup on another XCD reads the
// row in the next step, and a plain store would sit in this XCD's L2.
MQ_DEV void attn_cache_row(const MqDecodeParams& p, int layer, int h, int pos, const float* lds) {
  const int lane = lane_id();
  const size_t row = (((size_t)layer * MQ_NKV + h) * p.max_seq + pos) * MQ_D;
  const uint32_t k2 = (uint32_t)f32_to_bf16(lds[ALDS_KN + 2 * lane]) |
                      ((uint32_t)f32_to_bf16(lds[ALDS_KN + 2 * lane + 1]) << 16);
  const uint32_t v2 = (uint32_t)f32_to_bf16(lds[ALDS_VN + 2 * lane]) |
                      ((uint32_t)f32_to_bf16(lds[ALDS_VN + 2 * lane + 1]) << 16);
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p.kc + row) + lane, k2, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p.vc + row) + lane, v2, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// K/V of up to MQ_ATT_BLOCK positions: position blk + k*28 + wave*4 + (lane/16) goes to compute
// wave `wave`, row lane/16, each lane holding 8 of the 128 dims (16 bytes).
//
// The row of the position being decoded (pos_new) is never loaded: it is written during this
// step (attn_cache_row) and its values come from LDS instead.  Fetching it before the write would
// leave a stale copy in this CU's L1 and this XCD's L2, and a chained launch reads the row with
// plain loads in the next step.  Every row below pos_new was written by an earlier step (of this
// launch, with device-scope stores ordered by the barriers in between, or of an earlier kernel)
// and was not loaded by anyone before that write, so a plain load of it cannot hit a stale line.
struct KvBlock {
  uint4 k[MQ_ATT_NK], v[MQ_ATT_NK];
};
MQ_DEV void kv_block_load(KvBlock& b, const bf16_t* Kb, const bf16_t* Vb, int blk, int bend,
                          int pos_new, bool small = false) {
  const int lane = lane_id(), wave = wave_id();
  // small chunks (<= 28 positions): wave 0 holds position blk + 4k + row in slot k
  if (wave >= (small ? 1 : MQ_CWAVES)) return;
#pragma unroll
  for (int k = 0; k < MQ_ATT_NK; ++k) {
    const int pp = small ? blk + k * 4 + (lane >> 4)
                         : blk + k * 4 * MQ_CWAVES + wave * 4 + (lane >> 4);
    if (pp < bend && pp != pos_new && (!small || k < MQ_ATT_SLOT / 4)) {
      b.k[k] = ld16(Kb + (size_t)pp * MQ_D);
      b.v[k] = ld16(Vb + (size_t)pp * MQ_D);
    } else {
      b.k[k] = b.v[k] = make_uint4(0, 0, 0, 0);
    }
  }
}
// Same block with a fixed instruction count: every compute wave issues all 2 * MQ_ATT_NK loads.
// Lanes whose position is past bend or is pos_new read the read-only row `dummy` (16 bytes per
// lane of a 256-byte row) instead, so no unwritten cache row is fetched; attn_core masks the
// former and replaces the latter from LDS.  Used for the early prefetch of long contexts, where
// the compiler must know how many loads follow the q|k|v weights to wait for those alone.
template <bool K, bool V>
MQ_DEV void kv_block_load_all(KvBlock& b, const bf16_t* Kb, const bf16_t* Vb, int blk, int bend,
                              int pos_new, const bf16_t* dummy) {
  const int lane = lane_id(), wave = wave_id();
  if (wave >= MQ_CWAVES) return;
#pragma unroll
  for (int k = 0; k < MQ_ATT_NK; ++k) {
    const int pp = blk + k * 4 * MQ_CWAVES + wave * 4 + (lane >> 4);
    const bool row = pp < bend && pp != pos_new;
    if constexpr (K) b.k[k] = ld16(row ? Kb + (size_t)pp * MQ_D : dummy);
    if constexpr (V) b.v[k] = ld16(row ? Vb + (size_t)pp * MQ_D : dummy);
  }
}
MQ_DEV const bf16_t* kv_base(const bf16_t* cache, const MqDecodeParams& p, int layer, int h) {
  return cache + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D + (lane_id() & 15) * 8;
}

// Core of one attention item: kv head h, cache positions [p0, p1), first block already in `b`.
// Rotated queries in ALDS_QS; position `pos_new` (if inside the range) takes its K/V from
// ALDS_KN/ALDS_VN instead of the cache.  Each compute wave runs its own online softmax over its
// positions (4 per wave-instruction: 16 lanes x 8 dims, DPP row sums), keeping scores, running
// max, sum and p * V in registers; one merge over the waves at the end.  Leaves m[2], l[2] in
// ALDS_STAT and the unnormalised o[2][128] in ALDS_ORED[0..255] (reference:
// fused_decode_ldg_common.inl:417-602).
MQ_DEV void attn_core(const MqDecodeParams& p, int layer, int h, int p0, int p1, int pos_new,
                      KvBlock& b, float* lds, bool small = false) {
  const float* qs = lds + ALDS_QS;
  const float* kn = lds + ALDS_KN;
  const float* vn = lds + ALDS_VN;
  float* wml = lds + ALDS_WML;
  float* stat = lds + ALDS_STAT;
  float* ored = lds + ALDS_ORED;
  const int lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, sub = lane & 15;
  // small chunks (<= 28 positions, one block): wave 0 alone takes every position, slot k holding
  // position blk + 4k + row, and the merge below has a single wave to combine
  const int nwaves = small ? 1 : MQ_CWAVES;
  if (wave < nwaves) {
    const bf16_t* Kb = kv_base(p.kc, p, layer, h);
    const bf16_t* Vb = kv_base(p.vc, p, layer, h);
    float q0[8], q1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q0[e] = qs[sub * 8 + e];
      q1[e] = qs[MQ_D + sub * 8 + e];
    }
    float acc0[8], acc1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc0[e] = acc1[e] = 0.f;
    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;   // l: this lane's row only
    for (int blk = p0; blk < p1; blk += MQ_ATT_BLOCK) {
      // keeps the next block's loads from being hoisted into this one (two blocks would not
      // fit in registers)
      asm volatile("" ::: "memory");
      const int bend = min(p1, blk + MQ_ATT_BLOCK);
      if (blk != p0) kv_block_load(b, Kb, Vb, blk, bend, pos_new);
      if (pos_new >= blk && pos_new < bend) {
        // the new position is not in the cache yet: its bf16 K/V (exact as bf16) replace the
        // registers of the lane row that holds it
        const uint4 knp = pack8_bf16(kn + sub * 8), vnp = pack8_bf16(vn + sub * 8);
#pragma unroll
        for (int k = 0; k < MQ_ATT_NK; ++k) {
          if ((small ? blk + k * 4 + g : blk + k * 4 * MQ_CWAVES + wave * 4 + g) == pos_new) {
            b.k[k] = knp;
            b.v[k] = vnp;
          }
        }
      }
      // scores of this wave's 32 positions, (head, k * 4 + row), in its own LDS slice
      float* wsc = lds + ALDS_WSC + wave * 64;
      float mx0 = -INFINITY, mx1 = -INFINITY;
      // position slots k of this wave holding at least one position below bend (wave-uniform)
      const int nk = small ? (bend - blk + 3) / 4
                           : min(MQ_ATT_NK, max(0, (bend - blk - wave * 4 + 4 * MQ_CWAVES - 1) /
                                                      (4 * MQ_CWAVES)));
#pragma unroll
      for (int k = 0; k < MQ_ATT_NK; ++k) {
        if (k >= nk) break;
        const int pp = small ? blk + k * 4 + g : blk + k * 4 * MQ_CWAVES + wave * 4 + g;
        float kv[8];
        unpack8(b.k[k], kv);
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          d0 = fmaf(q0[e], kv[e], d0);
          d1 = fmaf(q1[e], kv[e], d1);
        }
        d0 = pp < bend ? row16_sum(d0) * p.scale_log2 : -INFINITY;
        d1 = pp < bend ? row16_sum(d1) * p.scale_log2 : -INFINITY;
        if (sub == 0) {
          wsc[k * 4 + g] = d0;
          wsc[32 + k * 4 + g] = d1;
        }
        mx0 = fmaxf(mx0, d0);
        mx1 = fmaxf(mx1, d1);
      }
      mx0 = max_xor32(max_xor16(mx0));
      mx1 = max_xor32(max_xor16(mx1));
      const float n0 = fmaxf(m0, mx0), n1 = fmaxf(m1, mx1);
      // rescale of what this wave accumulated so far (nothing yet while its max is -inf)
      const float al0 = n0 == -INFINITY ? 1.f : exp2_fast(m0 - n0);
      const float al1 = n1 == -INFINITY ? 1.f : exp2_fast(m1 - n1);
      l0 *= al0;
      l1 *= al1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc0[e] *= al0;
        acc1[e] *= al1;
      }
#pragma unroll
      for (int k = 0; k < MQ_ATT_NK; ++k) {
        if (k >= nk) break;
        const int pp = small ? blk + k * 4 + g : blk + k * 4 * MQ_CWAVES + wave * 4 + g;
        const float w0 = pp < bend ? exp2_fast(wsc[k * 4 + g] - n0) : 0.f;
        const float w1 = pp < bend ? exp2_fast(wsc[32 + k * 4 + g] - n1) : 0.f;
        l0 += w0;
        l1 += w1;
        float vv[8];
        unpack8(b.v[k], vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc0[e] = fmaf(w0, vv[e], acc0[e]);
          acc1[e] = fmaf(w1, vv[e], acc1[e]);
        }
      }
      m0 = n0;
      m1 = n1;
    }
    // sum the wave's 4 position rows (lane groups of 16 share the wave's max) with row swaps,
    // so that the merge below reads one row per wave
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc0[e] = sum_xor32(sum_xor16(acc0[e]));
      acc1[e] = sum_xor32(sum_xor16(acc1[e]));
    }
    l0 = sum_xor32(sum_xor16(l0));
    l1 = sum_xor32(sum_xor16(l1));
    if (g == 0) {
      float4* arow = reinterpret_cast<float4*>(lds + LDS_AROW + wave * 256 + sub * 8);
      arow[0] = make_float4(acc0[0], acc0[1], acc0[2], acc0[3]);
      arow[1] = make_float4(acc0[4], acc0[5], acc0[6], acc0[7]);
      arow[MQ_D / 4] = make_float4(acc1[0], acc1[1], acc1[2], acc1[3]);
      arow[MQ_D / 4 + 1] = make_float4(acc1[4], acc1[5], acc1[6], acc1[7]);
    }
    if (lane == 0) {
      wml[wave * 4 + 0] = m0;
      wml[wave * 4 + 1] = m1;
      lds[LDS_AL + wave * 2 + 0] = l0;
      lds[LDS_AL + wave * 2 + 1] = l1;
    }
  }
  __syncthreads();
  // merge the compute waves (every item has at least one valid position, so M is finite); all
  // LDS reads are issued up front, waves past nwaves are masked by selects (their LDS is stale)
  if (tid() < 256) {
    const int j = tid() >> 7;
    float mw[MQ_CWAVES], ow[MQ_CWAVES], lw[MQ_CWAVES];
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) {
      mw[w8] = wml[w8 * 4 + j];
      ow[w8] = lds[LDS_AROW + w8 * 256 + tid()];
      lw[w8] = lds[LDS_AL + w8 * 2 + j];
    }
    float M = -INFINITY;
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8)
      if (w8 < nwaves) M = fmaxf(M, mw[w8]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) {
      const bool use = w8 < nwaves && mw[w8] != -INFINITY;
      const float f = use ? exp2_fast(mw[w8] - M) : 0.f;
      o = use ? fmaf(f, ow[w8], o) : o;
      L = use ? fmaf(f, lw[w8], L) : L;
    }
    ored[tid()] = o;
    if ((tid() & 127) == 0) {
      stat[j] = M;
      stat[2 + j] = L;
    }
  }
  __syncthreads();
}

// Writes this item's partial (m, l, o) of both query heads to `part` (coherent stores).
MQ_DEV void attn_write_partial(float* part, int h, int c, const float* lds) {
  if (tid() < 256) {
    const int j = tid() >> 7, d = tid() & 127;
    float* dst = part_ptr(part, h, c, j);
    st_coh(dst + 4 + d, lds[ALDS_ORED + tid()]);
    if (d == 0) {
      st_coh(dst, lds[ALDS_STAT + j]);
      st_coh(dst + 1, lds[ALDS_STAT + 2 + j]);
    }
  }
}

// Log-sum-exp merge of the nch (<= 64) partials of kv head h into att[2h*128, 2h*128 + 256),
// by all 512 threads with every load issued up front (one memory round trip):
//   att_j = sum_c exp2(m_c - M_j) o_c / sum_c exp2(m_c - M_j) l_c.
// Thread t owns query head j = t / 256, dims 2*((t / 4) % 64) + {0, 1} and chunks c = t % 4 + 4i.
template <class Out>
MQ_DEV void attn_merge(const float* part, int h, int nch, float* lds, Out out) {
  float* mw = lds + ALDS_MW;      // (m, l) pairs [2][64] -> weights [2][64] at +256
  float* msum = lds + ALDS_MSUM;  // [4][2][128]
  const int t = tid();
  const int j = t >> 8, pr = (t >> 2) & 63, q = t & 3;
  float* pbase = const_cast<float*>(part);
  float2 ml = make_float2(0.f, 0.f);
  const int mj = t >= nch ? 1 : 0, mc = t - mj * nch;   // (query head, chunk) of t < 2 nch
  if (t < 2 * nch) ml = ld_coh2(part_ptr(pbase, h, mc, mj));
  float2 o2[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = q + 4 * i;
    o2[i] = c < nch ? ld_coh2(part_ptr(pbase, h, c, j) + 4 + 2 * pr) : make_float2(0.f, 0.f);
  }
  if (t < 2 * nch) reinterpret_cast<float2*>(mw)[mj * 64 + mc] = ml;
  __syncthreads();
  if (t < 2 * 64) {
    // wave 0 and wave 1 (lanes = chunks) compute the weights of query head t / 64
    const int jj = t >> 6, c = t & 63;
    const float2 v = c < nch ? reinterpret_cast<const float2*>(mw)[jj * 64 + c]
                             : make_float2(-INFINITY, 0.f);
    const float M = wave_max(v.x);
    const float e = c < nch ? exp2f(v.x - M) : 0.f;
    const float L = wave_sum(e * v.y);
    mw[256 + jj * 64 + c] = e / L;
  }
  __syncthreads();
  const float* wj = mw + 256 + j * 64;
  float2 s = make_float2(0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = q + 4 * i;
    if (c < nch) {
      s.x = fmaf(wj[c], o2[i].x, s.x);
      s.y = fmaf(wj[c], o2[i].y, s.y);
    }
  }
  reinterpret_cast<float2*>(msum)[(q * 2 + j) * 64 + pr] = s;
  __syncthreads();
  if (t < 256) {
    const int jj = t >> 7, d = t & 127;
    float o = 0.f;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) o += msum[(qq * 2 + jj) * 128 + d];
    out(jj, d, o);
  }
}
MQ_DEV void attn_merge_head(const float* part, int h, int nch, float* att, float* lds) {
  attn_merge(part, h, nch, lds,
             [&](int jj, int d, float o) { st_coh(att + (2 * h + jj) * MQ_D + d, o); });
}

// Attention item of workgroup wg (items are (kv head h, chunk c), wg = c * NKV + h, so that
// with the round-robin workgroup -> XCD dispatch all chunks of one kv head share an XCD).
struct AttnItem {
  bool active;
  int h, c, p0, p1;
};
MQ_DEV AttnItem attn_item(int wg, int nch, int cache_len) {
  AttnItem it;
  it.active = wg < MQ_NKV * nch;
  it.h = wg % MQ_NKV;
  it.c = wg / MQ_NKV;
  const int clen = mq_attn_chunk_len(cache_len, nch);
  it.p0 = it.c * clen;
  it.p1 = min(cache_len, it.p0 + clen);
  return it;
}

// ---------------------------------------------------------------------------- P3: O proj
MQ_DEV void o_load(OSet& ws, const MqLayerW& w, int wg, int G) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  ws.load([&](int i) { return w.wo + (size_t)(r0 + i) * MQ_QDIM; }, nr);
}
// Input: att in LDS_IN; segment dot products -> LDS_PR.
MQ_DEV void o_run(const OSet& ws, const MqLayerW& w, int wg, int G, float* lds) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  ws.compute([&](int i) { return w.wo + (size_t)(r0 + i) * MQ_QDIM; }, nr, lds + LDS_IN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: lane t < nr (<= 64) holds the residual of hidden row r0 + t in `res`
// and leaves a[r0 + t] = W_o att + res in it (fused_decode_ldg_mlp.inl:24-68).
MQ_DEV void o_publish(float* a_out, int wg, int G, const float* lds, float& res) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  const int t = lane_id();
  if (t < nr) {
    res = (lds[LDS_PR + 2 * t] + lds[LDS_PR + 2 * t + 1]) + res;
    st_coh(a_out + r0 + t, res);
  }
}

// ------------------------------------------------------------------------- P4: gate / up
MQ_DEV void gu_load(GateUpSet& ws, const MqLayerW& w, int wg, int G) {
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  ws.load([&](int i) {
    return i < nr ? w.wg + (size_t)(r0 + i) * MQ_H : w.wu + (size_t)(r0 + i - nr) * MQ_H;
  }, 2 * nr);
}
// Input: a in LDS_IN; gate and up dot products -> LDS_PR.
MQ_DEV void gu_run(const GateUpSet& ws, const MqLayerW& w, int wg, int G, float* lds) {
  norm_1024(lds + LDS_IN, w.post_ln, lds + LDS_XN, lds + LDS_RED);
  __syncthreads();
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  ws.compute([&](int i) {
    return i < nr ? w.wg + (size_t)(r0 + i) * MQ_H : w.wu + (size_t)(r0 + i - nr) * MQ_H;
  }, 2 * nr, lds + LDS_XN, [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: m = silu(g) * u with silu(x) = x / (1 + e^-x)
// (fused_decode_ldg_mlp.inl:120-175, fused_decode_ldg_common.inl:123-125).
MQ_DEV void gu_publish(float* m, int wg, int G, const float* lds) {
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) {
    const float gv = lds[LDS_PR + t], uv = lds[LDS_PR + nr + t];
    st_coh(m + r0 + t, gv / (1.0f + expf(-gv)) * uv);
  }
}

// ----------------------------------------------------------------------------- P5: down
MQ_DEV void down_load(DownSet& ws, const MqLayerW& w, int wg, int G) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  ws.load([&](int i) { return w.wd + (size_t)(r0 + i) * MQ_I; }, nr);
}
// Input: m in LDS_IN; segment dot products -> LDS_PR.
MQ_DEV void down_run(const DownSet& ws, const MqLayerW& w, int wg, int G, float* lds) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  ws.compute([&](int i) { return w.wd + (size_t)(r0 + i) * MQ_I; }, nr, lds + LDS_IN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: lane t < nr holds a[r0 + t] in `res` and leaves the bf16-rounded layer
// output of that row in it (fused_decode_ldg_mlp.inl:177-217); out(r, v) publishes it.
template <class Out>
MQ_DEV void down_publish(int wg, int G, const float* lds, float& res, Out out) {
  int r0, nr;
  row_range(MQ_H, wg, G, r0, nr);
  const int t = lane_id();
  if (t < nr) {
    res = round_bf16((lds[LDS_PR + 2 * t] + lds[LDS_PR + 2 * t + 1]) + res);
    out(r0 + t, res);
  }
}

// ------------------------------------------------------------------------------ LM head
// Final RMSNorm of the hidden state in LDS_IN + logits of this workgroup's vocabulary rows +
// argmax.  Each workgroup folds its best (value, row) into one 64-bit atomic max; the last
// workgroup to finish (completion counter) publishes the token, clears the sync state for the
// next step and advances the device position when `advance_pos` (fused_decode_ldg_lm.inl:47-163
// is the two-kernel reference equivalent).  Ordering between a workgroup's two atomics comes
// from waiting for the first to return; no cache-wide fences are used.
MQ_DEV void lm_head_run(const MqDecodeParams& p, int wg, int G, float* lds, int* tok_out,
                        float* logits, int pos, bool advance_pos, bool round_norm = false,
                        bool publish_epoch = false, uint32_t step_epoch = 0) {
  float* xn = lds + LDS_XN;
  uint64_t* keys = reinterpret_cast<uint64_t*>(lds + LDS_KEYS);
  norm_1024(lds + LDS_IN, p.final_norm, xn, lds + LDS_RED, round_norm);
  __syncthreads();
  const int lane = lane_id(), wave = wave_id();
  float xl[16];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xl[e] = xn[lane * 8 + e];
    xl[8 + e] = xn[512 + lane * 8 + e];
  }
  int r0, nr;
  row_range(p.vocab, wg, G, r0, nr);
  uint64_t best = 0;
  constexpr int U = 4;
  for (int i = wave; i < nr; i += U * MQ_WAVES) {
    uint4 v[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ii = i + u * MQ_WAVES;
      if (ii < nr) {
        const bf16_t* row = p.lm_head + (size_t)(r0 + ii) * MQ_H + lane * 8;
        v[u][0] = ld_nt16(row);
        v[u][1] = ld_nt16(row + 512);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ii = i + u * MQ_WAVES;
      if (ii < nr) {
        float s = dot8(v[u][0], xl, 0.f);
        s = dot8(v[u][1], xl + 8, s);
        s = wave_sum(s);
        if (logits != nullptr && lane == 0) logits[r0 + ii] = s;
        best = u64_max(best, argmax_key(s, (uint32_t)(r0 + ii)));
      }
    }
  }
  if (lane == 0) keys[wave] = best;
  __syncthreads();
  if (tid() == 0) {
    uint64_t k = keys[0];
#pragma unroll
    for (int i = 1; i < MQ_WAVES; ++i) k = u64_max(k, keys[i]);
    MqSync* sy = &p.st->sync;
    __hip_atomic_fetch_max(&sy->argmax.v, (unsigned long long)k, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    wait_all_memory();
    const uint32_t old =
        __hip_atomic_fetch_add(&sy->done.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)G - 1) {
      const unsigned long long kk =
          __hip_atomic_load(&sy->argmax.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // device-scope store: the next step of a multi-step launch reads it in other workgroups
      __hip_atomic_store(reinterpret_cast<uint32_t*>(tok_out), argmax_key_index(kk),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sy->argmax.v, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int i = 0; i < MQ_BAR_STRIPES; ++i)
        __hip_atomic_store(&sy->bar[i].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int i = 0; i < MQ_NKV; ++i)
        __hip_atomic_store(&sy->attn[i].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (advance_pos)
        __hip_atomic_store(&p.st->pos.v, (uint32_t)(pos + 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sy->done.v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (publish_epoch) {
        // every reset above and the token are complete before the epoch releases the next step
        wait_all_memory();
        __hip_atomic_store(&p.st->steps.v, step_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// ------------------------------------------------------------------- head-group decode
// The persistent kernel assigns workgroup wg to kv-head group h = wg % 8 with index j = wg / 8
// (NG = G / 8 workgroups per group).  Workgroups are dispatched round-robin over the 8 XCDs, so
// a group shares one XCD and its L2; every exchange still uses device-scope (sc1) operations, so
// correctness does not depend on that placement, only the cost of the group-local steps does.
// Per layer:
//   1. q|k|v: group h computes the 512 rows of its kv head (q heads 2h, 2h+1, k and v of h).
//   2. group barrier; attention split over the group's workgroups by position chunks, partials
//      (m, l, o) published per chunk.
//   3. group barrier; every workgroup of the group merges the partials (att of its two query
//      heads) and computes its rows of the O projection restricted to the head's 256 columns.
//   4. grid barrier; a = x + sum_h opart_h, RMSNorm, gate|up rows.
//   5. grid barrier; down rows + a -> bf16 layer output.   6. grid barrier -> next layer.
// That is 3 grid-wide and 2 group-local barriers per layer.  For short contexts (cache length
// <= attn_local_max) steps 2-3 collapse: every workgroup of the group attends over all
// positions itself (its O rows prefetched with the K/V rows), and the merge barrier goes away.
// Measured at 1 and 64 positions this wins; at 129 positions the longer attention of every
// workgroup costs more than the barrier it saves (1404 against 1464 tok/s).

// Local row i of group h's 512 q|k|v rows -> row of the fused q|k|v projection.
MQ_DEV int grp_row(int h, int i) {
  if (i < 2 * MQ_D) return 2 * h * MQ_D + i;
  if (i < 3 * MQ_D) return MQ_QDIM + h * MQ_D + (i - 2 * MQ_D);
  return MQ_QDIM + MQ_KVDIM + h * MQ_D + (i - 3 * MQ_D);
}
MQ_DEV void gqkv_load(QkvSet& ws, const MqLayerW& w, int h, int j, int NG) {
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  ws.load([&](int i) { return qkv_row(w, grp_row(h, r0 + i)); }, nr);
}
MQ_DEV void gqkv_run(const QkvSet& ws, const MqLayerW& w, int h, int j, int NG, float* lds) {
  norm_1024(lds + LDS_IN, w.in_ln, lds + LDS_XN, lds + LDS_RED);
  __syncthreads();
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  ws.compute([&](int i) { return qkv_row(w, grp_row(h, r0 + i)); }, nr, lds + LDS_XN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
MQ_DEV void gqkv_publish(float* qkv, int h, int j, int NG, const float* lds) {
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) st_coh(qkv + grp_row(h, r0 + t), lds[LDS_PR + t]);
}

// Position chunks of a group: as many chunks of at least one register slot (28 positions) as
// the group has workgroups; chunk j = [p0, p1).  All chunks c < nch are non-empty.
// Local mode (cache_len <= local_max): one chunk over all positions.  With `all_local` (the
// persistent kernel) every workgroup of the group computes it, so the attention output needs no
// exchange; otherwise (one kernel per phase) workgroup 0 of the group computes it and publishes
// it as the only partial.  Either way the K/V cache row is written by workgroup 0 (has_pos).
struct GAttn {
  int nch, p0, p1;
  bool active, has_pos, small, local;
};
MQ_DEV GAttn gattn_plan(int j, int NG, int cache_len, int pos, int local_max, bool all_local) {
  GAttn g;
  g.local = cache_len <= local_max;
  if (g.local) {
    g.nch = 1;
    g.p0 = 0;
    g.p1 = cache_len;
    g.active = all_local || j == 0;
    g.has_pos = j == 0;
    g.small = cache_len <= 8;
    return g;
  }
  const int want = (cache_len + MQ_ATT_SLOT - 1) / MQ_ATT_SLOT;
  const int n0 = min(min(NG, MQ_MAX_CHUNKS), want);
  const int clen = (cache_len + n0 - 1) / n0;
  g.nch = (cache_len + clen - 1) / clen;
  g.p0 = j * clen;
  g.p1 = min(cache_len, g.p0 + clen);
  g.active = j < g.nch;
  g.has_pos = g.active && pos >= g.p0 && pos < g.p1;
  // one wave has no other wave to hide its dependent reduction steps: it wins only for chunks of
  // at most two position slots (measured 1.5 against 2.0 us at 4 positions, 3.5 against 2.2 at 28)
  g.small = clen <= 8;
  return g;
}
// Attention output of a single chunk covering every position: o / l as the log-sum-exp merge
// computes it for one partial (weight exp2(m - m) / l = 1 / l, then one fused multiply), so the
// persistent kernel's local result and the one-kernel-per-phase merge of the published partial
// are bitwise equal.
MQ_DEV float att_single(float o, float l) { return fmaf(1.0f / l, o, 0.f); }
// All threads, local mode: attention output of query heads 2h, 2h+1 from attn_core's LDS
// result (ALDS_ORED, ALDS_STAT) into LDS_ATTH; ends with __syncthreads.
MQ_DEV void attn_local_out(float* lds) {
  const int t = tid();
  float o = 0.f;
  if (t < 2 * MQ_D) o = att_single(lds[ALDS_ORED + t], lds[ALDS_STAT + 2 + (t >> 7)]);
  __syncthreads();
  if (t < 2 * MQ_D) lds[LDS_ATTH + t] = o;
  __syncthreads();
}
// Same from the single published partial of kv head h (one kernel per phase, local mode).
MQ_DEV void group_single(const float* part, int h, float* lds) {
  const int t = tid();
  if (t < 2 * MQ_D) {
    const float* src = part_ptr(const_cast<float*>(part), h, 0, t >> 7);
    lds[LDS_ATTH + t] = att_single(ld_coh(src + 4 + (t & 127)), ld_coh(src + 1));
  }
  __syncthreads();
}
// Sync wave, after attn_core: this chunk's partial (m, l, o) of both query heads, and the new
// position's K/V cache row from the chunk that holds it.
MQ_DEV void gattn_publish(const MqDecodeParams& p, int layer, int pos, int h, int j,
                          const GAttn& g, const float* lds) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = lane + 64 * i, jj = t >> 7, d = t & 127;
    st_coh(part_ptr(p.s->part, h, j, jj) + 4 + d, lds[ALDS_ORED + t]);
  }
  if (lane < 2) {
    st_coh(part_ptr(p.s->part, h, j, lane), lds[ALDS_STAT + lane]);
    st_coh(part_ptr(p.s->part, h, j, lane) + 1, lds[ALDS_STAT + 2 + lane]);
  }
  if (g.has_pos) attn_cache_row(p, layer, h, pos, lds);
}
// All threads: merged attention output of query heads 2h, 2h+1 into LDS_ATTH.
MQ_DEV void group_merge(const float* part, int h, int nch, float* lds) {
  attn_merge(part, h, nch, lds, [&](int jj, int d, float o) { lds[LDS_ATTH + jj * MQ_D + d] = o; });
  __syncthreads();
}

// GEMV over rows of 256 elements (the O projection restricted to one kv head's two query
// heads): one wave instruction covers a pair of rows, lanes 0-31 the first and 32-63 the second.
template <int PF>
struct PairSet {
  uint4 w[PF];
  template <class RowPtr>
  MQ_DEV void load(RowPtr rowptr, int nr) {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int np = (nr + 1) / 2;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int it = wave + i * MQ_CWAVES, row = 2 * it + (lane >> 5);
      w[i] = (it < np && row < nr) ? ld_nt16(rowptr(row) + (lane & 31) * 8)
                                   : make_uint4(0, 0, 0, 0);
    }
  }
  template <class RowPtr, class Out>
  MQ_DEV void compute(RowPtr rowptr, int nr, const float* __restrict__ x, Out out) const {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int np = (nr + 1) / 2;
    const float* xs = x + (lane & 31) * 8;
    // items i and i + 1 are reduced together by sum2_halves: lane group k = lane / 16 receives
    // the total of item i + (k & 1), row 2 it + (k >> 1) (the low / high 32-lane half); items past
    // np hold zero weights
#pragma unroll
    for (int i = 0; i < PF; i += 2) {
      const float a0 = dot8_lds(w[i], xs, 0.f);
      const float a1 = i + 1 < PF ? dot8_lds(w[i + 1 < PF ? i + 1 : i], xs, 0.f) : 0.f;
      const float tot = sum2_halves(a0, a1);
      const int k = lane >> 4, ii = i + (k & 1);
      const int it = wave + ii * MQ_CWAVES, row = 2 * it + (k >> 1);
      if ((lane & 15) == 0 && ii < PF && it < np && row < nr) out(row, tot);
    }
    for (int it = wave + PF * MQ_CWAVES; it < np; it += MQ_CWAVES) {
      const int row = 2 * it + (lane >> 5);
      const uint4 v = row < nr ? ld_nt16(rowptr(row) + (lane & 31) * 8) : make_uint4(0, 0, 0, 0);
      const float acc = sum_xor16(row16_sum(dot8_lds(v, xs, 0.f)));
      if ((lane & 31) == 0 && row < nr) out(row, acc);
    }
  }
};
typedef PairSet<3> OPairSet;   // 32 rows (16 pairs) per workgroup at 256 workgroups

MQ_DEV const bf16_t* opart_row(const MqLayerW& w, int h, int r) {
  return w.wo + (size_t)r * MQ_QDIM + 2 * h * MQ_D;
}
MQ_DEV void opart_load(OPairSet& ws, const MqLayerW& w, int h, int j, int NG) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  ws.load([&](int i) { return opart_row(w, h, r0 + i); }, nr);
}
// Input: att of the group's query heads in LDS_ATTH; dot products -> LDS_PR.
MQ_DEV void opart_run(const OPairSet& ws, const MqLayerW& w, int h, int j, int NG, float* lds) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  ws.compute([&](int i) { return opart_row(w, h, r0 + i); }, nr, lds + LDS_ATTH,
             [&](int i, float v) { lds[LDS_PR + i] = v; });
}
MQ_DEV void opart_publish(float* opart, int h, int j, int NG, const float* lds) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) st_coh(opart + h * MQ_H + r0 + t, lds[LDS_PR + t]);
}
// a = x + sum_h opart_h, summed in head order (the single-row form for the multi-kernel mode).
MQ_DEV float a_elem(float x, const float* opart, int r) {
  float a = x;
#pragma unroll
  for (int h = 0; h < MQ_NKV; ++h) a += ld_coh(opart + h * MQ_H + r);
  return a;
}
// Sync wave: a for all 1024 rows from the layer input in LDS_HID -> LDS_IN (gate|up input) and
// LDS_A (residual of the down rows).  Loads of half the rows are issued before any is summed.
MQ_DEV void gu_input(const float* opart, float* lds) {
  const int lane = lane_id();
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    float2 o[4][MQ_NKV];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int h = 0; h < MQ_NKV; ++h)
        o[i][h] = ld_coh2(opart + h * MQ_H + 2 * (lane + 64 * (4 * b + i)));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = lane + 64 * (4 * b + i);
      float2 a = reinterpret_cast<const float2*>(lds + LDS_HID)[q];
#pragma unroll
      for (int h = 0; h < MQ_NKV; ++h) {
        a.x += o[i][h].x;
        a.y += o[i][h].y;
      }
      reinterpret_cast<float2*>(lds + LDS_IN)[q] = a;
      reinterpret_cast<float2*>(lds + LDS_A)[q] = a;
    }
  }
}
// All threads: a for all 1024 rows (thread t: rows 2t, 2t+1), same summation order as
// gu_input and a_elem; ends with __syncthreads.
MQ_DEV void gu_input_all(const float* opart, float* lds) {
  const int t = tid();
  if (t < MQ_H / 2) {
    float2 o[MQ_NKV];
#pragma unroll
    for (int h = 0; h < MQ_NKV; ++h) o[h] = ld_coh2(opart + h * MQ_H + 2 * t);
    float2 a = reinterpret_cast<const float2*>(lds + LDS_HID)[t];
#pragma unroll
    for (int h = 0; h < MQ_NKV; ++h) {
      a.x += o[h].x;
      a.y += o[h].y;
    }
    reinterpret_cast<float2*>(lds + LDS_IN)[t] = a;
    reinterpret_cast<float2*>(lds + LDS_A)[t] = a;
  }
  __syncthreads();
}
// Sync wave: the layer input into LDS_IN and LDS_HID (coherent fp32, or the bf16 embedding row).
MQ_DEV void input_hidden_coh(float* lds, const float* src) {
  const int lane = lane_id();
  float2 v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = ld_coh2(src + 2 * (lane + 64 * i));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    reinterpret_cast<float2*>(lds + LDS_IN)[lane + 64 * i] = v[i];
    reinterpret_cast<float2*>(lds + LDS_HID)[lane + 64 * i] = v[i];
  }
}
MQ_DEV void input_hidden_bf16(float* lds, const bf16_t* src) {
  wave_copy_bf16_1024(lds + LDS_IN, src);
  wave_copy_bf16_1024(lds + LDS_HID, src);
}

// Phase boundary of the head-group kernel.  Order of the workgroup's memory operations: the
// sync wave's output stores (waited for), its barrier arrival, then the compute waves' weight
// prefetch, then the sync wave's barrier polls and input loads.  A workgroup's memory queue is
// first-in first-out in practice, so arriving before the prefetch is issued keeps the arrival
// from waiting behind tens of KB of weight loads, and the prefetch drains while the barrier
// completes.
template <class Epi, class Arrive, class Prefetch, class Wait, class Input>
MQ_DEV void phase_step(Epi epilogue, Arrive arrive, Prefetch prefetch, Wait wait, Input input) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) {
    epilogue();
    wait_all_memory();
    arrive();
  }
  __syncthreads();
  if (wave_id() < MQ_CWAVES) prefetch();
  if (wave_id() == MQ_SYNC_WAVE) {
    wait();
    input();
    wait_all_memory();
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------- kernels
// Reads and validates the step's position and input token.  The result is identical in every
// workgroup, so an invalid step makes all of them return before the first barrier.
MQ_DEV bool step_inputs(const MqDecodeParams& p, const int* tok_in, int& pos, int& tok) {
  // uniform by construction; readfirstlane lets the compiler treat everything derived from them
  // as scalar (uniform branches, no per-lane copies of alternative code paths)
  pos = __builtin_amdgcn_readfirstlane(
      (int)__hip_atomic_load(&p.st->pos.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  tok = __builtin_amdgcn_readfirstlane((int)__hip_atomic_load(
      reinterpret_cast<const uint32_t*>(tok_in), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  if (pos < 0 || pos >= p.max_seq || tok < 0 || tok >= p.vocab) {
    if (blockIdx.x == 0 && tid() == 0)
      __hip_atomic_store(&p.st->sync.err.v, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
  }
  return true;
}

MQ_DEV void hidden_out(const MqDecodeParams& p, int l, int r, float v) {
  st_coh(p.s->hidden + r, v);
  if (p.trace != nullptr) p.trace[(size_t)l * MQ_H + r] = v;
}

MQ_DEV void stamp(const MqDecodeParams& p, int wg, int l, int k) {
  if (p.stamps != nullptr && tid() == 0)
    p.stamps[((size_t)wg * p.num_layers + l) * MQ_NSTAMP + k] = __builtin_amdgcn_s_memrealtime();
}

// Layer `l` of the weight-pointer table copied into LDS, moved to scalar registers: the pointers
// are uniform, and reading them from LDS keeps them off the vector memory queue, where the
// weight prefetches of the previous phase would delay them.
MQ_DEV uintptr_t uniform_u64(uintptr_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (uintptr_t)(((uint64_t)hi << 32) | lo);
}
MQ_DEV MqLayerW lds_layer(const MqLayerW* table, int l) {
  const MqLayerW& t = table[l];
  MqLayerW w;
#define MQ_U(f) w.f = reinterpret_cast<const bf16_t*>(uniform_u64(reinterpret_cast<uintptr_t>(t.f)))
  MQ_U(in_ln); MQ_U(wq); MQ_U(wk); MQ_U(wv); MQ_U(q_norm); MQ_U(k_norm);
  MQ_U(wo); MQ_U(post_ln); MQ_U(wg); MQ_U(wu); MQ_U(wd);
#undef MQ_U
  return w;
}
static_assert(sizeof(MqLayerW) == 11 * sizeof(void*), "MqLayerW holds exactly the 11 pointers");

// Sync wave: waits until the multi-step epoch reaches `target` (the last workgroup of a step
// publishes it after resetting the step's sync state), then the workgroup proceeds.
MQ_DEV void step_wait(const MqDecodeParams& p, uint32_t target) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) {
    const int lane = lane_id();
    uint32_t spins = 0;
    while (true) {
      uint32_t v = 0;
      if (lane == 0)
        v = __hip_atomic_load(&p.st->steps.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else if (lane == 63)
        v = __hip_atomic_load(&p.st->sync.err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t e = __builtin_amdgcn_readlane(v, 63);
      const uint32_t c = __builtin_amdgcn_readlane(v, 0);
      if (e != 0 || (int32_t)(c - target) >= 0) break;
      __builtin_amdgcn_s_sleep(2);   // back-off, as in the grid barrier
      if (++spins > MQ_SPIN_LIMIT) {
        if (lane == 0)
          __hip_atomic_store(&p.st->sync.err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// EARLY: the long-context variant (chosen per launch by the host, MqDecodeParams.early_kv): a
// layer's K rows are issued right after its q|k|v weights, one phase earlier than otherwise, so
// they stream in during the q|k|v dot products and the group barrier; its V rows follow at the
// q|k|v barrier.  Both K/V loads have a fixed instruction count (kv_block_load_all), so the
// compiler waits for the q|k|v weights alone.  The variant is correct at any position: steps
// where a workgroup has no chunk load a stand-in K row and ignore it (and issue their gate|up
// weights at the q|k|v boundary, as in the other variant), and chunks of <= 8 positions use the
// 7-wave layout.  (One kernel holding both variants spilled ~600 VGPRs.)
template <bool EARLY>
__global__ void __launch_bounds__(MQ_THREADS) mq_decode_persistent_kernel(MqDecodeParams p) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  __shared__ MqLayerW s_layers[MQ_MAX_LAYERS];
  const int G = gridDim.x, wg = blockIdx.x;
  {
    const int nw = p.num_layers * (int)(sizeof(MqLayerW) / 4);
    for (int i = tid(); i < nw; i += MQ_THREADS)
      reinterpret_cast<uint32_t*>(s_layers)[i] = reinterpret_cast<const uint32_t*>(p.layers)[i];
    __syncthreads();
  }
  const int h = wg % MQ_GROUPS, j = wg / MQ_GROUPS, NG = G / MQ_GROUPS;
  MqSync* sy = &p.st->sync;
  MqScratch* s = p.s;
  int r0h, nrh;
  row_range(MQ_H, wg, G, r0h, nrh);
  // the step-done epoch before this launch: read by every workgroup before any can complete the
  // first step (completion needs every workgroup's arrival at the LM head)
  const uint32_t epoch0 = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&p.st->steps.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  QkvSet wq;
  OPairSet wo;
  GateUpSet wgu;
  DownSet wd;
  KvBlock kv;
  if (p.num_layers > 0) gqkv_load(wq, lds_layer(s_layers, 0), h, j, NG);
  for (int step = 0; step < p.nsteps; ++step) {
    int pos, tok;
    if (!step_inputs(p, step == 0 ? p.tok_in : p.tok_out + (step - 1), pos, tok)) return;
    const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, true);
    const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
    const bf16_t* cs = p.cos + (size_t)pos * MQ_D;
    const bf16_t* sn = p.sin + (size_t)pos * MQ_D;
    uint32_t nbar = 0, ngb = 0;
    phase_step(MQ_NOTHING, MQ_NOTHING, MQ_NOTHING, MQ_NOTHING, [&] { input_hidden_bf16(lds, xe); });
    // K/V block of this workgroup's chunk (EARLY: row 0 for a workgroup without one)
    const bool small = EARLY ? false : ga.small;
    const int kv0 = ga.active ? ga.p0 : 0;
    const int kv1 = ga.active ? min(ga.p1, ga.p0 + MQ_ATT_BLOCK) : 1;
    // read-only stand-in row for lanes that must not fetch a cache row (row 0 of the cos table)
    const bf16_t* kv_dummy = p.cos + (lane_id() & 15) * 8;
    auto k_early = [&](int l) {
      kv_block_load_all<true, false>(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), kv0, kv1,
                                     pos, kv_dummy);
    };
    if constexpr (EARLY) {
      if (p.num_layers > 0) k_early(0);
    }
    for (int l = 0; l < p.num_layers; ++l) {
      const MqLayerW w = lds_layer(s_layers, l);
      stamp(p, wg, l, 0);
      gqkv_run(wq, w, h, j, NG, lds);
      stamp(p, wg, l, 1);
      // the gate|up weights go out two phases ahead, during the attention phase, from workgroups
      // without an attention chunk; the others issue them once they have arrived at the grid
      // barrier after the O projection (a deep queue stalls the issue of loads and would delay
      // their attention, the partial merge and the O projection, which are on the critical path).
      // Workgroups with a chunk issue its K/V rows here instead, after arriving: issued before
      // the q|k|v dot products (whose loads are conditional), they made the compiler's wait for
      // the q|k|v weights wait for them too.
      phase_step([&] { gqkv_publish(s->qkv, h, j, NG, lds); },
                 [&] { group_barrier_arrive(sy, h); },
                 [&] {
                   if constexpr (EARLY) {
                     // a workgroup without a chunk (some cache lengths below ~990 leave the
                     // last one idle) takes the gate|up weights here, as in the other variant
                     if (!ga.active) {
                       gu_load(wgu, w, wg, G);
                     } else {
                       kv_block_load_all<false, true>(kv, kv_base(p.kc, p, l, h),
                                                      kv_base(p.vc, p, l, h), kv0, kv1, pos,
                                                      kv_dummy);
                       if (ga.local) opart_load(wo, w, h, j, NG);
                     }
                   } else {
                     if (!ga.active) {
                       gu_load(wgu, w, wg, G);
                     } else {
                       kv_block_load(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), ga.p0,
                                     min(ga.p1, ga.p0 + MQ_ATT_BLOCK), pos, ga.small);
                       // local mode: no exchange follows the attention, so the O rows go now
                       if (ga.local) opart_load(wo, w, h, j, NG);
                     }
                   }
                 },
                 [&] { group_barrier_wait(sy, h, (++ngb) * (uint32_t)NG); },
                 [&] { if (ga.active) attn_input(s->qkv, w.q_norm, w.k_norm, cs, sn, h, lds); });
      stamp(p, wg, l, 2);
      if (ga.active) {
        attn_prologue(lds);
        __syncthreads();
        attn_core(p, l, h, ga.p0, ga.p1, pos, kv, lds, small);
      }
      stamp(p, wg, l, 3);
      if (ga.local) {
        attn_local_out(lds);
      } else {
        phase_step([&] { if (ga.active) gattn_publish(p, l, pos, h, j, ga, lds); },
                   [&] { group_barrier_arrive(sy, h); },
                   [&] { opart_load(wo, w, h, j, NG); },
                   [&] { group_barrier_wait(sy, h, (++ngb) * (uint32_t)NG); }, MQ_NOTHING);
        group_merge(s->part, h, ga.nch, lds);
      }
      stamp(p, wg, l, 4);
      opart_run(wo, w, h, j, NG, lds);
      stamp(p, wg, l, 5);
      phase_step([&] {
                   opart_publish(&s->opart[0][0], h, j, NG, lds);
                   // local mode: the new position's K/V row (ALDS_KN/VN are still intact)
                   if (ga.local && ga.has_pos) attn_cache_row(p, l, h, pos, lds);
                 },
                 [&] { grid_barrier_arrive(sy); },
                 [&] { if (ga.active) gu_load(wgu, w, wg, G); },
                 [&] { grid_barrier_wait(sy, (++nbar) * (uint32_t)G); }, MQ_NOTHING);
      gu_input_all(&s->opart[0][0], lds);
      stamp(p, wg, l, 6);
      gu_run(wgu, w, wg, G, lds);
      stamp(p, wg, l, 7);
      phase_step([&] { gu_publish(s->mlp, wg, G, lds); },
                 [&] { grid_barrier_arrive(sy); },
                 [&] { down_load(wd, w, wg, G); },
                 [&] { grid_barrier_wait(sy, (++nbar) * (uint32_t)G); },
                 [&] { wave_copy_coh<MQ_I>(lds + LDS_IN, s->mlp); });
      stamp(p, wg, l, 8);
      down_run(wd, w, wg, G, lds);
      stamp(p, wg, l, 9);
      phase_step(
          [&] {
            float res = lane_id() < nrh ? lds[LDS_A + r0h + lane_id()] : 0.f;
            down_publish(wg, G, lds, res, [&](int r, float v) { hidden_out(p, l, r, v); });
          },
          [&] { grid_barrier_arrive(sy); },
          [&] {
            if (l + 1 < p.num_layers) {
              gqkv_load(wq, lds_layer(s_layers, l + 1), h, j, NG);
              if constexpr (EARLY) k_early(l + 1);
            }
          },
          [&] { grid_barrier_wait(sy, (++nbar) * (uint32_t)G); },
          [&] { input_hidden_coh(lds, s->hidden); });
      stamp(p, wg, l, 10);
    }
    const bool more = step + 1 < p.nsteps;
    lm_head_run(p, wg, G, lds, p.tok_out + step, p.nsteps == 1 ? p.logits : nullptr, pos, true,
                false, more, epoch0 + (uint32_t)step + 1);
    if (more) {
      // the next step's first weights do not depend on its token: in flight during the wait
      if (p.num_layers > 0) gqkv_load(wq, lds_layer(s_layers, 0), h, j, NG);
      step_wait(p, epoch0 + (uint32_t)step + 1);
    }
  }
}

// One kernel per phase of the head-group step (kernel boundaries replace the barriers).  Every
// value is computed by the same functions in the same order as in the persistent kernel, so
// both modes produce bit-identical results.
template <int PH>
__global__ void __launch_bounds__(MQ_THREADS) mq_decode_phase_kernel(MqDecodeParams p, int l) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  const int G = gridDim.x, wg = blockIdx.x;
  int pos, tok;
  if (!step_inputs(p, p.tok_in, pos, tok)) return;
  MqScratch* s = p.s;
  MqSync* sy = &p.st->sync;
  const int h = wg % MQ_GROUPS, j = wg / MQ_GROUPS, NG = G / MQ_GROUPS;
  const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
  // the layer input: the embedding row for layer 0, else the previous layer's output
  auto load_x = [&](float* dst) {
    if (l == 0) wave_copy_bf16_1024(dst, xe);
    else wave_copy_coh<MQ_H>(dst, s->hidden);
  };
  if constexpr (PH == 5) {
    phase_sync(sy, 0, false, MQ_NOTHING, [&] {
      if (p.num_layers == 0) wave_copy_bf16_1024(lds + LDS_IN, xe);
      else wave_copy_coh<MQ_H>(lds + LDS_IN, s->hidden);
    });
    lm_head_run(p, wg, G, lds, p.tok_out, p.logits, pos, true);
  } else {
    const MqLayerW w = p.layers[l];
    if constexpr (PH == 0) {
      QkvSet ws;
      gqkv_load(ws, w, h, j, NG);
      phase_sync(sy, 0, false, MQ_NOTHING, [&] { load_x(lds + LDS_IN); });
      gqkv_run(ws, w, h, j, NG, lds);
      phase_finish([&] { gqkv_publish(s->qkv, h, j, NG, lds); });
    }
    if constexpr (PH == 1) {
      const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, false);
      if (ga.active) {
        KvBlock kv;
        kv_block_load(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), ga.p0,
                      min(ga.p1, ga.p0 + MQ_ATT_BLOCK), pos, ga.small);
        phase_sync(sy, 0, false, MQ_NOTHING, [&] {
          attn_input(s->qkv, w.q_norm, w.k_norm, p.cos + (size_t)pos * MQ_D,
                     p.sin + (size_t)pos * MQ_D, h, lds);
        });
        attn_prologue(lds);
        __syncthreads();
        attn_core(p, l, h, ga.p0, ga.p1, pos, kv, lds, ga.small);
        phase_finish([&] { gattn_publish(p, l, pos, h, j, ga, lds); });
      }
    }
    if constexpr (PH == 2) {
      const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, false);
      OPairSet ws;
      opart_load(ws, w, h, j, NG);
      if (ga.local)
        group_single(s->part, h, lds);
      else
        group_merge(s->part, h, ga.nch, lds);
      opart_run(ws, w, h, j, NG, lds);
      phase_finish([&] { opart_publish(&s->opart[0][0], h, j, NG, lds); });
    }
    if constexpr (PH == 3) {
      GateUpSet ws;
      gu_load(ws, w, wg, G);
      phase_sync(sy, 0, false, MQ_NOTHING, [&] {
        load_x(lds + LDS_HID);
        wait_all_memory();
        gu_input(&s->opart[0][0], lds);
      });
      gu_run(ws, w, wg, G, lds);
      phase_finish([&] { gu_publish(s->mlp, wg, G, lds); });
    }
    if constexpr (PH == 4) {
      DownSet ws;
      down_load(ws, w, wg, G);
      int r0h, nrh;
      row_range(MQ_H, wg, G, r0h, nrh);
      const int t = lane_id();
      float res = 0.f;
      if (wave_id() == MQ_SYNC_WAVE && t < nrh) {
        const float x = l == 0 ? bf16_to_f32(xe[r0h + t]) : ld_coh(s->hidden + r0h + t);
        res = a_elem(x, &s->opart[0][0], r0h + t);
      }
      phase_sync(sy, 0, false, MQ_NOTHING, [&] { wave_copy_coh<MQ_I>(lds + LDS_IN, s->mlp); });
      down_run(ws, w, wg, G, lds);
      phase_finish([&] {
        down_publish(wg, G, lds, res, [&](int r, float v) { hidden_out(p, l, r, v); });
      });
    }
  }
}

// ------------------------------------------------------------------ op-level kernels
// (a) fused RMSNorm + q|k|v GEMV, then q/k RMSNorm + RoPE + K/V cache write at `pos`.
__global__ void __launch_bounds__(MQ_THREADS) mq_op_qkv_kernel(MqDecodeParams p, int l,
                                                                const bf16_t* x) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  QkvSet ws;
  qkv_load(ws, p.layers[l], blockIdx.x, gridDim.x);
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING, [&] { wave_copy_bf16_1024(lds + LDS_IN, x); });
  qkv_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] { qkv_publish(p.s->qkv, blockIdx.x, gridDim.x, lds); });
}
__global__ void __launch_bounds__(MQ_THREADS) mq_op_rope_kernel(MqDecodeParams p, int l, int pos,
                                                                 float* q_out) {
  __shared__ __align__(16) float lds[ALDS_WML];
  const int h = blockIdx.x;
  const MqLayerW w = p.layers[l];
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING, [&] {
    attn_input(p.s->qkv, w.q_norm, w.k_norm, p.cos + (size_t)pos * MQ_D,
               p.sin + (size_t)pos * MQ_D, h, lds);
  });
  attn_prologue(lds);
  __syncthreads();
  if (tid() < 256) q_out[2 * h * MQ_D + tid()] = lds[ALDS_QS + tid()];
  if (wave_id() == MQ_SYNC_WAVE) attn_cache_row(p, l, h, pos, lds);
}
// (b) attention of pre-rotated queries over cache rows [0, cache_len) -> partials, then merge.
__global__ void __launch_bounds__(MQ_THREADS) mq_op_attn_kernel(MqDecodeParams p, int l,
                                                                 const float* q_hat,
                                                                 int cache_len, int nch) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  const AttnItem it = attn_item(blockIdx.x, nch, cache_len);
  if (!it.active) return;
  KvBlock kv;
  kv_block_load(kv, kv_base(p.kc, p, l, it.h), kv_base(p.vc, p, l, it.h), it.p0,
                min(it.p1, it.p0 + MQ_ATT_BLOCK), -1);
  if (tid() < 256) lds[ALDS_QS + tid()] = q_hat[2 * it.h * MQ_D + tid()];
  __syncthreads();
  attn_core(p, l, it.h, it.p0, it.p1, -1, kv, lds);
  attn_write_partial(p.s->part, it.h, it.c, lds);
}
__global__ void __launch_bounds__(MQ_THREADS) mq_op_merge_kernel(MqDecodeParams p, int nch,
                                                                  float* att_out) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  attn_merge_head(p.s->part, blockIdx.x, nch, att_out, lds);
}
// O projection with residual: a_out = W_o att + x (x bf16, the layer input).
__global__ void __launch_bounds__(MQ_THREADS) mq_op_o_kernel(MqDecodeParams p, int l,
                                                              const float* att, const bf16_t* x,
                                                              float* a_out) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  OSet ws;
  o_load(ws, p.layers[l], blockIdx.x, gridDim.x);
  int r0, nr;
  row_range(MQ_H, blockIdx.x, gridDim.x, r0, nr);
  float res = lane_id() < nr ? bf16_to_f32(x[r0 + lane_id()]) : 0.f;
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING,
             [&] { wave_copy_coh<MQ_QDIM>(lds + LDS_IN, att); });
  o_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] { o_publish(a_out, blockIdx.x, gridDim.x, lds, res); });
}
// (c) SwiGLU MLP with residual: x_out = bf16(W_d (silu(W_g n) * W_u n) + a), n = RMSNorm(a).
__global__ void __launch_bounds__(MQ_THREADS) mq_op_gateup_kernel(MqDecodeParams p, int l,
                                                                   const float* a) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  GateUpSet ws;
  gu_load(ws, p.layers[l], blockIdx.x, gridDim.x);
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING, [&] { wave_copy_coh<MQ_H>(lds + LDS_IN, a); });
  gu_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] { gu_publish(p.s->mlp, blockIdx.x, gridDim.x, lds); });
}
__global__ void __launch_bounds__(MQ_THREADS) mq_op_down_kernel(MqDecodeParams p, int l,
                                                                 const float* a, bf16_t* x_out) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  DownSet ws;
  down_load(ws, p.layers[l], blockIdx.x, gridDim.x);
  int r0, nr;
  row_range(MQ_H, blockIdx.x, gridDim.x, r0, nr);
  float res = lane_id() < nr ? ld_coh(a + r0 + lane_id()) : 0.f;
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING,
             [&] { wave_copy_coh<MQ_I>(lds + LDS_IN, p.s->mlp); });
  down_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] {
    down_publish(blockIdx.x, gridDim.x, lds, res,
                 [&](int r, float v) { x_out[r] = f32_to_bf16(v); });
  });
}
// (d) final RMSNorm + LM head + argmax of a given bf16 hidden state; `round_norm` rounds the
// normalised vector to bf16 first (the prefill path).
__global__ void __launch_bounds__(MQ_THREADS) mq_op_lm_kernel(MqDecodeParams p, const bf16_t* x,
                                                               int* tok_out, float* logits,
                                                               bool round_norm) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING,
             [&] { wave_copy_bf16_1024(lds + LDS_IN, x); });
  lm_head_run(p, blockIdx.x, gridDim.x, lds, tok_out, logits, 0, false, round_norm);
}

// ---------------------------------------------------------------------- state kernels
__global__ void mq_fill_state_kernel(MqState* st, int pos, int clear_err) {
  const int t = threadIdx.x;
  if (t < MQ_BAR_STRIPES) st->sync.bar[t].v = 0;
  if (t < MQ_NKV) st->sync.attn[t].v = 0;
  if (t == 0) {
    st->sync.done.v = 0;
    if (clear_err) st->sync.err.v = 0;
    st->sync.argmax.v = 0;
    st->pos.v = (uint32_t)pos;
    st->steps.v = 0;
  }
}
__global__ void mq_zero_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

// ------------------------------------------------------------------------ host side
static int g_cu_count = 0;
static int g_coop_ok = -1;
static int g_persist_blocks_per_cu = 0;

static int device_info() {
  if (g_cu_count > 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  int cu = 0, coop = 0;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess)
    coop = 0;
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &nb, reinterpret_cast<const void*>(mq_decode_persistent_kernel<false>), MQ_THREADS, 0) !=
      hipSuccess)
    nb = 0;
  g_cu_count = cu;
  g_coop_ok = coop;
  g_persist_blocks_per_cu = nb;
  return 0;
}

int mq_decode_grid(int mode, int* grid_out) {
  if (device_info() != 0) return -1;
  if (mode == MQ_MODE_PERSISTENT) {
    if (!g_coop_ok || g_persist_blocks_per_cu < 1) return -2;
  }
  // one 512-thread workgroup per CU, a whole number of kv-head groups (8)
  *grid_out = g_cu_count / MQ_GROUPS * MQ_GROUPS;
  return 0;
}

static int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -(int)e - 1000;
}

int mq_launch_decode(const MqDecodeParams& p, int mode, int grid, hipStream_t stream) {
  if (grid < 64 || grid > 4096 || grid % MQ_GROUPS != 0) return -3;
  if (mode == MQ_MODE_PERSISTENT) {
    MqDecodeParams pc = p;
    void* args[] = {&pc};
    const void* fn = p.early_kv ? reinterpret_cast<const void*>(mq_decode_persistent_kernel<true>)
                                : reinterpret_cast<const void*>(mq_decode_persistent_kernel<false>);
    hipError_t e = hipLaunchCooperativeKernel(fn, dim3(grid), dim3(MQ_THREADS), args, 0, stream);
    return e == hipSuccess ? 0 : -(int)e - 1000;
  }
  for (int l = 0; l < p.num_layers; ++l) {
    mq_decode_phase_kernel<0><<<grid, MQ_THREADS, 0, stream>>>(p, l);
    mq_decode_phase_kernel<1><<<grid, MQ_THREADS, 0, stream>>>(p, l);
    mq_decode_phase_kernel<2><<<grid, MQ_THREADS, 0, stream>>>(p, l);
    mq_decode_phase_kernel<3><<<grid, MQ_THREADS, 0, stream>>>(p, l);
    mq_decode_phase_kernel<4><<<grid, MQ_THREADS, 0, stream>>>(p, l);
  }
  mq_decode_phase_kernel<5><<<grid, MQ_THREADS, 0, stream>>>(p, 0);
  return launch_status();
}

int mq_launch_fill_state(MqState* st, int pos, hipStream_t stream, bool clear_err) {
  mq_fill_state_kernel<<<1, 64, 0, stream>>>(st, pos, clear_err ? 1 : 0);
  return launch_status();
}

int mq_launch_zero(void* ptr, size_t bytes, hipStream_t stream) {
  if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(ptr) & 15) != 0) return -3;
  if (bytes == 0) return 0;
  const size_t n16 = bytes / 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  mq_zero_kernel<<<(unsigned)blocks, 256, 0, stream>>>(reinterpret_cast<uint4*>(ptr), n16);
  return launch_status();
}

int mq_read_error(MqState* st, hipStream_t stream, uint32_t* err_out) {
  uint32_t v = 0;
  if (hipMemcpyAsync(&v, &st->sync.err.v, 4, hipMemcpyDeviceToHost, stream) != hipSuccess)
    return -1;
  if (hipStreamSynchronize(stream) != hipSuccess) return -1;
  *err_out = v;
  return 0;
}

int mq_launch_op_qkv_rope(const MqDecodeParams& p, int layer, const bf16_t* x, int pos,
                          float* q_out, int grid, hipStream_t stream) {
  mq_op_qkv_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, x);
  mq_op_rope_kernel<<<MQ_NKV, MQ_THREADS, 0, stream>>>(p, layer, pos, q_out);
  return launch_status();
}

int mq_launch_op_attention(const MqDecodeParams& p, int layer, const float* q_hat, int cache_len,
                           float* att_out, int grid, hipStream_t stream) {
  const int nch = mq_attn_nchunks(cache_len, grid);
  mq_op_attn_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, q_hat, cache_len, nch);
  mq_op_merge_kernel<<<MQ_NKV, MQ_THREADS, 0, stream>>>(p, nch, att_out);
  return launch_status();
}

// ------------------------------------------------------ allocation-free attention op
// Device memory of mq_launch_op_attention_noalloc: one MqScratch (its split-K partials are the
// only part the attention op uses) in a file-scope device array, so callers that cannot allocate
// (code under graph capture, serving loops) need no workspace.  Each GPU the library runs on
// holds its own copy until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is only a stand-in for the symbol): the device address of each
// GPU's copy comes from hipGetSymbolAddress, resolved once per device with that device current.
static __device__ __align__(256) unsigned char scratch[MQ_NOALLOC_SCRATCH_BYTES];
static_assert(sizeof(MqScratch) <= MQ_NOALLOC_SCRATCH_BYTES, "scratch holds one MqScratch");

#define MQ_NOALLOC_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MQ_NOALLOC_MAX_DEVICES] = {};

// Device address of the current device's `scratch` (resolved on the first call per device).
static int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MQ_NOALLOC_MAX_DEVICES) return -1;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return -2;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int mq_launch_op_attention_noalloc(const MqDecodeParams& p, int layer, const float* q_hat,
                                   int cache_len, float* att_out, int grid, hipStream_t stream) {
  if (mq_attn_nchunks(cache_len, grid) > MQ_MAX_CHUNKS) return -3;
  void* s = nullptr;
  const int rc = scratch_address(&s);
  if (rc != 0) return rc;
  MqDecodeParams pc = p;
  pc.s = static_cast<MqScratch*>(s);
  // every partial the merge reads is written by the attention kernel first: nothing to clear
  return mq_launch_op_attention(pc, layer, q_hat, cache_len, att_out, grid, stream);
}

int mq_launch_op_mlp(const MqDecodeParams& p, int layer, const float* a_in, bf16_t* x_out,
                     int grid, hipStream_t stream) {
  mq_op_gateup_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, a_in);
  mq_op_down_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, a_in, x_out);
  return launch_status();
}

int mq_launch_op_layer(const MqDecodeParams& p, int layer, const bf16_t* x, int pos,
                       bf16_t* x_out, int grid, hipStream_t stream) {
  // Scratch use: q_hat -> s->mlp (free until gate/up), attention -> s->att, O output -> s->a.
  MqScratch* s = p.s;
  const int nch = mq_attn_nchunks(pos + 1, grid);
  mq_op_qkv_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, x);
  mq_op_rope_kernel<<<MQ_NKV, MQ_THREADS, 0, stream>>>(p, layer, pos, s->mlp);
  mq_op_attn_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, s->mlp, pos + 1, nch);
  mq_op_merge_kernel<<<MQ_NKV, MQ_THREADS, 0, stream>>>(p, nch, s->att);
  mq_op_o_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, s->att, x, s->a);
  mq_op_gateup_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, s->a);
  mq_op_down_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, layer, s->a, x_out);
  return launch_status();
}

int mq_launch_op_lm_head(const MqDecodeParams& p, const bf16_t* x, int* tok_out, float* logits,
                         int grid, hipStream_t stream) {
  mq_op_lm_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, x, tok_out, logits, false);
  return launch_status();
}

int mq_launch_lm_head_bf16norm(const MqDecodeParams& p, const bf16_t* x, int* tok_out,
                               float* logits, int grid, hipStream_t stream) {
  mq_op_lm_kernel<<<grid, MQ_THREADS, 0, stream>>>(p, x, tok_out, logits, true);
  return launch_status();
}
