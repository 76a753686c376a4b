// Batch-1 bf16 decode for the Qwen3-0.6B layer shape on gfx950.
//
// One decode step = 28 layers x 5 phases + the LM head:
//   P1  RMSNorm(x) and the fused q|k|v GEMV (4096 rows x 1024)
//   P2  per-(kv head, position chunk) attention: q/k RMSNorm + RoPE prologue, K/V cache write of
//       the new position, two-pass softmax over the chunk; with several chunks per head each
//       publishes a split-K partial (m, l, o[128]), merged by every workgroup that needs the
//       head's output
//   P3  O GEMV (1024 x 2048) + residual
//   P4  RMSNorm(a) + gate/up GEMVs (2 x 3072 x 1024) + silu(g) * u
//   P5  down GEMV (1024 x 3072) + residual, rounded to bf16 (the layer output)
//   LM  final RMSNorm + LM-head GEMV (vocab x 1024) + argmax (packed 64-bit atomic max)
// The phases run either inside one persistent cooperative kernel, which hands data between
// workgroups through device-coherent exchange words that carry the layer's epoch (no barrier
// between workgroups at all, against 225 grid.sync() per token in the reference's
// ldg_decode_kernel, csrc/megakernel/fused_decode_ldg_kernel.inl:5-259), or as one kernel launch
// per phase.
//
// Workgroup organisation (512 threads): waves 0..6 are compute waves, wave 7 is the sync wave.
// Per phase the compute waves finish their dot products; the sync wave publishes the outputs with
// coherent (sc1) stores; then the compute waves issue the NEXT phase's weight loads into
// registers while the sync wave (or, for the two larger exchanges, every wave) polls the next
// phase's input words until they carry the expected epoch and copies them into LDS.  Because gfx9
// returns a wave's loads in order, keeping the prefetches out of the sync wave is what lets the
// exchange proceed while weights stream in.
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
#define LDS_QA (LDS_AROW + MQ_CWAVES * 256)   // [4][64][8] bf16: q-hat as the MFMA A operand
#define MQ_LDS_FLOATS (LDS_QA + 4 * 64 * 4)

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
//
// Paced prefetch (`paced`, the persistent kernel's prefetches): a wave sleeps MQ_PF_PACE x 64
// clocks between consecutive 1 KB wave loads.  The CU returns loads in order, so an exchange's
// poll issued behind a burst of tens of KB of weight loads waits for them to drain; issued 1 KB
// at a time the weights still land within the exchange (which lasts ~2.5 us) while the queue
// ahead of each poll stays short.  Measured per token, chained, A/B on one box:
//   pause between loads 0 / 2 / 3 / 4 / 5 / 6: 521.1 / 517.6 / 514.6 / 512.7 / 514.2 / 518.0 us
//   at pos 128, 621.5 / 624.1 / 622.3 / 621.1 / 622.2 / 626.6 at pos 4096;
//   pause between items (rows of 2 or 3 loads) instead, 0 / 1 / 3 / 8 / 12 / 16 / 24 / 32:
//   520.3 / 520.1 / 520.7 / 518.9 / 516.7 / 518.1 / 534.7 / 556.7 us at pos 128.
#define MQ_PF_PACE 4
template <int K, int S, int PF>
struct RowSet {
  static constexpr int KS = K / S;
  static constexpr int NL = KS / 512;
  static_assert(KS % 512 == 0, "segments are whole 512-element wave loads");
  uint4 w[PF][NL];

  // fixed: items past the row count load row 0 instead of zeros (their totals are never handed
  // out), so the number of loads after earlier ones is known to the compiler
  template <class RowPtr>
  MQ_DEV void load(RowPtr rowptr, int nr, bool paced = false, bool fixed = false) {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int nitems = nr * S;
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int it0 = wave + j * MQ_CWAVES;
      const int it = fixed && it0 >= nitems ? 0 : it0;
      if (it < nitems) {
        const bf16_t* r = rowptr(it / S) + (it % S) * KS + lane * 8;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
          if (paced && (j > 0 || l > 0)) __builtin_amdgcn_s_sleep(MQ_PF_PACE);
          w[j][l] = ld_nt16(r + l * 512);
        }
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

// Sync wave: polls P (value, epoch) words per lane (word idx(i) of `src` for lane's i < P) until
// every one carries epoch e, then hands out(i, value).  Only words still carrying an old epoch are
// loaded again.  e == 0 takes the words as they are: only the one-kernel-per-phase mode passes
// it, for words written by an earlier kernel; the persistent kernel's epochs are never 0
// (mq_xep_epoch).  A set error flag (read on every 16th round) or the spin bound ends the wait
// early; the step's results are then invalid and mq_decoder_check reports it.
template <int P, class Idx, class Out>
MQ_DEV void x_poll(const uint64_t* src, Idx idx, uint32_t e, MqSync* sy, Out out) {
  const int lane = lane_id();
  uint64_t v[P];
#pragma unroll
  for (int i = 0; i < P; ++i) v[i] = ld_coh64(src + idx(i));
  if (e != 0) {
    uint32_t spins = 0;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < P; ++i) ok = ok && xepoch(v[i]) == e;
      if (__all(ok)) break;
      uint32_t ev = 0;
      if (lane == 0 && (spins & 15) == 15)
        ev = __hip_atomic_load(&sy->err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__builtin_amdgcn_readlane(ev, 0) != 0) break;
      if (++spins > MQ_SPIN_LIMIT) {
        if (lane == 0)
          __hip_atomic_store(&sy->err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (xepoch(v[i]) != e) v[i] = ld_coh64(src + idx(i));
    }
  }
#pragma unroll
  for (int i = 0; i < P; ++i) out(i, xvalue(v[i]));
}
// The N contiguous words of src into LDS dst (and dst2 if given) as fp32.
template <int N>
MQ_DEV void x_gather(float* dst, float* dst2, const uint64_t* src, uint32_t e, MqSync* sy) {
  static_assert(N % 64 == 0, "whole words per lane");
  const int lane = lane_id();
  x_poll<N / 64>(src, [&](int i) { return lane + 64 * i; }, e, sy, [&](int i, float v) {
    dst[lane + 64 * i] = v;
    if (dst2 != nullptr) dst2[lane + 64 * i] = v;
  });
}

// Phase boundary inside one kernel of the one-kernel-per-phase mode and the op-level kernels
// (the kernel boundaries order the phases).  Compute waves arrive with this phase's dot products
// in LDS and the next phase's weight prefetch in flight.  The sync wave then runs `epilogue()`
// (finishes this phase's outputs and publishes them with coherent stores), waits for those
// stores and runs `input()` (the next phase's input vector into LDS).  The compute waves never
// wait for a store, so their prefetches are never waited on either.
template <class Epi, class Input>
MQ_DEV void phase_sync(Epi epilogue, Input input) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) {
    epilogue();
    wait_all_memory();
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
// Tagged fp32 exchange words (the O-projection partials, the MLP vector and the split-mode
// attention partials): the two lowest mantissa bits of each value carry xtag(e) = 1 + e mod 3
// for the layer's exchange epoch e, so a reader polls the data itself, with no store
// acknowledgement, counter or separate barrier.  The buffers alternate by layer parity and every
// word of a buffer is rewritten in every layer of its parity (or was cleared to zero, which no
// tag matches), so the word a reader may see before the new one was written one or two epochs
// earlier and carries another tag.  A workgroup cannot run two layers ahead of another, since
// every layer needs every workgroup's values.  The one-kernel-per-phase mode publishes the same
// truncated values with the same epochs (and reads without polling), so the modes stay
// bit-identical and either may follow the other; the truncation is below 2^-22 relative, far
// under the bf16 rounding these values meet downstream.  The epochs of consecutive layers stay
// consecutive across the wrap of the epoch count (mq_xep_epoch), so the three tags stay distinct.
MQ_DEV uint32_t xtag(uint32_t e) { return mq_xtag(e); }
MQ_DEV uint32_t tag_bits(float v, uint32_t e) { return (__float_as_uint(v) & ~3u) | xtag(e); }
MQ_DEV float untag(uint32_t u) { return __uint_as_float(u & ~3u); }
MQ_DEV void st_tag(float* p, float v, uint32_t e) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), tag_bits(v, e), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// The same for a word read only on the writer's XCD (st_local32).
MQ_DEV void st_tag_local(float* p, float v, uint32_t e) {
  st_local32(reinterpret_cast<uint32_t*>(p), tag_bits(v, e));
}
MQ_DEV bool tag_ok2(uint64_t w, uint32_t tag) {
  return ((uint32_t)w & 3u) == tag && ((uint32_t)(w >> 32) & 3u) == tag;
}
// All threads: P 64-bit words per thread (two tagged values each, word idx(i)) polled until both
// tags are `tag` (tag < 0: taken as they are), then out(i, lo, hi) with the tags removed.  Only
// stale words are loaded again.  A set error flag (read on every 16th round) or the spin bound
// ends the wait early, as in x_poll.
template <int P, class Idx, class Out>
MQ_DEV void tag_poll_all(const float* src, Idx idx, int tag, MqSync* sy, Out out) {
  uint64_t w[P];
#pragma unroll
  for (int i = 0; i < P; ++i) w[i] = ld_coh64(reinterpret_cast<const uint64_t*>(src) + idx(i));
  if (tag >= 0) {
    uint32_t spins = 0;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < P; ++i) ok = ok && tag_ok2(w[i], (uint32_t)tag);
      if (__all(ok)) break;
      uint32_t ev = 0;
      if (lane_id() == 0 && (spins & 15) == 15)
        ev = __hip_atomic_load(&sy->err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__builtin_amdgcn_readlane(ev, 0) != 0) break;
      if (++spins > MQ_SPIN_LIMIT) {
        if (lane_id() == 0)
          __hip_atomic_store(&sy->err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (!tag_ok2(w[i], (uint32_t)tag))
          w[i] = ld_coh64(reinterpret_cast<const uint64_t*>(src) + idx(i));
    }
  }
#pragma unroll
  for (int i = 0; i < P; ++i) out(i, untag((uint32_t)w[i]), untag((uint32_t)(w[i] >> 32)));
}

// 2^x with the hardware v_exp_f32 (results below the normal range flush to zero, as the
// reference's fast-math __expf does); used for softmax weights, whose arguments are <= 0.
MQ_DEV float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------- RMSNorm
// xn = x * rsqrt(mean(x^2) + eps) * w over the 1024 values in LDS `x`, two per thread.
// fused_decode_ldg_common.inl:150-191 (input norm), fused_decode_ldg_mlp.inl:70-118 (post norm),
// fused_decode_ldg_kernel.inl:103-137 (final norm).
// With `round_out` the result is rounded to bf16 (the prefill path's final norm,
// prefill_final_norm_kernel, fused_prefill_kernels.inl:655-700).
// All threads of the workgroup call it; the caller syncs before anything reads xn, and that
// barrier also keeps the next norm from overwriting `red` while it is still being read.
MQ_DEV void norm_1024(const float* x, const bf16_t* __restrict__ w, float* xn, float* red,
                      bool round_out = false) {
  const int t = tid();
  // the weights are loaded before the reduction: a load after block_sum's barriers cannot be
  // hoisted above them and put its latency on every norm's critical path (572 against 576 us per
  // token at pos 128)
  const uint32_t wv = ld32(w + 2 * t);
  const float2 v = reinterpret_cast<const float2*>(x)[t];
  // workgroup sum of squares with one barrier (block_sum's second one only protects `red` from
  // the next reduction, and every caller syncs right after the norm; 570 against 571.4 us per
  // token at pos 128); the same order of additions as block_sum
  float ss = 0.f;
  {
    const float ws = wave_sum(v.x * v.x + v.y * v.y);
    if (lane_id() == 0) red[wave_id()] = ws;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MQ_WAVES; ++i) ss += red[i];
  }
  const float r = rsqrtf(ss * (1.0f / MQ_H) + MQ_EPS);
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
// [0, 256): LDS_ATTH, the attention output of a single-chunk (local) item
#define ALDS_QS 512       // [256] rotated q of the two query heads (sync wave input)
#define ALDS_KN 768       // [128] new-position k-hat (bf16 values)
#define ALDS_VN 896       // [128] new-position v (bf16 values)
#define ALDS_WML 1536     // [MQ_CWAVES][4] per-wave m0, m1, l0, l1
#define ALDS_STAT 1568    // m[2], l[2] of the item
#define ALDS_SNEW 1576    // [2] scores (log2 domain) of the new position for both query heads
#define ALDS_ORED 1584    // [MQ_CWAVES][256] per-wave unnormalised outputs; the item's in [0, 256)
#define ALDS_WSC (ALDS_ORED + MQ_CWAVES * 256)   // [MQ_CWAVES][32][2] each wave's weights
// The merge of several chunks runs after this item's partial has been published, so it reuses
// the per-wave areas.
#define ALDS_MW 1024                             // merge: (m, l)[2][64] then weights [2][64]
#define ALDS_MSUM (ALDS_MW + 512)                // merge: [4][2][128] partial sums
static_assert(ALDS_WSC + MQ_CWAVES * 64 <= MQ_LDS_FLOATS, "attention LDS carve");
static_assert(ALDS_MSUM + 1024 <= MQ_LDS_FLOATS, "attention merge LDS carve");
static_assert(ALDS_MSUM + 1024 <= ALDS_ORED + MQ_CWAVES * 256, "merge stays in the phase carve");

// q/k RMSNorm of one head held by one wave as two consecutive dims per lane (lane l: dims 2l,
// 2l + 1), then rotate-half RoPE with the bf16 table row (fused_decode_ldg_common.inl:268-394):
//   o_i = x_i c_i - x_{i+64} s_i,  o_{i+64} = x_i s_{i+64} + x_{i+64} c_{i+64}.
// The RoPE partner of lane l's dims is lane l ^ 32 (dims +- 64), one v_permlane32_swap away.
// w, c, s: this lane's two norm weights, cos and sin values.
MQ_DEV float2 head_norm_rope2(float2 x, float2 w, float2 c, float2 s) {
  const float ss = wave_sum(x.x * x.x + x.y * x.y);
  const float r = rsqrtf(ss * (1.0f / MQ_D) + MQ_EPS);
  const float a0 = x.x * r * w.x, a1 = x.y * r * w.y;
  const float2 p0 = swap32(a0), p1 = swap32(a1);     // (lanes 0-31 | 32-63), both orders
  const bool low = lane_id() < 32;                    // dims < 64
  const float b0 = low ? p0.y : p0.x, b1 = low ? p1.y : p1.x;   // partner lane's values
  return low ? make_float2(a0 * c.x - b0 * s.x, a1 * c.y - b1 * s.y)
             : make_float2(b0 * s.x + a0 * c.x, b1 * s.y + a1 * c.y);
}

MQ_DEV float* part_ptr(float* part, int h, int c, int j) {
  return part + ((size_t)(h * MQ_MAX_CHUNKS + c) * MQ_GQA + j) * MQ_PART_STRIDE;
}

// q-hat of both query heads as the A operand of v_mfma_f32_16x16x32_bf16 in LDS_QA: A rows
// 4 hh + t (hh = query head, t = 0, 1, 2) hold the bf16 parts q = hi + mid + lo (residuals exact
// in fp32, so the three products with a bf16 key sum to the fp32 q . k up to ~2^-26 relative);
// rows 3 and 7..15 stay zero.  Lane l of the calling wave holds dims 2l, 2l + 1 of each head.
// Element (row r, dim d) of k-step s = d / 32 sits at lane r + 16 ((d % 32) / 8), entry d % 8.
MQ_DEV void q_operand_store(float2 q0, float2 q1, float* lds) {
  bf16_t* qa = reinterpret_cast<bf16_t*>(lds + LDS_QA);
  const int lane = lane_id();
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int dd = 2 * lane + e;
      const float x = hh == 0 ? (e == 0 ? q0.x : q0.y) : (e == 0 ? q1.x : q1.y);
      const bf16_t hi = f32_to_bf16(x);
      const float r1 = x - bf16_to_f32(hi);
      const bf16_t mid = f32_to_bf16(r1);
      const bf16_t lo = f32_to_bf16(r1 - bf16_to_f32(mid));
      const int s = dd >> 5, col = 16 * ((dd & 31) >> 3), el = dd & 7;
      bf16_t* base = qa + (size_t)(s * 64 + col) * 8 + el;
      base[(4 * hh + 0) * 8] = hi;
      base[(4 * hh + 1) * 8] = mid;
      base[(4 * hh + 2) * 8] = lo;
    }
  }
}
// All threads: zero LDS_QA (the rows q_operand_store never writes stay zero afterwards).
MQ_DEV void q_operand_clear(float* lds) {
  for (int i = tid(); i < 4 * 64 * 4; i += MQ_THREADS) lds[LDS_QA + i] = 0.f;
}

// Sync-wave prologue of an attention item on the raw q of query heads 2h, 2h+1 and the k and v
// of kv head h (v[0..3], dims 2 lane, 2 lane + 1 each) and the read-only parameters (q_norm and
// k_norm weight pairs wq / wk, RoPE row pairs c2 / s2, as bf16x2): per-head RMSNorm + RoPE in
// registers.  Leaves q-hat of both query heads in LDS_QA (MFMA operand) and ALDS_QS (fp32), the
// new position's k-hat and v rounded to bf16 (kept as fp32) in ALDS_KN / ALDS_VN, and the new
// position's two scores (q-hat . bf16 k-hat, log2 domain) in ALDS_SNEW; the compute waves read
// them after the phase's closing __syncthreads.  The cache row itself is written later by the
// sync wave (attn_cache_row), so no compute wave ever waits for a store.
MQ_DEV void attn_prologue(const float2* v, uint32_t wq, uint32_t wk, uint32_t c2, uint32_t s2,
                          float scale_log2, float* lds) {
  const int lane = lane_id();
  const float2 c = make_float2(bf16_lo(c2), bf16_hi(c2));
  const float2 s = make_float2(bf16_lo(s2), bf16_hi(s2));
  const float2 wqf = make_float2(bf16_lo(wq), bf16_hi(wq));
  const float2 q0 = head_norm_rope2(v[0], wqf, c, s);
  const float2 q1 = head_norm_rope2(v[1], wqf, c, s);
  const float2 k = head_norm_rope2(v[2], make_float2(bf16_lo(wk), bf16_hi(wk)), c, s);
  const float2 kb = make_float2(round_bf16(k.x), round_bf16(k.y));
  const float sn0 = wave_sum(q0.x * kb.x + q0.y * kb.y) * scale_log2;
  const float sn1 = wave_sum(q1.x * kb.x + q1.y * kb.y) * scale_log2;
  reinterpret_cast<float2*>(lds + ALDS_QS)[lane] = q0;
  reinterpret_cast<float2*>(lds + ALDS_QS + MQ_D)[lane] = q1;
  reinterpret_cast<float2*>(lds + ALDS_KN)[lane] = kb;
  reinterpret_cast<float2*>(lds + ALDS_VN)[lane] =
      make_float2(round_bf16(v[3].x), round_bf16(v[3].y));
  if (lane == 0) reinterpret_cast<float2*>(lds + ALDS_SNEW)[0] = make_float2(sn0, sn1);
  q_operand_store(q0, q1, lds);
}
// Sync-wave input of an attention item of the decode kernels: group h's q|k|v words of the layer
// (xq, epoch e; the parameters are loaded before the poll, in the same round trip), then the
// prologue.
MQ_DEV void attn_input(const uint64_t* xq, uint32_t e, MqSync* sy, const bf16_t* qn,
                       const bf16_t* kn, const bf16_t* cs, const bf16_t* sn, float scale_log2,
                       float* lds) {
  const int lane = lane_id();
  const uint32_t wq = ld32(qn + 2 * lane), wk = ld32(kn + 2 * lane);
  const uint32_t c2 = ld32(cs + 2 * lane), s2 = ld32(sn + 2 * lane);
  float r[8];
  // word i of this lane: vector i / 2 (q0, q1, k, v of the group's 512 rows), dim 2 lane + i % 2
  x_poll<8>(xq, [&](int i) { return (i >> 1) * MQ_D + 2 * lane + (i & 1); }, e, sy,
            [&](int i, float v) { r[i] = v; });
  float2 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = make_float2(r[2 * i], r[2 * i + 1]);
  attn_prologue(v, wq, wk, c2, s2, scale_log2, lds);
}
// The same from the op-level fp32 q|k|v vector (rows in the fused q|k|v order).
MQ_DEV void attn_input_f(const float* qkv, const bf16_t* qn, const bf16_t* kn, const bf16_t* cs,
                         const bf16_t* sn, int h, float scale_log2, float* lds) {
  const int lane = lane_id();
  float2 v[4];
  v[0] = ld_coh2(qkv + 2 * h * MQ_D + 2 * lane);
  v[1] = ld_coh2(qkv + 2 * h * MQ_D + 128 + 2 * lane);
  v[2] = ld_coh2(qkv + MQ_QDIM + h * MQ_D + 2 * lane);
  v[3] = ld_coh2(qkv + MQ_QDIM + MQ_KVDIM + h * MQ_D + 2 * lane);
  const uint32_t wq = ld32(qn + 2 * lane), wk = ld32(kn + 2 * lane);
  const uint32_t c2 = ld32(cs + 2 * lane), s2 = ld32(sn + 2 * lane);
  attn_prologue(v, wq, wk, c2, s2, scale_log2, lds);
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

// A block of up to MQ_ATT_BLOCK (224) cache positions of an attention item: position
// blk + w + 7 i is the i-th position (i < 32) of compute wave w.
//   K, in the B-operand order of v_mfma_f32_16x16x32_bf16 (lane l: column l % 16, k-dims
//   8 (l / 16) .. + 8 of a 32-dim step): k[g][s] holds dims 32 s + 8 (lane / 16) .. + 8 of the
//   wave's position 16 g + lane % 16;
//   V: v[i] holds dims 2 lane, 2 lane + 1 of the wave's position i (one 256-byte row per wave
//   load).
// The row of the position being decoded (pos_new) is never loaded: it is written during this
// step (attn_cache_row) and enters the softmax from LDS instead (ALDS_SNEW / ALDS_VN).  Fetching
// it before the write would leave a stale copy in this CU's L1 and this XCD's L2, and a chained
// launch reads the row with plain loads in the next step.  Every row below pos_new was written
// either by an earlier kernel (complete at the kernel boundary) or by an earlier step of this
// launch, and was not loaded by anyone before that write, so a plain load of it cannot hit a
// stale line.  Within a launch, what completes the row before any later step loads it:
//   1. the sync wave stores the row with device-scope (sc1) stores in a phase_step epilogue
//      (attn_cache_row: with the O partials in local mode, with the attention partial in split
//      mode) and, in the same phase_step, waits for all its memory operations
//      (wait_all_memory, s_waitcnt vmcnt(0), which counts stores) before the closing
//      __syncthreads;
//   2. so the store has completed before wave 0 of that workgroup, after that barrier, adds its
//      arrival to the LM head's completion count (lm_head_run);
//   3. the last arriver publishes the step-done epoch only after observing every arrival, and
//      every workgroup issues the next step's K/V loads only after step_wait has seen that epoch.
// No barrier between workgroups is involved: the exchanges within a step carry epoch- or
// tag-stamped words and order nothing else.
#define MQ_ATT_PER_WAVE (MQ_ATT_BLOCK / MQ_CWAVES)
static_assert(MQ_ATT_PER_WAVE == 32, "two 16-position MFMA column groups per compute wave");
struct KvBlock {
  uint4 k[2][4];
  uint32_t v[MQ_ATT_PER_WAVE];
};
MQ_DEV const bf16_t* kv_base(const bf16_t* cache, const MqDecodeParams& p, int layer, int h) {
  return cache + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D;
}
MQ_DEV int att_pos(int blk, int wave, int i) { return blk + wave + MQ_CWAVES * i; }
// Positions [blk, bend) of the wave that exist: i < n_i (wave-uniform).
MQ_DEV int att_count(int blk, int bend, int wave) {
  return __builtin_amdgcn_readfirstlane(
      min(MQ_ATT_PER_WAVE, max(0, (bend - blk - wave + MQ_CWAVES - 1) / MQ_CWAVES)));
}
// K rows of a block.  FIXED issues every load (positions past bend or equal to pos_new read the
// read-only 256-byte row `dummy` instead), so the compiler knows how many loads follow earlier
// ones; otherwise groups past bend are skipped and their registers zeroed.
template <bool FIXED>
MQ_DEV void kv_load_k(KvBlock& b, const bf16_t* Kb, int blk, int bend, int pos_new,
                      const bf16_t* dummy) {
  const int lane = lane_id(), wave = wave_id();
  if (wave >= MQ_CWAVES) return;
  const int n = att_count(blk, bend, wave);
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    if (!FIXED && 16 * g >= n) {
#pragma unroll
      for (int s = 0; s < 4; ++s) b.k[g][s] = make_uint4(0, 0, 0, 0);
      continue;
    }
    const int pp = att_pos(blk, wave, 16 * g + (lane & 15));
    const bf16_t* row = (pp < bend && pp != pos_new ? Kb + (size_t)pp * MQ_D : dummy) +
                        8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < 4; ++s) b.k[g][s] = ld16(row + 32 * s);
  }
}
template <bool FIXED>
MQ_DEV void kv_load_v(KvBlock& b, const bf16_t* Vb, int blk, int bend, int pos_new,
                      const bf16_t* dummy) {
  const int lane = lane_id(), wave = wave_id();
  if (wave >= MQ_CWAVES) return;
  const int n = att_count(blk, bend, wave);
#pragma unroll
  for (int i = 0; i < MQ_ATT_PER_WAVE; ++i) {
    if (!FIXED && i >= n) {
      b.v[i] = 0;
      continue;
    }
    const int pp = att_pos(blk, wave, i);
    b.v[i] = ld32((pp < bend && pp != pos_new ? Vb + (size_t)pp * MQ_D : dummy) + 2 * lane);
  }
}
template <bool FIXED>
MQ_DEV void kv_block_load(KvBlock& b, const bf16_t* Kb, const bf16_t* Vb, int blk, int bend,
                          int pos_new, const bf16_t* dummy) {
  kv_load_k<FIXED>(b, Kb, blk, bend, pos_new, dummy);
  kv_load_v<FIXED>(b, Vb, blk, bend, pos_new, dummy);
}

typedef __bf16 mq_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float mq_f32x4_t __attribute__((ext_vector_type(4)));
MQ_DEV mq_bf16x8_t bf16x8_of(uint4 v) { return __builtin_bit_cast(mq_bf16x8_t, v); }

// Attention output of a single chunk covering every position: o / l as the log-sum-exp merge
// computes it for one partial (weight exp2(m - m) / l = 1 / l, then one fused multiply), so the
// persistent kernel's local result and the one-kernel-per-phase merge of the published partial
// are bitwise equal.
MQ_DEV float att_single(float o, float l) { return fmaf(1.0f / l, o, 0.f); }

// Core of one attention item (reference: fused_decode_ldg_common.inl:417-602): query heads 2h,
// 2h + 1 over cache positions [p0, p1) of kv head h, first block already in `b`, q-hat in LDS_QA;
// with `has_new` the item also holds the position being decoded, whose score and bf16 v come
// from ALDS_SNEW / ALDS_VN (its cache row is never read).  Per compute wave and block:
//   scores on MFMA: S^T[q-part][position] = A (three bf16 parts per query head) x K^T, summed
//   over the parts: lanes 0-15 hold head 0's scores of the 16 positions of a column group,
//   lanes 16-31 head 1's;
//   online softmax per wave (DPP row max / sum over the 16 lanes of a head), weights through
//   the wave's LDS slice;
//   p . V on VALU: lane l accumulates dims 2l, 2l + 1 of both heads over the wave's positions,
//   so no cross-lane reduction is needed.
// Then one log-sum-exp merge over the waves (and the new position) by 256 threads, leaving
// m[2], l[2] in ALDS_STAT and the unnormalised o[2][128] in ALDS_ORED[0..255], or with `to_att`
// (an item over every position) the attention output o / l in LDS_ATTH.
MQ_DEV void attn_core(const MqDecodeParams& p, int layer, int h, int p0, int p1, int pos_new,
                      bool has_new, KvBlock& b, float* lds, bool to_att = false) {
  float* wml = lds + ALDS_WML;
  float* stat = lds + ALDS_STAT;
  float* ored = lds + ALDS_ORED;
  const int lane = lane_id(), wave = wave_id();
  if (wave < MQ_CWAVES) {
    const bf16_t* Kb = kv_base(p.kc, p, layer, h);
    const bf16_t* Vb = kv_base(p.vc, p, layer, h);
    const bf16_t* dummy = p.cos;
    const uint4* qa = reinterpret_cast<const uint4*>(lds + LDS_QA);
    mq_bf16x8_t a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = bf16x8_of(qa[s * 64 + lane]);
    float* pw = lds + ALDS_WSC + wave * 64;      // this wave's weights [i][head]
    const bool lead = lane < 32;                 // lanes holding scores (head lane / 16)
    float m = -INFINITY, lsum = 0.f;             // per head (lanes 0-15 / 16-31)
    float acc00 = 0.f, acc01 = 0.f, acc10 = 0.f, acc11 = 0.f;   // [head][dim 2 lane + e]
    for (int blk = p0; blk < p1; blk += MQ_ATT_BLOCK) {
      // keeps the next block's loads from being hoisted into this one
      asm volatile("" ::: "memory");
      const int bend = min(p1, blk + MQ_ATT_BLOCK);
      if (blk != p0) kv_block_load<false>(b, Kb, Vb, blk, bend, pos_new, dummy);
      const int n = att_count(blk, bend, wave);
      float sc[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        sc[g] = -INFINITY;
        if (16 * g < n) {
          mq_f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s)
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], bf16x8_of(b.k[g][s]), c, 0, 0, 0);
          const float sv = ((c[0] + c[1]) + c[2]) * p.scale_log2;
          const int pp = att_pos(blk, wave, 16 * g + (lane & 15));
          sc[g] = lead && pp < bend && pp != pos_new ? sv : -INFINITY;
        }
      }
      const float n_m = fmaxf(m, row16_max(fmaxf(sc[0], sc[1])));
      const bool empty = n_m == -INFINITY;      // no position of this head so far
      const float al = empty ? 1.f : exp2_fast(m - n_m);
      const float w0 = empty ? 0.f : exp2_fast(sc[0] - n_m);
      const float w1 = empty ? 0.f : exp2_fast(sc[1] - n_m);
      lsum = fmaf(lsum, al, row16_sum(w0 + w1));
      m = n_m;
      if (lead) {
        pw[(lane & 15) * 2 + (lane >> 4)] = w0;
        pw[(16 + (lane & 15)) * 2 + (lane >> 4)] = w1;
      }
      // rescale by each head's factor (lane 0: head 0, lane 16: head 1)
      const float al0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al), 0));
      const float al1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al), 16));
      acc00 *= al0;
      acc01 *= al0;
      acc10 *= al1;
      acc11 *= al1;
      // in runs of 8 positions (a data-dependent exit inside the unrolled loop kept the block out
      // of registers); weights past n are 0
#pragma unroll
      for (int q8 = 0; q8 < MQ_ATT_PER_WAVE / 8; ++q8) {
        if (8 * q8 < n) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = 8 * q8 + e;
            const float2 w = reinterpret_cast<const float2*>(pw)[i];
            const float v0 = bf16_lo(b.v[i]), v1 = bf16_hi(b.v[i]);
            acc00 = fmaf(w.x, v0, acc00);
            acc01 = fmaf(w.x, v1, acc01);
            acc10 = fmaf(w.y, v0, acc10);
            acc11 = fmaf(w.y, v1, acc11);
          }
        }
      }
    }
    float* arow = lds + LDS_AROW + wave * 256;
    reinterpret_cast<float2*>(arow)[lane] = make_float2(acc00, acc01);
    reinterpret_cast<float2*>(arow + MQ_D)[lane] = make_float2(acc10, acc11);
    if ((lane & 15) == 0 && lead) {
      wml[wave * 4 + (lane >> 4)] = m;
      wml[wave * 4 + 2 + (lane >> 4)] = lsum;
    }
  }
  __syncthreads();
  // merge the compute waves (waves without a position have m = -inf and weigh 0) and the new
  // position; every item has at least one position, so M is finite.  All LDS reads first.
  if (tid() < 256) {
    const int j = tid() >> 7, d = tid() & 127;
    float mw[MQ_CWAVES], ow[MQ_CWAVES], lw[MQ_CWAVES];
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) {
      mw[w8] = wml[w8 * 4 + j];
      ow[w8] = lds[LDS_AROW + w8 * 256 + tid()];
      lw[w8] = wml[w8 * 4 + 2 + j];
    }
    const float sn = lds[ALDS_SNEW + j], vn = lds[ALDS_VN + d];
    float M = has_new ? sn : -INFINITY;
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) M = fmaxf(M, mw[w8]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) {
      const bool use = mw[w8] != -INFINITY;
      const float f = use ? exp2_fast(mw[w8] - M) : 0.f;
      o = use ? fmaf(f, ow[w8], o) : o;
      L = use ? fmaf(f, lw[w8], L) : L;
    }
    if (has_new) {
      const float f = exp2_fast(sn - M);
      o = fmaf(f, vn, o);
      L += f;
    }
    if (to_att) {
      // a single chunk over every position: the attention output itself (att_single, as the
      // one-kernel-per-phase merge computes it from this chunk's published partial)
      lds[LDS_ATTH + tid()] = att_single(o, L);
    } else {
      ored[tid()] = o;
      if (d == 0) {
        stat[j] = M;
        stat[2 + j] = L;
      }
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
// TAGGED: the partials are tagged words (tag_bits); with tag >= 1 every thread polls its words
// until they carry it, with tag < 0 they are read as they are; either way the tags are removed.
// NI: chunk words per thread (nch <= 4 NI); the group merges use 8, which keeps the persistent
// kernel's prefetched weights and the polled words within its registers.
template <bool TAGGED = false, int NI = 16, class Out>
MQ_DEV void attn_merge(const float* part, int h, int nch, float* lds, Out out, int tag = -1,
                       MqSync* sy = nullptr) {
  float* mw = lds + ALDS_MW;      // (m, l) pairs [2][64] -> weights [2][64] at +256
  float* msum = lds + ALDS_MSUM;  // [4][2][128]
  const int t = tid();
  const int j = t >> 8, pr = (t >> 2) & 63, q = t & 3;
  float* pbase = const_cast<float*>(part);
  float2 ml = make_float2(0.f, 0.f);
  const int mj = t >= nch ? 1 : 0, mc = t - mj * nch;   // (query head, chunk) of t < 2 nch
  float2 o2[NI];
  if constexpr (TAGGED) {
    auto mlw = [&] { return reinterpret_cast<const uint64_t*>(part_ptr(pbase, h, mc, mj)); };
    auto ow = [&](int i) {
      return reinterpret_cast<const uint64_t*>(part_ptr(pbase, h, q + 4 * i, j) + 4 + 2 * pr);
    };
    uint64_t wml = t < 2 * nch ? ld_coh64(mlw()) : 0ull;
    uint64_t wo[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) wo[i] = q + 4 * i < nch ? ld_coh64(ow(i)) : 0ull;
    if (tag >= 0) {
      const uint32_t tg = (uint32_t)tag;
      uint32_t spins = 0;
      while (true) {
        bool ok = t >= 2 * nch || tag_ok2(wml, tg);
#pragma unroll
        for (int i = 0; i < NI; ++i) ok = ok && (q + 4 * i >= nch || tag_ok2(wo[i], tg));
        if (__all(ok)) break;
        uint32_t ev = 0;
        if (lane_id() == 0 && (spins & 15) == 15)
          ev = __hip_atomic_load(&sy->err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readlane(ev, 0) != 0) break;
        if (++spins > MQ_SPIN_LIMIT) {
          if (lane_id() == 0)
            __hip_atomic_store(&sy->err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        if (t < 2 * nch && !tag_ok2(wml, tg)) wml = ld_coh64(mlw());
#pragma unroll
        for (int i = 0; i < NI; ++i)
          if (q + 4 * i < nch && !tag_ok2(wo[i], tg)) wo[i] = ld_coh64(ow(i));
      }
    }
    ml = make_float2(untag((uint32_t)wml), untag((uint32_t)(wml >> 32)));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      o2[i] = make_float2(untag((uint32_t)wo[i]), untag((uint32_t)(wo[i] >> 32)));
  } else {
    if (t < 2 * nch) ml = ld_coh2(part_ptr(pbase, h, mc, mj));
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int c = q + 4 * i;
      o2[i] = c < nch ? ld_coh2(part_ptr(pbase, h, c, j) + 4 + 2 * pr) : make_float2(0.f, 0.f);
    }
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
  for (int i = 0; i < NI; ++i) {
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
MQ_DEV void gu_load(GateUpSet& ws, const MqLayerW& w, int wg, int G,
                    bool paced = false, bool fixed = false) {
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  ws.load([&](int i) {
    return i < nr ? w.wg + (size_t)(r0 + i) * MQ_H : w.wu + (size_t)(r0 + i - nr) * MQ_H;
  }, 2 * nr, paced, fixed);
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
// (fused_decode_ldg_mlp.inl:120-175, fused_decode_ldg_common.inl:123-125), published to every
// group's copy of m [MQ_GROUPS][MQ_I] as tagged words of epoch e (tag_bits).
MQ_DEV void gu_publish(float* m, int wg, int G, const float* lds, uint32_t e) {
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) {
    const float gv = lds[LDS_PR + t], uv = lds[LDS_PR + nr + t];
    const float v = gv / (1.0f + expf(-gv)) * uv;
#pragma unroll
    for (int c = 0; c < MQ_GROUPS; ++c) st_tag(m + (size_t)c * MQ_I + r0 + t, v, e);
  }
}
// The op-level form (fp32 array, plain coherent stores).
MQ_DEV void gu_publish_f(float* m, int wg, int G, const float* lds) {
  int r0, nr;
  row_range(MQ_I, wg, G, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) {
    const float gv = lds[LDS_PR + t], uv = lds[LDS_PR + nr + t];
    st_coh(m + r0 + t, gv / (1.0f + expf(-gv)) * uv);
  }
}

// ----------------------------------------------------------------------------- P5: down
// Hidden rows of workgroup wg for the down projection and the layer output: whole row pairs, so
// that a pair of bf16 outputs is one exchange word (hidden_publish).
MQ_DEV void hid_rows(int wg, int G, int& r0, int& nr) {
  int p0, np;
  row_range(MQ_H / 2, wg, G, p0, np);
  r0 = 2 * p0;
  nr = 2 * np;
}
MQ_DEV void down_load(DownSet& ws, const MqLayerW& w, int wg, int G,
                      bool paced = false) {
  int r0, nr;
  hid_rows(wg, G, r0, nr);
  ws.load([&](int i) { return w.wd + (size_t)(r0 + i) * MQ_I; }, nr, paced);
}
// Input: m in LDS_IN; segment dot products -> LDS_PR.
MQ_DEV void down_run(const DownSet& ws, const MqLayerW& w, int wg, int G, float* lds) {
  int r0, nr;
  hid_rows(wg, G, r0, nr);
  ws.compute([&](int i) { return w.wd + (size_t)(r0 + i) * MQ_I; }, nr, lds + LDS_IN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: lane t < nr holds a[r0 + t] in `res` and leaves the bf16-rounded layer
// output of that row in it (fused_decode_ldg_mlp.inl:177-217); out(r, v) publishes it.
template <class Out>
MQ_DEV void down_publish(int wg, int G, const float* lds, float& res, Out out) {
  int r0, nr;
  hid_rows(wg, G, r0, nr);
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
                        bool publish_epoch = false, uint32_t step_epoch = 0,
                        bool set_xep = false, uint32_t xep_next = 0, bool reset_place = false) {
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
  if (wave == 0) {
    MqSync* sy = &p.st->sync;
    uint32_t old = 0;
    if (lane == 0) {
      uint64_t k = keys[0];
#pragma unroll
      for (int i = 1; i < MQ_WAVES; ++i) k = u64_max(k, keys[i]);
      __hip_atomic_fetch_max(&sy->argmax.v, (unsigned long long)k, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      wait_all_memory();
      old = __hip_atomic_fetch_add(&sy->done.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__builtin_amdgcn_readlane(old, 0) == (uint32_t)G - 1) {
      // the last workgroup: token, then the step's sync state cleared
      if (lane == 0) {
        const unsigned long long kk =
            __hip_atomic_load(&sy->argmax.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // device-scope store: the next step of a multi-step launch reads it in other workgroups
        __hip_atomic_store(reinterpret_cast<uint32_t*>(tok_out), argmax_key_index(kk),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&sy->argmax.v, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (advance_pos)
          __hip_atomic_store(&p.st->pos.v, (uint32_t)(pos + 1), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        if (set_xep)   // the next base, already reduced (mq_xep_advance; 0 is a valid base)
          __hip_atomic_store(&p.st->xep.v, xep_next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (reset_place)   // a launch's last step: every workgroup claimed its role at its start
          for (int i = 0; i < MQ_GROUPS; ++i)
            __hip_atomic_store(&p.st->place[i].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&sy->done.v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (publish_epoch) {
        // every reset above and the token are complete before the epoch releases the next step
        wait_all_memory();
        if (lane == 0)
          __hip_atomic_store(&p.st->steps.v, step_epoch, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
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
//   1. q|k|v: group h computes the 512 rows of its kv head (q heads 2h, 2h+1, k and v of h),
//      published as (value, epoch) words read by the group.
//   2. attention split over the group's workgroups by position chunks, partials (m, l, o)
//      published per chunk as tagged words (an empty partial from a workgroup without a chunk).
//   3. every workgroup of the group polls and merges the partials (att of its two query heads)
//      and computes its rows of the O projection restricted to the head's 256 columns,
//      published as tagged words to every group's copy.
//   4. a = x + sum_h opart_h (every thread polls its rows), RMSNorm, gate|up rows; silu(g) * u
//      published as tagged words.
//   5. down rows + a -> bf16 layer output, published as (bf16 pair, epoch) words -> next layer.
// That is 5 exchanges (4 for short contexts) and no barrier per layer.  For short contexts
// (cache length <= attn_local_max) steps 2-3 collapse: every workgroup of the group attends over
// all positions itself (its O rows prefetched with the K/V rows), and the partial exchange goes
// away.
// Measured per layer (MFMA scores, epoch-word exchanges): at 128 positions local mode takes
// 18.7 us against 19.2 us split; at 200 positions 19.7 against 19.6, so the default switches
// to split chunks above 176 positions.

// Local row i of group h's 512 q|k|v rows -> row of the fused q|k|v projection.
MQ_DEV int grp_row(int h, int i) {
  if (i < 2 * MQ_D) return 2 * h * MQ_D + i;
  if (i < 3 * MQ_D) return MQ_QDIM + h * MQ_D + (i - 2 * MQ_D);
  return MQ_QDIM + MQ_KVDIM + h * MQ_D + (i - 3 * MQ_D);
}
MQ_DEV void gqkv_load(QkvSet& ws, const MqLayerW& w, int h, int j, int NG,
                      bool paced = false) {
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  ws.load([&](int i) { return qkv_row(w, grp_row(h, r0 + i)); }, nr, paced);
}
MQ_DEV void gqkv_run(const QkvSet& ws, const MqLayerW& w, int h, int j, int NG, float* lds) {
  norm_1024(lds + LDS_IN, w.in_ln, lds + LDS_XN, lds + LDS_RED);
  __syncthreads();
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  ws.compute([&](int i) { return qkv_row(w, grp_row(h, r0 + i)); }, nr, lds + LDS_XN,
             [&](int it, float v) { lds[LDS_PR + it] = v; });
}
// Sync-wave epilogue: this workgroup's rows of group h's q|k|v as (value, epoch e) words into
// xq [4 * MQ_D] (the group's local row order, grp_row).  `local`: every reader is on this XCD
// (the persistent kernel places a group on one XCD), so plain stores into its L2 suffice.
MQ_DEV void gqkv_publish(uint64_t* xq, uint32_t e, int j, int NG, const float* lds,
                         bool local = false) {
  int r0, nr;
  row_range(4 * MQ_D, j, NG, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) {
    const uint64_t w = xword(lds[LDS_PR + t], e);
    if (local) st_local64(xq + r0 + t, w);
    else st_coh64(xq + r0 + t, w);
  }
}

// Position chunks of a group: as many chunks of at least mq_attn_min_chunk positions as the group
// has workgroups; chunk j = [p0, p1).  All chunks c < nch are non-empty.
// Local mode (cache_len <= local_max): one chunk over all positions.  With `all_local` (the
// persistent kernel) every workgroup of the group computes it, so the attention output needs no
// exchange; otherwise (one kernel per phase) workgroup 0 of the group computes it and publishes
// it as the only partial.  Either way the K/V cache row is written by workgroup 0 (has_pos).
struct GAttn {
  int nch, p0, p1;
  bool active, has_pos, has_new, local;   // has_pos: writes the new K/V row; has_new: the
                                          // chunk holds the new position
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
    g.has_new = g.active;
    return g;
  }
  const int mc = mq_attn_min_chunk(cache_len);
  const int want = (cache_len + mc - 1) / mc;
  const int n0 = min(min(NG, MQ_GROUP_CHUNKS), want);
  const int clen = (cache_len + n0 - 1) / n0;
  g.nch = (cache_len + clen - 1) / clen;
  g.p0 = j * clen;
  g.p1 = min(cache_len, g.p0 + clen);
  g.active = j < g.nch;
  g.has_pos = g.active && pos >= g.p0 && pos < g.p1;
  g.has_new = g.has_pos;
  return g;
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
// Sync wave, one kernel per phase, local mode: workgroup 0's single partial (plain values, read
// by group_single in the next kernel) and the new position's K/V cache row.
MQ_DEV void gattn_publish_local(const MqDecodeParams& p, int layer, int pos, int h,
                                const GAttn& g, const float* lds) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = lane + 64 * i, jj = t >> 7, d = t & 127;
    st_coh(part_ptr(p.s->part, h, 0, jj) + 4 + d, lds[ALDS_ORED + t]);
  }
  if (lane < 2) {
    st_coh(part_ptr(p.s->part, h, 0, lane), lds[ALDS_STAT + lane]);
    st_coh(part_ptr(p.s->part, h, 0, lane) + 1, lds[ALDS_STAT + 2 + lane]);
  }
  if (g.has_pos) attn_cache_row(p, layer, h, pos, lds);
}
// Sync wave, after attn_core: this member's partial (m, l, o) of both query heads as tagged words
// of epoch e into slot j of `part` (one layer-parity half of MqExchange.part), and the new
// position's K/V cache row from the chunk that holds it.  A member without a chunk writes an
// empty partial (m = -inf, l = 0, o = 0; never read), so that every slot is rewritten in every
// split-mode layer, as the tags require.
MQ_DEV void gattn_publish(const MqDecodeParams& p, int layer, int pos, int h, int j,
                          const GAttn& g, const float* lds, float* part, uint32_t e,
                          bool local = false) {
  const int lane = lane_id();
  auto put = [&](float* q, float v) {
    if (local) st_tag_local(q, v, e);
    else st_tag(q, v, e);
  };
  if (j < MQ_GROUP_CHUNKS) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = lane + 64 * i, jj = t >> 7, d = t & 127;
      put(part_ptr(part, h, j, jj) + 4 + d, g.active ? lds[ALDS_ORED + t] : 0.f);
    }
    if (lane < 2) {
      put(part_ptr(part, h, j, lane), g.active ? lds[ALDS_STAT + lane] : -INFINITY);
      put(part_ptr(part, h, j, lane) + 1, g.active ? lds[ALDS_STAT + 2 + lane] : 0.f);
    }
  }
  if (g.has_pos) attn_cache_row(p, layer, h, pos, lds);
}
// All threads: merged attention output of query heads 2h, 2h+1 into LDS_ATTH from tagged
// partials (tag >= 1: polled until they carry it; tag < 0: read as they are).
MQ_DEV void group_merge(const float* part, int h, int nch, float* lds, int tag, MqSync* sy) {
  attn_merge<true, MQ_GROUP_CHUNKS / 4>(part, h, nch, lds,
                   [&](int jj, int d, float o) { lds[LDS_ATTH + jj * MQ_D + d] = o; }, tag, sy);
  __syncthreads();
}

// GEMV over rows of 256 elements (the O projection restricted to one kv head's two query
// heads): one wave instruction covers a pair of rows, lanes 0-31 the first and 32-63 the second.
// `paced`: a wave sleeps MQ_PF_PAIR_PACE x 64 clocks between its items (one 1 KB load each), only
// where the loads overlap an exchange: at the split-mode partial exchange 562.0 against 566.7 us
// per token at pos 1024 and 619.2 against 627.7 at 4096; issued with local attention's K/V rows
// 521.5 against 518.4 at pos 128.
#define MQ_PF_PAIR_PACE 8
template <int PF>
struct PairSet {
  uint4 w[PF];
  template <class RowPtr>
  MQ_DEV void load(RowPtr rowptr, int nr, bool paced) {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int np = (nr + 1) / 2;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int it = wave + i * MQ_CWAVES, row = 2 * it + (lane >> 5);
      if (paced && i > 0) __builtin_amdgcn_s_sleep(MQ_PF_PAIR_PACE);
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
MQ_DEV void opart_load(OPairSet& ws, const MqLayerW& w, int h, int j, int NG,
                       bool paced = false) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  ws.load([&](int i) { return opart_row(w, h, r0 + i); }, nr, paced);
}
// Input: att of the group's query heads in LDS_ATTH; dot products -> LDS_PR.
MQ_DEV void opart_run(const OPairSet& ws, const MqLayerW& w, int h, int j, int NG, float* lds) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  ws.compute([&](int i) { return opart_row(w, h, r0 + i); }, nr, lds + LDS_ATTH,
             [&](int i, float v) { lds[LDS_PR + i] = v; });
}
// opart: one layer-parity half of MqExchange.opart, [MQ_GROUPS copies][MQ_NKV][MQ_H]; each
// value goes to every copy as a tagged word of epoch e (tag_bits).
MQ_DEV void opart_publish(float* opart, int h, int j, int NG, const float* lds, uint32_t e) {
  int r0, nr;
  row_range(MQ_H, j, NG, r0, nr);
  for (int t = lane_id(); t < nr; t += 64) {
    const float v = lds[LDS_PR + t];
#pragma unroll
    for (int c = 0; c < MQ_GROUPS; ++c) st_tag(opart + (c * MQ_NKV + h) * MQ_H + r0 + t, v, e);
  }
}
// a = x + sum_h opart_h, summed in head order (the single-row form for the multi-kernel mode).
MQ_DEV float a_elem(float x, const float* opart, int r) {
  float a = x;
#pragma unroll
  for (int h = 0; h < MQ_NKV; ++h)
    a += untag(__float_as_uint(ld_coh(opart + h * MQ_H + r)));
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
        a.x += untag(__float_as_uint(o[i][h].x));
        a.y += untag(__float_as_uint(o[i][h].y));
      }
      reinterpret_cast<float2*>(lds + LDS_IN)[q] = a;
      reinterpret_cast<float2*>(lds + LDS_A)[q] = a;
    }
  }
}
// All threads: a for all 1024 rows (thread t: rows 2t, 2t+1), same summation order as
// gu_input and a_elem; ends with __syncthreads.
MQ_DEV void gu_input_all(const float* opart, float* lds, int tag, MqSync* sy) {
  const int t = tid();
  static_assert(MQ_H / 2 == MQ_THREADS, "one row pair per thread");
  float2 o[MQ_NKV];
  tag_poll_all<MQ_NKV>(opart, [&](int h) { return (h * MQ_H) / 2 + t; }, tag, sy,
                       [&](int h, float lo, float hi) { o[h] = make_float2(lo, hi); });
  float2 a = reinterpret_cast<const float2*>(lds + LDS_HID)[t];
#pragma unroll
  for (int h = 0; h < MQ_NKV; ++h) {
    a.x += o[h].x;
    a.y += o[h].y;
  }
  reinterpret_cast<float2*>(lds + LDS_IN)[t] = a;
  reinterpret_cast<float2*>(lds + LDS_A)[t] = a;
  __syncthreads();
}
// All threads: the MLP vector (MQ_I tagged values) into LDS dst; ends with __syncthreads.
MQ_DEV void m_input_all(const float* m, float* dst, int tag, MqSync* sy) {
  const int t = tid();
  constexpr int P = MQ_I / 2 / MQ_THREADS;
  static_assert(P * 2 * MQ_THREADS == MQ_I, "whole pairs per thread");
  tag_poll_all<P>(m, [&](int i) { return t + MQ_THREADS * i; }, tag, sy,
                  [&](int i, float lo, float hi) {
                    reinterpret_cast<float2*>(dst)[t + MQ_THREADS * i] = make_float2(lo, hi);
                  });
  __syncthreads();
}
// Sync wave: a layer output (MQ_H / 2 pair words of `src`, epoch e) into LDS dst (and dst2).
MQ_DEV void hidden_gather(float* dst, float* dst2, const uint64_t* src, uint32_t e, MqSync* sy) {
  const int lane = lane_id();
  x_poll<MQ_H / 128>(src, [&](int i) { return lane + 64 * i; }, e, sy, [&](int i, float v) {
    const uint32_t u = __float_as_uint(v);
    const float2 f = make_float2(bf16_to_f32((bf16_t)(u & 0xffffu)), bf16_to_f32((bf16_t)(u >> 16)));
    reinterpret_cast<float2*>(dst)[lane + 64 * i] = f;
    if (dst2 != nullptr) reinterpret_cast<float2*>(dst2)[lane + 64 * i] = f;
  });
}
// All threads: the same, thread t polling pair word t (one per thread), then __syncthreads.  Every
// wave polls its own 64 words, so the exchange has 8 waves' loads in flight instead of the sync
// wave's 8 per lane.
MQ_DEV void hidden_input_all(float* dst, float* dst2, const uint64_t* src, uint32_t e,
                             MqSync* sy) {
  static_assert(MQ_H / 2 == MQ_THREADS, "one pair word per thread");
  const int t = tid();
  x_poll<1>(src, [&](int) { return t; }, e, sy, [&](int, float v) {
    const uint32_t u = __float_as_uint(v);
    const float2 f = make_float2(bf16_to_f32((bf16_t)(u & 0xffffu)), bf16_to_f32((bf16_t)(u >> 16)));
    reinterpret_cast<float2*>(dst)[t] = f;
    reinterpret_cast<float2*>(dst2)[t] = f;
  });
  __syncthreads();
}
MQ_DEV void input_hidden_bf16(float* lds, const bf16_t* src) {
  wave_copy_bf16_1024(lds + LDS_IN, src);
  wave_copy_bf16_1024(lds + LDS_HID, src);
}

// Phase boundary of the head-group kernel.  Order of the workgroup's memory operations: the
// sync wave's output stores, then the compute waves' weight prefetch, then the sync wave's input
// loads (polled where the input is an epoch-word exchange; the tagged exchanges are polled by
// every thread after this returns).  A workgroup's memory queue is first-in first-out in
// practice, so publishing before the prefetch is issued keeps the outputs from waiting behind
// tens of KB of weight loads, and the prefetch drains while the exchange completes.  The sync
// wave does not wait for its stores to be acknowledged: readers recognise the words by their
// epoch or tag, so no store needs to land before another.
template <class Epi, class Prefetch, class Input>
MQ_DEV void phase_step(Epi epilogue, Prefetch prefetch, Input input) {
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) epilogue();
  __syncthreads();
  if (wave_id() < MQ_CWAVES) prefetch();
  if (wave_id() == MQ_SYNC_WAVE) {
    input();
    wait_all_memory();
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------- kernels
// Reads and validates the step's position and input token.  The result is identical in every
// workgroup, so an invalid step makes all of them return before the first exchange.
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

// Sync wave, after down_publish: lane t < nr holds the bf16-valued layer output of row r0 + t
// (r0, nr even).  Each row pair goes as one exchange word (bf16 of row 2k in bits 0-15, of row
// 2k + 1 in bits 16-31, epoch e in bits 32-63) to every group's copy of the layer's buffer
// [MQ_H / 2 words]; the rows also go to the debug trace.
MQ_DEV void hidden_publish(const MqDecodeParams& p, int l, int r0, int nr, float res,
                           uint32_t e) {
  const int t = lane_id();
  const float other = __shfl_xor(res, 1);
  if (t < nr && (t & 1) == 0) {
    const uint64_t w = ((uint64_t)e << 32) | (uint64_t)((uint32_t)f32_to_bf16(other) << 16) |
                       (uint64_t)f32_to_bf16(res);
#pragma unroll
    for (int c = 0; c < MQ_GROUPS; ++c) st_coh64(&p.x->h[l & 1][c][(r0 + t) >> 1], w);
  }
  if (p.trace != nullptr && t < nr) p.trace[(size_t)l * MQ_H + r0 + t] = res;
}
// Row r of a layer-output buffer copy (any epoch).
MQ_DEV float hidden_row(const uint64_t* src, int r) {
  const uint32_t u = (uint32_t)ld_coh64(src + (r >> 1));
  return bf16_to_f32((bf16_t)((r & 1) ? (u >> 16) : (u & 0xffffu)));
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
      __builtin_amdgcn_s_sleep(2);   // back-off between polls
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
// they stream in during the q|k|v dot products and exchange; its V rows follow at the q|k|v
// exchange.  Both K/V loads have a fixed instruction count (kv_block_load_all), so the
// compiler waits for the q|k|v weights alone.  The variant is correct at any position: steps
// where a workgroup has no chunk load a stand-in K row and ignore it (and issue their gate|up
// weights at the q|k|v boundary, as in the other variant), and chunks of <= 8 positions use the
// 7-wave layout.  (One kernel holding both variants spilled ~600 VGPRs.)
template <bool EARLY>
__global__ void __launch_bounds__(MQ_THREADS) mq_decode_persistent_kernel(MqDecodeParams p) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  __shared__ MqLayerW s_layers[MQ_MAX_LAYERS];
  const int G = gridDim.x;
  {
    const int nw = p.num_layers * (int)(sizeof(MqLayerW) / 4);
    for (int i = tid(); i < nw; i += MQ_THREADS)
      reinterpret_cast<uint32_t*>(s_layers)[i] = reinterpret_cast<const uint32_t*>(p.layers)[i];
    q_operand_clear(lds);
    __syncthreads();
  }
  // Workgroup roles from the hardware placement: kv-head group h is the XCD the workgroup runs
  // on, member j the order in which it claimed a slot there, so the group-local exchanges (plain
  // stores into the XCD's L2, st_local64) are read only on their writer's XCD whatever the
  // dispatch order.  The workgroup's role index rw = h + 8 j takes the place of its launch index
  // in every row assignment (a bijection onto [0, G) when every XCD holds G / 8 workgroups, as
  // one 512-thread workgroup per CU on 8 XCDs of G / 8 CUs gives).  Any other placement claims a
  // member index >= G / 8 somewhere: that workgroup flags error 4 and returns, and the others'
  // waits end on the error flag.  The claims are reset by the launch's last step.
  __shared__ int s_role;
  if (tid() == 0) {
    const uint32_t xc = (uint32_t)xcc_id() & (MQ_GROUPS - 1);
    const uint32_t c = __hip_atomic_fetch_add(&p.st->place[xc].v, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    s_role = (int)(xc + MQ_GROUPS * c);
  }
  __syncthreads();
  const int NG = G / MQ_GROUPS;
  const int rw = __builtin_amdgcn_readfirstlane(s_role);
  const int h = rw % MQ_GROUPS, j = rw / MQ_GROUPS;
  if (j >= NG) {
    if (tid() == 0)
      __hip_atomic_store(&p.st->sync.err.v, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // All waves keep the default issue priority.  Raising the sync wave's (s_setprio 3) helped
  // while it alone polled counter barriers (576.7 against 579.5 us per token at pos 128); with
  // every thread polling tagged words it costs 0.5% at pos 4096 (647.5 against 643.7 us).
  MqSync* sy = &p.st->sync;
  MqExchange* x = p.x;
  const int copy = h;                     // the exchange copy this workgroup reads (its XCD's)
  int r0h, nrh;
  hid_rows(rw, G, r0h, nrh);
  // the step-done epoch and the exchange epoch base before this launch: read by every workgroup
  // before any can complete the first step (completion needs every workgroup's arrival at the
  // LM head, where the last one advances them)
  const uint32_t epoch0 = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&p.st->steps.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const uint32_t xep0 = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&p.st->xep.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  QkvSet wq;
  OPairSet wo;
  GateUpSet wgu;
  DownSet wd;
  KvBlock kv;
  if (p.num_layers > 0) gqkv_load(wq, lds_layer(s_layers, 0), h, j, NG, true);
  for (int step = 0; step < p.nsteps; ++step) {
    int pos, tok;
    if (!step_inputs(p, step == 0 ? p.tok_in : p.tok_out + (step - 1), pos, tok)) return;
    const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, true);
    const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
    const bf16_t* cs = p.cos + (size_t)pos * MQ_D;
    const bf16_t* sn = p.sin + (size_t)pos * MQ_D;
    phase_step(MQ_NOTHING, MQ_NOTHING, [&] { input_hidden_bf16(lds, xe); });
    // first K/V block of this workgroup's chunk (EARLY: stand-ins for a workgroup without one)
    const int kv0 = ga.active ? ga.p0 : 0;
    const int kv1 = ga.active ? min(ga.p1, ga.p0 + MQ_ATT_BLOCK) : 0;
    // read-only stand-in row for positions that must not fetch a cache row (row 0 of the cos table)
    const bf16_t* kv_dummy = p.cos;
    auto k_early = [&](int l) { kv_load_k<true>(kv, kv_base(p.kc, p, l, h), kv0, kv1, pos, kv_dummy); };
    if constexpr (EARLY) {
      if (p.num_layers > 0) k_early(0);
    }
    for (int l = 0; l < p.num_layers; ++l) {
      const MqLayerW w = lds_layer(s_layers, l);
      const int par = l & 1;
      // exchange epoch of this step and layer: never 0, and consecutive layers have consecutive
      // epochs (cyclic in [1, MQ_XEP_PERIOD]), so a buffer's previous words carry other epochs
      // and other tags
      const uint32_t e = mq_xep_epoch(xep0, (uint64_t)step * (uint32_t)p.num_layers + (uint32_t)l);
      stamp(p, rw, l, 0);
      gqkv_run(wq, w, h, j, NG, lds);
      stamp(p, rw, l, 1);
      // q|k|v -> attention: epoch words inside the kv-head group.  The gate|up weights go out two
      // phases ahead, during the attention phase, from workgroups without an attention chunk;
      // the others issue them after the O projection (a deep queue stalls the issue of loads and
      // would delay their attention, the partial merge and the O projection, which are on the
      // critical path).  Workgroups with a chunk issue its K/V rows here instead: issued before
      // the q|k|v dot products (whose loads are conditional), they made the compiler's wait for
      // the q|k|v weights wait for them too.
      phase_step(
          [&] { gqkv_publish(x->q[par][h], e, j, NG, lds, true); },
          [&] {
            if constexpr (EARLY) {
              // a workgroup without a chunk (some cache lengths below ~990 leave the last one
              // idle) takes the gate|up weights here, as in the other variant
              if (!ga.active) {
                gu_load(wgu, w, rw, G, true);
              } else {
                kv_load_v<true>(kv, kv_base(p.vc, p, l, h), kv0, kv1, pos, kv_dummy);
                if (ga.local) {
                  opart_load(wo, w, h, j, NG);
                  gu_load(wgu, w, rw, G, true, true);
                }
              }
            } else {
              if (!ga.active) {
                gu_load(wgu, w, rw, G, true);
              } else if (ga.local) {
                // local mode: no exchange follows the attention, so the O rows go now, and the
                // gate|up weights too, landing during the attention instead of during the
                // O-partial exchange; fixed load counts keep the compiler's wait for the K/V
                // rows from waiting for them
                kv_block_load<true>(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), kv0,
                                    kv1, pos, kv_dummy);
                opart_load(wo, w, h, j, NG);
                gu_load(wgu, w, rw, G, true, true);
              } else {
                kv_block_load<false>(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), kv0,
                                     kv1, pos, kv_dummy);
              }
            }
          },
          [&] {
            if (ga.active)
              attn_input(x->q[par][h], e, sy, w.q_norm, w.k_norm, cs, sn, p.scale_log2, lds);
          });
      stamp(p, rw, l, 2);
      if (ga.active) attn_core(p, l, h, ga.p0, ga.p1, pos, ga.has_new, kv, lds, ga.local);
      stamp(p, rw, l, 3);
      if (!ga.local) {
        // chunk partials -> merge: tagged words of the group's slots, polled by every thread
        phase_step([&] { gattn_publish(p, l, pos, h, j, ga, lds, x->part[par], e, true); },
                   [&] { opart_load(wo, w, h, j, NG, true); }, MQ_NOTHING);
        group_merge(x->part[par], h, ga.nch, lds, (int)xtag(e), sy);
      }
      stamp(p, rw, l, 4);
      opart_run(wo, w, h, j, NG, lds);
      stamp(p, rw, l, 5);
      // O partials -> a: tagged words in every group's copy, polled by every thread
      phase_step([&] {
                   opart_publish(&x->opart[par][0][0][0], h, j, NG, lds, e);
                   // local mode: the new position's K/V row (ALDS_KN/VN are still intact)
                   if (ga.local && ga.has_pos) attn_cache_row(p, l, h, pos, lds);
                 },
                 [&] { if (ga.active && !ga.local) gu_load(wgu, w, rw, G, true); }, MQ_NOTHING);
      gu_input_all(&x->opart[par][copy][0][0], lds, (int)xtag(e), sy);
      stamp(p, rw, l, 6);
      gu_run(wgu, w, rw, G, lds);
      stamp(p, rw, l, 7);
      // silu(gate) * up -> down: tagged words in every group's copy, polled by every thread
      phase_step([&] { gu_publish(&x->m[par][0][0], rw, G, lds, e); },
                 [&] { down_load(wd, w, rw, G, true); }, MQ_NOTHING);
      m_input_all(x->m[par][copy], lds + LDS_IN, (int)xtag(e), sy);
      stamp(p, rw, l, 8);
      down_run(wd, w, rw, G, lds);
      stamp(p, rw, l, 9);
      // layer output -> next layer (or the LM head): epoch words
      phase_step(
          [&] {
            float res = lane_id() < nrh ? lds[LDS_A + r0h + lane_id()] : 0.f;
            down_publish(rw, G, lds, res, [](int, float) {});
            hidden_publish(p, l, r0h, nrh, res, e);
          },
          [&] {
            if (l + 1 < p.num_layers) {
              gqkv_load(wq, lds_layer(s_layers, l + 1), h, j, NG, true);
              if constexpr (EARLY) k_early(l + 1);
            }
          },
          MQ_NOTHING);
      hidden_input_all(lds + LDS_IN, lds + LDS_HID, x->h[par][copy], e, sy);
      stamp(p, rw, l, 10);
    }
    const bool more = step + 1 < p.nsteps;
    lm_head_run(p, rw, G, lds, p.tok_out + step, p.nsteps == 1 ? p.logits : nullptr, pos, true,
                false, more, epoch0 + (uint32_t)step + 1, true,
                mq_xep_advance(xep0, (uint64_t)(step + 1) * (uint32_t)p.num_layers), !more);
    if (more) {
      // the next step's first weights do not depend on its token: in flight during the wait
      if (p.num_layers > 0) gqkv_load(wq, lds_layer(s_layers, 0), h, j, NG, true);
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
  MqExchange* x = p.x;
  MqSync* sy = &p.st->sync;
  const int h = wg % MQ_GROUPS, j = wg / MQ_GROUPS, NG = G / MQ_GROUPS;
  const int par = l & 1;
  const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
  // the (value, epoch) words of this mode carry epoch 0: written by a completed earlier kernel,
  // they are read without waiting (copy 0 of the grid-wide buffers).  Its tagged words carry the
  // epoch the persistent kernel would give this layer (mq_xep_epoch(xep, l); the LM-head kernel
  // advances xep by num_layers), so a persistent launch after steps of this mode never finds a
  // stale tagged word whose two tag bits match its expected epoch.
  const uint32_t xep = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&p.st->xep.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const uint32_t et = mq_xep_epoch(xep, (uint32_t)l);
  const uint64_t* xprev = x->h[(l + 1) & 1][0];   // layer l - 1's output
  // the layer input: the embedding row for layer 0, else the previous layer's output
  auto load_x = [&](float* dst) {
    if (l == 0) wave_copy_bf16_1024(dst, xe);
    else hidden_gather(dst, nullptr, xprev, 0, sy);
  };
  if constexpr (PH == 5) {
    phase_sync(MQ_NOTHING, [&] {
      if (p.num_layers == 0) wave_copy_bf16_1024(lds + LDS_IN, xe);
      else hidden_gather(lds + LDS_IN, nullptr, x->h[(p.num_layers - 1) & 1][0], 0, sy);
    });
    // the step's epochs were mq_xep_epoch(xep, 0 .. num_layers - 1)
    lm_head_run(p, wg, G, lds, p.tok_out, p.logits, pos, true, false, false, 0, true,
                mq_xep_advance(xep, (uint32_t)p.num_layers));
  } else {
    const MqLayerW w = p.layers[l];
    if constexpr (PH == 0) {
      QkvSet ws;
      gqkv_load(ws, w, h, j, NG);
      phase_sync(MQ_NOTHING, [&] { load_x(lds + LDS_IN); });
      gqkv_run(ws, w, h, j, NG, lds);
      phase_finish([&] { gqkv_publish(x->q[par][h], 0, j, NG, lds); });
    }
    if constexpr (PH == 1) {
      const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, false);
      if (ga.active) {
        KvBlock kv;
        kv_block_load<false>(kv, kv_base(p.kc, p, l, h), kv_base(p.vc, p, l, h), ga.p0,
                             min(ga.p1, ga.p0 + MQ_ATT_BLOCK), pos, p.cos);
        q_operand_clear(lds);
        phase_sync(MQ_NOTHING, [&] {
          attn_input(x->q[par][h], 0, sy, w.q_norm, w.k_norm, p.cos + (size_t)pos * MQ_D,
                     p.sin + (size_t)pos * MQ_D, p.scale_log2, lds);
        });
        attn_core(p, l, h, ga.p0, ga.p1, pos, ga.has_new, kv, lds);
        phase_finish([&] {
          if (ga.local) gattn_publish_local(p, l, pos, h, ga, lds);
          else gattn_publish(p, l, pos, h, j, ga, lds, x->part[par], et);
        });
      } else if (!ga.local) {
        // no chunk: the slot is still rewritten (an empty partial), as in the persistent kernel
        phase_finish([&] { gattn_publish(p, l, pos, h, j, ga, lds, x->part[par], et); });
      }
    }
    if constexpr (PH == 2) {
      const GAttn ga = gattn_plan(j, NG, pos + 1, pos, p.attn_local_max, false);
      OPairSet ws;
      opart_load(ws, w, h, j, NG);
      if (ga.local)
        group_single(s->part, h, lds);
      else
        group_merge(x->part[par], h, ga.nch, lds, -1, sy);
      opart_run(ws, w, h, j, NG, lds);
      phase_finish([&] { opart_publish(&x->opart[par][0][0][0], h, j, NG, lds, et); });
    }
    if constexpr (PH == 3) {
      GateUpSet ws;
      gu_load(ws, w, wg, G);
      phase_sync(MQ_NOTHING, [&] {
        load_x(lds + LDS_HID);
        wait_all_memory();
        gu_input(&x->opart[par][0][0][0], lds);
      });
      gu_run(ws, w, wg, G, lds);
      phase_finish([&] { gu_publish(&x->m[par][0][0], wg, G, lds, et); });
    }
    if constexpr (PH == 4) {
      DownSet ws;
      down_load(ws, w, wg, G);
      int r0h, nrh;
      hid_rows(wg, G, r0h, nrh);
      const int t = lane_id();
      float res = 0.f;
      if (wave_id() == MQ_SYNC_WAVE && t < nrh) {
        const float xv = l == 0 ? bf16_to_f32(xe[r0h + t]) : hidden_row(xprev, r0h + t);
        res = a_elem(xv, &x->opart[par][0][0][0], r0h + t);
      }
      phase_sync(MQ_NOTHING, MQ_NOTHING);
      m_input_all(x->m[par][0], lds + LDS_IN, -1, sy);
      down_run(ws, w, wg, G, lds);
      phase_finish([&] {
        down_publish(wg, G, lds, res, [](int, float) {});
        hidden_publish(p, l, r0h, nrh, res, 0);
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
  phase_sync(MQ_NOTHING, [&] { wave_copy_bf16_1024(lds + LDS_IN, x); });
  qkv_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] { qkv_publish(p.s->qkv, blockIdx.x, gridDim.x, lds); });
}
__global__ void __launch_bounds__(MQ_THREADS) mq_op_rope_kernel(MqDecodeParams p, int l, int pos,
                                                                 float* q_out) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  const int h = blockIdx.x;
  const MqLayerW w = p.layers[l];
  phase_sync(MQ_NOTHING, [&] {
    attn_input_f(p.s->qkv, w.q_norm, w.k_norm, p.cos + (size_t)pos * MQ_D,
                 p.sin + (size_t)pos * MQ_D, h, p.scale_log2, lds);
  });
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
  kv_block_load<false>(kv, kv_base(p.kc, p, l, it.h), kv_base(p.vc, p, l, it.h), it.p0,
                       min(it.p1, it.p0 + MQ_ATT_BLOCK), -1, p.cos);
  q_operand_clear(lds);
  __syncthreads();
  if (wave_id() == MQ_SYNC_WAVE) {
    const float* qh = q_hat + 2 * it.h * MQ_D;
    q_operand_store(make_float2(qh[2 * lane_id()], qh[2 * lane_id() + 1]),
                    make_float2(qh[MQ_D + 2 * lane_id()], qh[MQ_D + 2 * lane_id() + 1]), lds);
  }
  __syncthreads();
  attn_core(p, l, it.h, it.p0, it.p1, -1, false, kv, lds);
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
  phase_sync(MQ_NOTHING,
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
  phase_sync(MQ_NOTHING, [&] { wave_copy_coh<MQ_H>(lds + LDS_IN, a); });
  gu_run(ws, p.layers[l], blockIdx.x, gridDim.x, lds);
  phase_finish([&] { gu_publish_f(p.s->mlp, blockIdx.x, gridDim.x, lds); });
}
__global__ void __launch_bounds__(MQ_THREADS) mq_op_down_kernel(MqDecodeParams p, int l,
                                                                 const float* a, bf16_t* x_out) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  DownSet ws;
  down_load(ws, p.layers[l], blockIdx.x, gridDim.x);
  int r0, nr;
  hid_rows(blockIdx.x, gridDim.x, r0, nr);
  float res = lane_id() < nr ? ld_coh(a + r0 + lane_id()) : 0.f;
  phase_sync(MQ_NOTHING,
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
  phase_sync(MQ_NOTHING,
             [&] { wave_copy_bf16_1024(lds + LDS_IN, x); });
  lm_head_run(p, blockIdx.x, gridDim.x, lds, tok_out, logits, 0, false, round_norm);
}

// --------------------------------------------------------- fused short-prompt prefill
// The reference's prefill megakernel (prefill_megakernel, fused_prefill_megakernel_core.inl:
// 658-745, behind MegakernelFusedPrefillDecoder, bindings_fused_prefill.cpp:235-330): one
// cooperative launch runs every layer over all n <= 64 prompt positions with fp32 activations
// (bf16 weights, bf16 K/V cache rows, no rounding of the residual stream), then the final norm
// and the LM head of the last position.
// Here 256 workgroups x 512 threads run five stages per layer:
//   q|k|v GEMM (input RMSNorm folded in) -> attention per (kv head, 4-query block): q/k RMSNorm,
//   RoPE, K/V cache rows, causal softmax -> O GEMM + residual -> gate|up GEMM (post RMSNorm
//   folded in) + silu(g) * u -> down GEMM + residual.
// There is no barrier.  The activations that cross workgroups (the residual stream, q|k|v, the
// attention output, silu(g) * u) are tagged words (below) that each reader polls; q|k|v stays on
// the XCD that computes it, whose L2 serves its attention items.  A GEMM stage
// loads its weight tiles (16 rows each) first, then polls its fp32 input rows, which stream in
// behind the tiles.  The q|k|v and gate|up stages give a workgroup one 16-row block and 1-4
// column tiles (more as n grows, so that each workgroup reads one block of input rows, staged
// straight into LDS); the O and down stages give it one column tile and a group of rows.  Products run on v_mfma_f32_16x16x32_bf16 with
// the fp32 input split into three bf16 parts (hi + mid + lo represent it exactly), so each
// product is the exact product of the fp32 value and the bf16 weight, accumulated in fp32.
// The RMSNorm of a GEMM input is folded in: the MFMAs take x * w_norm and the epilogue scales
// each row by rsqrt(mean(x^2) + eps), which the same pass accumulates.
#define FPA_S 132                        // padded row stride (floats) of the attention tiles
#define FP_IN_FLOATS (MQ_WAVES * (MQ_H / 256) * 2 * 256)   // the staged input block (K = H)
#define FP_PART_FLOATS (8 * 4 * 256)                      // fp_gemm's partials
#define FP_LDS_FLOATS (FP_PART_FLOATS + 16 * MQ_I / 2)       // + the down stage's tile (bf16)
static_assert(FP_LDS_FLOATS >= 6 * 8 * 256 + 128 + FP_IN_FLOATS, "fp_gemm_rows16's carve fits");
#define FPA_KS 136                       // bf16 row stride of the attention's split q / k planes
static_assert(FP_LDS_FLOATS >= 3 * 72 * FPA_KS / 2 + 64 * FPA_S + 2 * 8 * 64,
              "the attention carve fits");
static_assert(FP_LDS_FLOATS >= MQ_LDS_FLOATS, "the LM head's LDS layout fits");

// The launch's synchronization area (zeroed by the launcher): one role-claim counter per XCD,
// each in its own 128-byte line.
#define FP_SYNC_WORDS (MQ_GROUPS * 32)
MQ_DEV uint32_t* fp_claims(uint32_t* bar) { return bar; }

// Tagged activation words.  Every fp32 activation that crosses workgroups between the fused
// prefill's stages (the residual stream, q|k|v, the attention output and silu(g) * u) is stored
// with its two lowest mantissa bits replaced by the launch's tag (1, 2 or 3; the host picks one
// that no row of the launch holds from an earlier launch, and cleared buffers hold 0): with a
// device-scope store, or for q|k|v, which only its own XCD reads, a plain store into that XCD's
// L2.  A reader polls its input words with device-scope loads until every one carries the tag,
// so the data and its arrival are one round trip and no barrier is needed; it removes the tag
// before use (a truncation below 2^-22 relative).  Each buffer is written once per launch (per
// layer and stage), so a word with the tag is the launch's final value.
MQ_DEV float fp_tagged(float v, uint32_t tag) {
  return __uint_as_float((__float_as_uint(v) & ~3u) | tag);
}
MQ_DEV float fp_untag(float v) { return __uint_as_float(__float_as_uint(v) & ~3u); }
MQ_DEV bool fp_tag4(uint4 u, uint32_t tag) {
  return ((u.x & 3u) == tag) & ((u.y & 3u) == tag) & ((u.z & 3u) == tag) & ((u.w & 3u) == tag);
}
MQ_DEV void fp_st_tag(float* p, float v, uint32_t tag) { st_coh(p, fp_tagged(v, tag)); }
// 16 bytes at byte offset `off` of the buffer from `base` (wave-uniform), with a device-scope
// (sc1) buffer load: coherent across the XCDs' L2s like the agent-scope atomics, but an ordinary
// load to the compiler (two 8-byte atomic loads per chunk made it spill the fused kernel's
// registers)
MQ_DEV uint4 fp_ld16_coh(const float* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7ffffff0, 0x00020000);
  const mq_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16);
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef unsigned int mq_u32x2 __attribute__((ext_vector_type(2)));
MQ_DEV uint2 fp_ld8_coh(const float* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7ffffff0, 0x00020000);
  const mq_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 16);
  return make_uint2(v.x, v.y);
}
// End of one round of a wave's poll: true once every lane's words carry the tag (`ok`), or when
// a set error flag (read every 16th round) or the spin bound (which sets it) ends the wait.
MQ_DEV bool fp_poll_done(bool ok, uint32_t& spins, MqSync* sy) {
  if (__all(ok)) return true;
  uint32_t ev = 0;
  if (lane_id() == 0 && (spins & 15) == 15)
    ev = __hip_atomic_load(&sy->err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (__builtin_amdgcn_readlane(ev, 0) != 0) return true;
  if (++spins > MQ_SPIN_LIMIT) {
    if (lane_id() == 0)
      __hip_atomic_store(&sy->err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  __builtin_amdgcn_s_sleep(1);
  return false;
}
// One tagged word, polled by this thread alone; returned without its tag.
MQ_DEV float fp_poll1(const float* p, uint32_t tag, MqSync* sy) {
  float v = ld_coh(p);
  for (uint32_t spins = 0; (__float_as_uint(v) & 3u) != tag; v = ld_coh(p)) {
    if ((spins & 15) == 15 &&
        __hip_atomic_load(&sy->err.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
      break;
    if (++spins > MQ_SPIN_LIMIT) {
      __hip_atomic_store(&sy->err.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return fp_untag(v);
}

// 16 weight rows (row0 .. row0 + 15, K bf16 each) as the B operand of the tile's MFMAs: wave w
// holds the 32-wide k-steps w, w + 8, ...; lane l holds row l % 16, k-dims 8 (l / 16) .. + 8.
template <int K>
struct FpTile {
  uint4 b[K / 256];
};
// `shared`: the tile is also loaded by other workgroups of this XCD in the same stage (plain
// loads, so that its L2 serves them after the first); otherwise non-temporal.
template <int K>
MQ_DEV void fp_tile_load(FpTile<K>& t, const bf16_t* row0, bool shared = false) {
  // after every store of the stage
  asm volatile("" ::: "memory");
  const int lane = lane_id(), wave = wave_id();
  const bf16_t* r = row0 + (size_t)(lane & 15) * K + 8 * (lane >> 4);
#pragma unroll
  for (int j = 0; j < K / 256; ++j)
    t.b[j] = shared ? ld16(r + 32 * (wave + 8 * j)) : ld_nt16(r + 32 * (wave + 8 * j));
}

// The same tile held in LDS instead of registers, for a stage whose input needs the registers
// (the down stage: 12 k-steps): wave w's operands at dst + (w (K / 256) + j) 64 + lane, where
// fp_tile_load would put them in t.b[j], loaded straight into LDS (global_load_lds_dwordx4).
// Counted by vmcnt like fp_tile_load's loads.
template <int K>
MQ_DEV void fp_tile_load_lds(uint4* dst, const bf16_t* row0) {
  asm volatile("" ::: "memory");
  const int lane = lane_id(), wave = wave_id();
  const bf16_t* r = row0 + (size_t)(lane & 15) * K + 8 * (lane >> 4);
  uint4* base = dst + __builtin_amdgcn_readfirstlane(wave) * (K / 256) * 64;
#pragma unroll
  for (int j = 0; j < K / 256; ++j)
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)(r + 32 * (wave + 8 * j)),
        (__attribute__((address_space(3))) void*)(base + j * 64), 16, 0, 0);
}

// x = hi + mid + lo exactly, each part bf16: v_cvt_pk_bf16_f32 rounds to nearest even, and each
// remainder is exact in fp32 (the leading part takes the top 8 significant bits, the next the
// following 8, the last the rest).
typedef float mq_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 mq_bf16x2_t __attribute__((ext_vector_type(2)));
MQ_DEV void split3_pair(float x0, float x1, uint32_t& h, uint32_t& m, uint32_t& l) {
  const mq_f32x2_t v = {x0, x1};
  const mq_bf16x2_t a = __builtin_convertvector(v, mq_bf16x2_t);
  const mq_f32x2_t r = v - __builtin_convertvector(a, mq_f32x2_t);
  const mq_bf16x2_t b = __builtin_convertvector(r, mq_bf16x2_t);
  const mq_bf16x2_t c = __builtin_convertvector(r - __builtin_convertvector(b, mq_f32x2_t),
                                                mq_bf16x2_t);
  h = __builtin_bit_cast(uint32_t, a);
  m = __builtin_bit_cast(uint32_t, b);
  l = __builtin_bit_cast(uint32_t, c);
}
MQ_DEV void split3_bf16(const float (&x)[8], mq_bf16x8_t& hi, mq_bf16x8_t& mid, mq_bf16x8_t& lo) {
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split3_pair(x[2 * i], x[2 * i + 1], h[i], m[i], l[i]);
  hi = bf16x8_of(make_uint4(h[0], h[1], h[2], h[3]));
  mid = bf16x8_of(make_uint4(m[0], m[1], m[2], m[3]));
  lo = bf16x8_of(make_uint4(l[0], l[1], l[2], l[3]));
}

// One residual GEMM tile (the O and down stages): C[r][c] = sum_k A[r][k] W[c][k] for the rows
// row_lo <= r < n of 16-row blocks rb0 .. rb0 + nbr - 1 (nbr <= 4) of the fp32 input A (row
// stride K; tagged words, polled until every one carries `tag`) and the 16 weight rows whose
// k-step j operand of this lane is tb(j) (FpTile order), then epi(row, col, v, res) for every
// such row and the tile's 16 columns, where res = pre(row, col) is loaded before the products
// (the residual), so its round trip overlaps them.  All 512 threads take part.
template <int K, class TB, class Pre, class Epi>
MQ_DEV void fp_gemm(const float* A, int n, int rb0, int nbr, TB tb, float* lds, Pre pre, Epi epi,
                    int row_lo, uint32_t tag, MqSync* sy) {
  // rows below row_lo are left to another workgroup (zero inputs, no outputs); block row i of
  // block b is row 16 (rb0 + b) + i
  const int lane = lane_id(), wave = wave_id();
  // per-wave partials [8 waves][4 blocks][16 rows][16 cols]: C element i of lane l is
  // (row 4 (l / 16) + i, column l % 16) of the block
  float* part = lds;
  // this thread's epilogue elements (idx = tid + 512 k) and their residuals, loaded first
  float res[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = tid() + MQ_THREADS * k, bl = idx >> 8, e = idx & 255;
    const int row = 16 * (rb0 + bl) + (e >> 4);
    res[k] = bl < nbr && row >= row_lo && row < n ? pre(row, e & 15) : 0.f;
  }
  for (int bb = 0; bb < nbr; ++bb) {
    // keeps the next block's loads from being hoisted into this one (they would pin registers)
    asm volatile("" ::: "memory");
    static_assert(K % 1024 == 0, "k-steps in groups of four");
    uint4 u[K / 256][2];
    const int row = 16 * (rb0 + bb) + (lane & 15);
    const bool in = row >= row_lo && row < n;
    // (rows outside [row_lo, n) load nothing and are zero)
    const uint32_t src = 4u * (uint32_t)(row * K + 8 * (lane >> 4) + 32 * wave);
    for (uint32_t spins = 0;;) {
      bool ok = true;
      if (in) {
#pragma unroll
        for (int j = 0; j < K / 256; ++j) {
          u[j][0] = fp_ld16_coh(A, src + 4u * 256u * j);
          u[j][1] = fp_ld16_coh(A, src + 4u * (256u * j + 4u));
          ok &= fp_tag4(u[j][0], tag);
          ok &= fp_tag4(u[j][1], tag);
        }
      }
      if (fp_poll_done(ok, spins, sy)) break;
    }
#pragma unroll
    for (int j = 0; j < K / 256; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        u[j][h] = in ? make_uint4(u[j][h].x & ~3u, u[j][h].y & ~3u, u[j][h].z & ~3u,
                                  u[j][h].w & ~3u)
                     : make_uint4(0, 0, 0, 0);
    // the weight operands are fetched four k-steps at a time (from LDS they would otherwise be
    // read one k-step at a time, each read's latency in series with the products; all at once
    // would take 48 more registers)
    mq_f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j0 = 0; j0 < K / 256; j0 += 4) {
      uint4 bt[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint4 t = tb(j0 + jj);
        mq_u32x4 v = {t.x, t.y, t.z, t.w};
        asm volatile("" : "+v"(v));   // keeps the scheduler from sinking each read to its use
        bt[jj] = make_uint4(v.x, v.y, v.z, v.w);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = j0 + jj;
        const float x[8] = {__uint_as_float(u[j][0].x), __uint_as_float(u[j][0].y),
                            __uint_as_float(u[j][0].z), __uint_as_float(u[j][0].w),
                            __uint_as_float(u[j][1].x), __uint_as_float(u[j][1].y),
                            __uint_as_float(u[j][1].z), __uint_as_float(u[j][1].w)};
        mq_bf16x8_t hi, mid, lo;
        split3_bf16(x, hi, mid, lo);
        const mq_bf16x8_t b = bf16x8_of(bt[jj]);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, b, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b, c, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      part[(wave * 4 + bb) * 256 + (4 * (lane >> 4) + i) * 16 + (lane & 15)] = c[i];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = tid() + MQ_THREADS * k, bl = idx >> 8, e = idx & 255;
    const int row = 16 * (rb0 + bl) + (e >> 4), col = e & 15;
    if (bl >= nbr || row < row_lo || row >= n) continue;
    float a = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < 8; ++w8) a += part[(w8 * 4 + bl) * 256 + e];
    epi(row, col, a, res[k]);
  }
  __syncthreads();
}

// One 16-row block of a normed GEMM stage over several column tiles: for the rows r < n of block
// rb of the fp32 input A (row stride K), C_q[r][c] = rsqrt(mean(A[r]^2) + eps) *
// sum_k A[r][k] w_norm[k] W_q[c][k] for the weight tiles q = g + NG s (g < ng, s < SUB) of t,
// then epi(row, g, col, v[SUB]) for every such row, tile group g < ng and column col < 16, with
// v[s] = C_{g + NG s} (SUB = 2: the gate and up tiles of one column range).  The block's input
// rows are loaded once, in one round trip, straight into LDS (global_load_lds_dwordx4: each wave
// stages its own k-steps, so they take no registers while in flight); all 512 threads take part,
// and the sums run in the same order as fp_gemm's.
template <int K, int NG, int SUB, class Epi>
MQ_DEV void fp_gemm_rows16(const float* A, int n, int rb, const bf16_t* w_norm,
                           const FpTile<K> (&t)[NG * SUB], int ng, float* lds, Epi epi,
                           uint32_t tag, MqSync* sy) {
  constexpr int NT = NG * SUB, KS = K / 256;
  static_assert(MQ_WAVES * KS * 2 * 256 <= FP_IN_FLOATS, "the staged input fits");
  const int lane = lane_id(), wave = wave_id();
  // per-wave partials [NT][8 waves][16 rows][16 cols] (C element i of lane l is row
  // 4 (l / 16) + i, column l % 16), the row sums of squares [8 waves][16 rows], then the staged
  // input [8 waves][KS][2][64 lanes][4 floats]: lane l's floats 4 h .. 4 h + 3 of k-step j
  float* part = lds;
  float* rs = lds + NT * 8 * 256;
  float* inp = rs + 128 + __builtin_amdgcn_readfirstlane(wave) * (KS * 2 * 256);
  // rows past n load row n - 1 (written, in range) and are zeroed when converted
  const int row = 16 * rb + (lane & 15);
  const bool in = row < n;
  const float* src = A + (size_t)min(row, n - 1) * K + 32 * wave + 8 * (lane >> 4);
  uint4 wn16[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) wn16[j] = ld16(w_norm + 32 * (wave + 8 * j) + 8 * (lane >> 4));
  // the wave's k-steps of the block, staged by device-scope (sc1) LDS loads and polled until
  // every word carries the tag
  for (uint32_t spins = 0;;) {
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(src + 256 * j + 4 * h),
            (__attribute__((address_space(3))) void*)(inp + (2 * j + h) * 256), 16, 0, 16);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        ok &= fp_tag4(reinterpret_cast<const uint4*>(inp + (2 * j + h) * 256)[lane], tag);
    if (fp_poll_done(ok, spins, sy)) break;
  }
  mq_f32x4_t c[NT];
#pragma unroll
  for (int q = 0; q < NT; ++q) c[q] = mq_f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const float4 a0 = reinterpret_cast<const float4*>(inp + 2 * j * 256)[lane];
    const float4 a1 = reinterpret_cast<const float4*>(inp + (2 * j + 1) * 256)[lane];
    float x[8] = {fp_untag(a0.x), fp_untag(a0.y), fp_untag(a0.z), fp_untag(a0.w),
                  fp_untag(a1.x), fp_untag(a1.y), fp_untag(a1.z), fp_untag(a1.w)};
    if (!in)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    float wn[8];
    unpack8(wn16[j], wn);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss = fmaf(x[e], x[e], ss);
      x[e] *= wn[e];
    }
    mq_bf16x8_t hi, mid, lo;
    split3_bf16(x, hi, mid, lo);
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      if (q % NG >= ng) continue;
      const mq_bf16x8_t b = bf16x8_of(t[q].b[j]);
      c[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b, c[q], 0, 0, 0);
      c[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, b, c[q], 0, 0, 0);
      c[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b, c[q], 0, 0, 0);
    }
    // one k-step's split parts live at a time (hoisting them all would exceed the registers)
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    if (q % NG >= ng) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      part[(q * 8 + wave) * 256 + (4 * (lane >> 4) + i) * 16 + (lane & 15)] = c[q][i];
  }
  const float sr = sum_xor32(sum_xor16(ss));   // the four lanes of row l % 16
  if (lane < 16) rs[wave * 16 + lane] = sr;
  __syncthreads();
  constexpr int KE = (NG * 256 + MQ_THREADS - 1) / MQ_THREADS;
#pragma unroll
  for (int k = 0; k < KE; ++k) {
    const int idx = tid() + MQ_THREADS * k, g = idx >> 8, e = idx & 255;
    const int r16 = e >> 4, rw = 16 * rb + r16;
    if (g >= ng || rw >= n) continue;
    float s = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < 8; ++w8) s += rs[w8 * 16 + r16];
    const float r = rsqrtf(s * (1.0f / K) + MQ_EPS);
    float v[SUB];
#pragma unroll
    for (int sb = 0; sb < SUB; ++sb) {
      float acc = 0.f;
#pragma unroll
      for (int w8 = 0; w8 < 8; ++w8) acc += part[((g + NG * sb) * 8 + w8) * 256 + e];
      v[sb] = acc * r;
    }
    epi(rw, g, e & 15, v);
  }
  __syncthreads();
}

// One row (128 dims, lane l: dims 2l, 2l + 1) of q or k: per-head RMSNorm with weight pair
// `w2`, then rotate-half RoPE with this lane's table pairs c2, s2 of the row's position
// (prefill_mk_qk_norm_rope_cache,
// fused_prefill_megakernel_core.inl:186-325): o_d = x_d c_d - x_{d+64} s_d for d < 64,
// o_d = x_{d-64} s_d + x_d c_d otherwise; the partner dims sit in lane l ^ 32.
MQ_DEV float2 fp_norm_rope(float2 x, uint32_t w2, uint32_t c2, uint32_t s2) {
  const int lane = lane_id();
  const float sc = rsqrtf(wave_sum(x.x * x.x + x.y * x.y) * (1.0f / MQ_D) + MQ_EPS);
  const float n0 = x.x * sc * bf16_lo(w2), n1 = x.y * sc * bf16_hi(w2);
  const float2 s0 = swap32(n0), s1 = swap32(n1);
  const float p0 = lane < 32 ? s0.y : s0.x, p1 = lane < 32 ? s1.y : s1.x;
  if (lane < 32)
    return make_float2(n0 * bf16_lo(c2) - p0 * bf16_lo(s2), n1 * bf16_hi(c2) - p1 * bf16_hi(s2));
  return make_float2(p0 * bf16_lo(s2) + n0 * bf16_lo(c2), p1 * bf16_hi(s2) + n1 * bf16_hi(c2));
}
// The same for two rows at once, 4 dims per lane: lanes 0-31 hold one row and lanes 32-63 the
// other, lane l dims 4 (l % 32) .. + 3 (weights w4, table entries c4, s4 of those dims); the
// RMSNorm sums over the lane's half and the partner dims sit in lane l ^ 16.
MQ_DEV float4 fp_norm_rope4(float4 x, uint2 w4, uint2 c4, uint2 s4) {
  const int lane = lane_id();
  const float sc = rsqrtf(sum_xor16(row16_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w)) *
                              (1.0f / MQ_D) + MQ_EPS);
  const float n0 = x.x * sc * bf16_lo(w4.x), n1 = x.y * sc * bf16_hi(w4.x);
  const float n2 = x.z * sc * bf16_lo(w4.y), n3 = x.w * sc * bf16_hi(w4.y);
  const bool lo = (lane & 16) == 0;              // dims < 64; the partner is lane ^ 16
  const float2 s0 = swap16(n0), s1 = swap16(n1), s2 = swap16(n2), s3 = swap16(n3);
  const float p0 = lo ? s0.y : s0.x, p1 = lo ? s1.y : s1.x;
  const float p2 = lo ? s2.y : s2.x, p3 = lo ? s3.y : s3.x;
  if (lo)
    return make_float4(n0 * bf16_lo(c4.x) - p0 * bf16_lo(s4.x), n1 * bf16_hi(c4.x) - p1 * bf16_hi(s4.x),
                       n2 * bf16_lo(c4.y) - p2 * bf16_lo(s4.y), n3 * bf16_hi(c4.y) - p3 * bf16_hi(s4.y));
  return make_float4(p0 * bf16_lo(s4.x) + n0 * bf16_lo(c4.x), p1 * bf16_hi(s4.x) + n1 * bf16_hi(c4.x),
                     p2 * bf16_lo(s4.y) + n2 * bf16_lo(c4.y), p3 * bf16_hi(s4.y) + n3 * bf16_hi(c4.y));
}

// Attention item (kv head h, query block qb = positions FP_QB qb .. FP_QB qb + FP_QB - 1) of
// layer `layer` (prefill_mk_causal_attention, fused_prefill_megakernel_core.inl:328-414): both
// query heads 2h, 2h + 1 of the block against keys 0 .. min(n, FP_QB (qb + 1)) - 1, fp32
// throughout (the keys normalised and rotated here from the raw q|k|v rows; the block's own
// positions' K/V rows are also written to the bf16 cache).  Scores use the reference's scale and
// an expf softmax.  The q k^T products run on MFMA from exact three-part bf16 splits of the fp32
// rows (below); then wave r holds query row r (position q0 + r / 2, head 2h + r % 2): lane j
// takes key j's score, the softmax is a wave reduction, and in P.V lane l accumulates dims
// 2l, 2l + 1 over the keys in order.
#define FP_QB 4
MQ_DEV float2 ldf2(const float* p) {
  const uint64_t u = *gptr<uint64_t>(p);
  return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}
MQ_DEV uint2 ld8(const void* p) {
  const uint64_t u = *gptr<uint64_t>(p);
  return make_uint2((uint32_t)u, (uint32_t)(u >> 32));
}
MQ_DEV float4 ldf4(const float* p) {
  const uint4 u = ld16(p);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                     __uint_as_float(u.w));
}
MQ_DEV void fp_attention(const MqDecodeParams& p, const MqFusedArgs& f, const MqLayerW& w,
                         int layer, int h, int qb, const float* qkv, float* att, float* lds) {
  static_assert(2 * FP_QB == MQ_WAVES, "one query row per wave");
  static_assert(MQ_FUSED_MAX_N <= 64, "one key per lane");
  // keys and query rows after norm + RoPE as three bf16 planes (hi, mid, lo: exact parts of the
  // fp32 values), the A / B operands of the score MFMAs
  bf16_t* Kp = reinterpret_cast<bf16_t*>(lds);  // [3][64][FPA_KS]
  bf16_t* Qp = Kp + 3 * 64 * FPA_KS;            // [3][8][FPA_KS]
  float* Vs = lds + 3 * 72 * FPA_KS / 2;        // [64][FPA_S] values
  float* Ss = Vs + 64 * FPA_S;                  // [8][64] scores
  float* Ps = Ss + 8 * 64;                      // [8][64] softmax weights
  const int n = f.n, q0 = FP_QB * qb, kn = min(n, q0 + FP_QB), qn = kn - q0;
  const int lane = lane_id(), wave = wave_id();
  constexpr int QKV = MQ_QDIM + 2 * MQ_KVDIM;
  const int half = lane >> 5, m4 = 4 * (lane & 31);
  const uint2 kw = ld8(w.k_norm + m4);
  const uint32_t qw = ld32(w.q_norm + 2 * lane);
  bf16_t* kc = p.kc + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D;
  bf16_t* vc = p.vc + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D;
  // key rows in pairs, lanes 0-31 row j0 = wave + 16 i and lanes 32-63 row j0 + 8 (4 dims per
  // lane, so a 16-byte load moves two rows), and this wave's query row: the RoPE table entries,
  // then the raw q|k|v words (tagged, written by this XCD), polled with device-scope loads until
  // all carry the tag.  The second row of a pair past the keys loads row kn - 1 and is not
  // stored.
  constexpr int KI = MQ_FUSED_MAX_N / (2 * MQ_WAVES);
  float4 kr[KI], vr[KI];
  uint2 kc4[KI], ks4[KI];
  float2 qr = make_float2(0.f, 0.f);
  uint32_t qc2 = 0, qs2 = 0;
  const int r = wave, pi = q0 + (r >> 1);        // this wave's query row and its position
  const bool has_q = r < 2 * qn;
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int j0 = wave + 2 * MQ_WAVES * i;
    if (j0 < kn) {
      const int j = min(j0 + MQ_WAVES * half, kn - 1);
      kc4[i] = ld8(p.cos + (size_t)j * MQ_D + m4);
      ks4[i] = ld8(p.sin + (size_t)j * MQ_D + m4);
    }
  }
  if (has_q) {
    qc2 = ld32(p.cos + (size_t)pi * MQ_D + 2 * lane);
    qs2 = ld32(p.sin + (size_t)pi * MQ_D + 2 * lane);
  }
  const uint32_t tag = (uint32_t)f.tag;
  for (uint32_t spins = 0;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int j0 = wave + 2 * MQ_WAVES * i;
      if (j0 < kn) {
        const int j = min(j0 + MQ_WAVES * half, kn - 1);
        const uint32_t off = 4u * (uint32_t)(j * QKV + MQ_QDIM + h * MQ_D + m4);
        const uint4 a = fp_ld16_coh(qkv, off), b = fp_ld16_coh(qkv, off + 4u * MQ_KVDIM);
        ok &= fp_tag4(a, tag);
        ok &= fp_tag4(b, tag);
        kr[i] = make_float4(fp_untag(__uint_as_float(a.x)), fp_untag(__uint_as_float(a.y)),
                            fp_untag(__uint_as_float(a.z)), fp_untag(__uint_as_float(a.w)));
        vr[i] = make_float4(fp_untag(__uint_as_float(b.x)), fp_untag(__uint_as_float(b.y)),
                            fp_untag(__uint_as_float(b.z)), fp_untag(__uint_as_float(b.w)));
      }
    }
    if (has_q) {
      const uint2 q = fp_ld8_coh(qkv, 4u * (uint32_t)(pi * QKV + (2 * h + (r & 1)) * MQ_D + 2 * lane));
      ok &= ((q.x & 3u) == tag) & ((q.y & 3u) == tag);
      qr = make_float2(fp_untag(__uint_as_float(q.x)), fp_untag(__uint_as_float(q.y)));
    }
    if (fp_poll_done(ok, spins, &p.st->sync)) break;
  }
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int j0 = wave + 2 * MQ_WAVES * i;
    if (j0 < kn) {
      const int j = j0 + MQ_WAVES * half;
      const float4 k = fp_norm_rope4(kr[i], kw, kc4[i], ks4[i]);
      if (j < kn) {
        uint32_t hw[2], mw[2], lw[2];
        split3_pair(k.x, k.y, hw[0], mw[0], lw[0]);
        split3_pair(k.z, k.w, hw[1], mw[1], lw[1]);
        *reinterpret_cast<uint2*>(Kp + j * FPA_KS + m4) = make_uint2(hw[0], hw[1]);
        *reinterpret_cast<uint2*>(Kp + (64 + j) * FPA_KS + m4) = make_uint2(mw[0], mw[1]);
        *reinterpret_cast<uint2*>(Kp + (128 + j) * FPA_KS + m4) = make_uint2(lw[0], lw[1]);
        *reinterpret_cast<float4*>(Vs + j * FPA_S + m4) = vr[i];
        if (j >= q0) {
          *reinterpret_cast<uint2*>(kc + (size_t)j * MQ_D + m4) =
              make_uint2((uint32_t)f32_to_bf16(k.x) | ((uint32_t)f32_to_bf16(k.y) << 16),
                         (uint32_t)f32_to_bf16(k.z) | ((uint32_t)f32_to_bf16(k.w) << 16));
          *reinterpret_cast<uint2*>(vc + (size_t)j * MQ_D + m4) =
              make_uint2((uint32_t)f32_to_bf16(vr[i].x) | ((uint32_t)f32_to_bf16(vr[i].y) << 16),
                         (uint32_t)f32_to_bf16(vr[i].z) | ((uint32_t)f32_to_bf16(vr[i].w) << 16));
        }
      }
    }
  }
  {
    // this wave's query row (zeros for a wave without one)
    uint32_t hq = 0, mq = 0, lq = 0;
    if (has_q) {
      const float2 q = fp_norm_rope(qr, qw, qc2, qs2);
      split3_pair(q.x, q.y, hq, mq, lq);
    }
    reinterpret_cast<uint32_t*>(Qp + r * FPA_KS)[lane] = hq;
    reinterpret_cast<uint32_t*>(Qp + (8 + r) * FPA_KS)[lane] = mq;
    reinterpret_cast<uint32_t*>(Qp + (16 + r) * FPA_KS)[lane] = lq;
  }
  __syncthreads();
  // Scores S = Q K^T on v_mfma_f32_16x16x32_bf16, wave w taking keys 16 w .. 16 w + 15: A rows
  // are the 8 query rows (rows 8-15 zero), B columns the keys.  The six products of the parts
  // down to hi * lo and mid * mid (smallest first) make each q k product exact to ~2^-23
  // relative (the dropped mid * lo, lo * mid and lo * lo terms), accumulated in fp32.
  if (wave < (kn + 15) / 16) {
    const int col = lane & 15, kd = 8 * (lane >> 4);
    const mq_bf16x8_t zero = bf16x8_of(make_uint4(0u, 0u, 0u, 0u));
    mq_f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < MQ_D / 32; ++ks) {
      mq_bf16x8_t a[3], b[3];
#pragma unroll
      for (int e = 0; e < 3; ++e) {
        b[e] = bf16x8_of(*reinterpret_cast<const uint4*>(
            Kp + (64 * e + 16 * wave + col) * FPA_KS + 32 * ks + kd));
        a[e] = col < 8 ? bf16x8_of(*reinterpret_cast<const uint4*>(
                             Qp + (8 * e + col) * FPA_KS + 32 * ks + kd))
                       : zero;
      }
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], c, 0, 0, 0);
    }
    // C element i of lane l: query row 4 (l / 16) + i, key 16 w + l % 16
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) Ss[(4 * (lane >> 4) + i) * 64 + 16 * wave + col] = c[i];
    }
  }
  __syncthreads();
  if (has_q) {
    // scores of keys j = lane <= pi (causal), the reference's scale
    const int j = lane;
    const float s = j < kn && j <= pi ? Ss[r * 64 + j] * rsqrtf((float)MQ_D) : -INFINITY;
    const float mx = wave_max(s);
    const float e = s == -INFINITY ? 0.f : expf(s - mx);
    const float inv = 1.0f / wave_sum(e);
    Ps[r * 64 + j] = e;
    // P.V (the weights just written by this wave: in-order LDS access within the wave)
    float o0 = 0.f, o1 = 0.f;
    const int jend = min(kn, pi + 1);
    for (int jj = 0; jj < jend; ++jj) {
      const float pw = Ps[r * 64 + jj];
      const float2 v = reinterpret_cast<const float2*>(Vs + jj * FPA_S)[lane];
      o0 = fmaf(pw, v.x, o0);
      o1 = fmaf(pw, v.y, o1);
    }
    st_coh64(reinterpret_cast<uint64_t*>(att + (size_t)pi * MQ_QDIM + (2 * h + (r & 1)) * MQ_D) +
                 lane,
             (uint64_t)__float_as_uint(fp_tagged(o0 * inv, (uint32_t)f.tag)) |
                 ((uint64_t)__float_as_uint(fp_tagged(o1 * inv, (uint32_t)f.tag)) << 32));
  }
  __syncthreads();
}

__global__ void __launch_bounds__(MQ_THREADS) mq_prefill_fused_kernel(MqDecodeParams p,
                                                                      MqFusedArgs f) {
  __shared__ __align__(16) float lds[FP_LDS_FLOATS];
  const int G = gridDim.x, n = f.n, t = tid();
  MqSync* sy = &p.st->sync;
  // Role from the hardware placement, as the persistent decode kernel claims it: xc is the XCD
  // the workgroup runs on and xj the order of its claim there; the role index wg = xc + 8 xj
  // replaces the launch index everywhere, so wg % 8 is the XCD (the L2-shared tiles and the
  // XCD-local q|k|v words rely on it).  A placement with more than G / 8 workgroups on one
  // XCD flags error 4; that workgroup returns and the others' waits end on the error flag.
  __shared__ int s_role;
  if (t == 0) {
    const uint32_t x = (uint32_t)xcc_id() & (MQ_GROUPS - 1);
    s_role = (int)(x + MQ_GROUPS * __hip_atomic_fetch_add(fp_claims(f.bar) + x, 1u,
                                                          __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT));
  }
  __syncthreads();
  const int wg = __builtin_amdgcn_readfirstlane(s_role);
  const int xc = wg % MQ_GROUPS, xj = wg / MQ_GROUPS, NX = G / MQ_GROUPS;
  if (xj >= NX) {
    if (t == 0) __hip_atomic_store(&sy->err.v, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const uint32_t tag = (uint32_t)f.tag;
  constexpr int QKV = MQ_QDIM + 2 * MQ_KVDIM;
  // this launch's buffers: each written once, by one stage, as tagged words its readers poll
  auto hbuf = [&](int i) { return f.h + (size_t)i * MQ_FUSED_MAX_N * MQ_H; };
  auto qkvbuf = [&](int l) { return f.qkv + (size_t)l * MQ_FUSED_MAX_N * QKV; };
  auto attbuf = [&](int l) { return f.att + (size_t)l * MQ_FUSED_MAX_N * MQ_QDIM; };
  auto mbuf = [&](int l) { return f.m + (size_t)l * MQ_FUSED_MAX_N * MQ_I; };
  // embedding rows (prefill_mk_embedding, fused_prefill_megakernel_core.inl:3-33; the audio
  // rows as the kernel's patch step, :693-703); a token id outside the vocabulary reads row 0
  // and sets the error flag to 2
  for (int row = wg; row < n; row += G) {
    const int pr = row - f.patch_start;
    const bool patched = pr >= 0 && pr < f.patch_len;
    int tok = patched ? 0 : f.tokens[row];
    if (tok < 0 || tok >= p.vocab) {
      if (t == 0) __hip_atomic_store(&sy->err.v, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      tok = 0;
    }
    const bf16_t* src = patched ? f.patch + (size_t)pr * MQ_H : p.embed + (size_t)tok * MQ_H;
    const uint32_t v = ld32(src + 2 * t);
    st_coh64(reinterpret_cast<uint64_t*>(hbuf(0) + (size_t)row * MQ_H) + t,
             (uint64_t)__float_as_uint(fp_tagged(bf16_lo(v), tag)) |
                 ((uint64_t)__float_as_uint(fp_tagged(bf16_hi(v), tag)) << 32));
  }
  const int nb = (n + 15) >> 4;
  // The O and down stages have 1024 / 16 = 64 column tiles, each shared by up to four
  // workgroups wg = tile + 64 part that take row groups of R rows, R the smallest of 1, 2, 4, 8,
  // 16 that is >= n / 4, so that a group never straddles two 16-row MFMA blocks (the block's
  // other rows are zero) and every workgroup reads only its rows of the input.  The workgroups
  // of a tile run on one XCD (wg % 8 = tile % 8) and share its weights through the L2.
  const int hb_tile = wg % (MQ_H / 16), hb_part = wg / (MQ_H / 16);
  const int hb_q = (n + 3) / 4;
  const int hb_rows = hb_q <= 1 ? 1 : hb_q <= 2 ? 2 : hb_q <= 4 ? 4 : hb_q <= 8 ? 8 : 16;
  const int hb_lo = hb_part * hb_rows, hb_hi = min(n, hb_lo + hb_rows), hb_rb = hb_lo / 16;
  const int hb_nb = hb_hi > hb_lo ? (hb_hi - 1) / 16 - hb_rb + 1 : 0;
  const bool hb_work = hb_lo < n;
  const bool hb_shared = n > hb_rows;
  // The q|k|v and gate|up stages give a workgroup one 16-row block and qn (gp) column tiles of 16
  // (gate|up: gp tiles of each), qn = 1, 2, 4, 4 and gp = 1, 2, 3, 3 for nb = 1 .. 4 row blocks,
  // and each reads one block of input rows, in one round trip.
  // q|k|v: XCD x computes the 32 tiles of kv head x (q heads 2x, 2x + 1, then k and v of x;
  // tile i of the head is qkv_tile(i)), so that its attention items poll them in its own L2:
  // member xj takes block xj / (32 / qn) and tiles qn (xj % (32 / qn)) + q.
  // gate|up: wg = block * groups + group, so the nb workgroups of a column group run on one XCD
  // and share its weight tiles through the L2.
  const int qn = nb == 1 ? 1 : nb == 2 ? 2 : 4, gp = nb == 1 ? 1 : nb == 2 ? 2 : 3;
  const int g_groups = MQ_I / 16 / gp;
  const int q_grp = xj % (32 / qn), q_rb = xj / (32 / qn);
  // tile i < 32 of kv head x: its 16-column index in q|k|v
  auto qkv_tile = [](int x, int i) {
    return i < 16 ? 16 * x + i : i < 24 ? 128 + 8 * x + (i - 16) : 192 + 8 * x + (i - 24);
  };
  const int g_grp = wg % g_groups, g_rb = wg / g_groups;
  const bool q_tile = q_rb < nb, g_tile = g_rb < nb;
  // Each GEMM stage loads its weight tiles, then polls its tagged input rows (the polls are
  // issued behind the tiles, which stream in meanwhile), then runs; the three sit in one branch
  // so that the tiles' registers never cross a join (the register allocator spills them
  // otherwise).  No grid barrier: every stage waits only for the words it reads.
  for (int l = 0; l < p.num_layers; ++l) {
    const MqLayerW* wl = p.layers + l;   // (fields read where used: fewer scalar registers held)
    const float* hin = hbuf(2 * l);
    float* hmid = hbuf(2 * l + 1);
    float* hout = hbuf(2 * l + 2);
    float* qkvl = qkvbuf(l);
    float* attl = attbuf(l);
    float* ml = mbuf(l);
    // q|k|v (prefill_mk_rmsnorm + prefill_mk_qkv_projection, :35-184)
    if (q_tile) {
      // (the head index passes through an empty asm so that the tile addresses are recomputed
      // here, not kept in registers across the layer loop)
      int hx = xc;
      asm volatile("" : "+s"(hx));
      FpTile<MQ_H> tq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < qn) fp_tile_load(tq[q], qkv_row(*wl, 16 * qkv_tile(hx, q_grp * qn + q)), nb > 1);
      // (tagged words with plain stores: only this XCD reads them, through its L2)
      fp_gemm_rows16<MQ_H, 4, 1>(hin, n, q_rb, wl->in_ln, tq, qn, lds,
                                 [&](int row, int g, int col, const float* v) {
        qkvl[(size_t)row * QKV + 16 * qkv_tile(hx, q_grp * qn + g) + col] = fp_tagged(v[0], tag);
      }, tag, sy);
    }
    // attention item (kv head xc, query block xj), from the q|k|v words of this XCD
    if (xj < (n + FP_QB - 1) / FP_QB) fp_attention(p, f, *wl, l, xc, xj, qkvl, attl, lds);
    // O projection + residual (prefill_mk_o_proj_residual, :417-472)
    if (hb_work) {
      FpTile<MQ_QDIM> to;
      fp_tile_load(to, wl->wo + (size_t)16 * hb_tile * MQ_QDIM, hb_shared);
      fp_gemm<MQ_QDIM>(attl, hb_hi, hb_rb, hb_nb, [&](int j) { return to.b[j]; }, lds,
                       [&](int row, int col) {
                         return fp_poll1(hin + (size_t)row * MQ_H + 16 * hb_tile + col, tag, sy);
                       },
                       [&](int row, int col, float v, float res) {
        fp_st_tag(hmid + (size_t)row * MQ_H + 16 * hb_tile + col, res + v, tag);
      }, hb_lo, tag, sy);
    }
    // post RMSNorm + gate|up + silu(g) * u (prefill_mk_mlp_gate_up, :474-544)
    if (g_tile) {
      // gate tiles in tgu[0 .. gp - 1], up tiles in tgu[3 .. 3 + gp - 1]
      FpTile<MQ_H> tgu[6];
#pragma unroll
      for (int q = 0; q < 3; ++q)
        if (q < gp) fp_tile_load(tgu[q], wl->wg + (size_t)16 * (g_grp * gp + q) * MQ_H, nb > 1);
#pragma unroll
      for (int q = 0; q < 3; ++q)
        if (q < gp) fp_tile_load(tgu[3 + q], wl->wu + (size_t)16 * (g_grp * gp + q) * MQ_H, nb > 1);
      fp_gemm_rows16<MQ_H, 3, 2>(hmid, n, g_rb, wl->post_ln, tgu, gp, lds,
                                 [&](int row, int g, int col, const float* v) {
        const float gt = v[0], u = v[1];
        fp_st_tag(ml + (size_t)row * MQ_I + 16 * (g_grp * gp + g) + col,
                  gt / (1.0f + expf(-gt)) * u, tag);
      }, tag, sy);
    }
    // down projection + residual (prefill_mk_mlp_down_residual, :546-599)
    if (hb_work) {
      // the tile in LDS (the stage's input rows take 96 registers)
      uint4* td = reinterpret_cast<uint4*>(lds + FP_PART_FLOATS);
      fp_tile_load_lds<MQ_I>(td, wl->wd + (size_t)16 * hb_tile * MQ_I);
      // (the tile's LDS reads wait for every load, the input polls included)
      const uint4* tdw = td + wave_id() * (MQ_I / 256) * 64 + lane_id();
      fp_gemm<MQ_I>(ml, hb_hi, hb_rb, hb_nb, [&](int j) { return tdw[j * 64]; }, lds,
                    [&](int row, int col) {
                      return fp_poll1(hmid + (size_t)row * MQ_H + 16 * hb_tile + col, tag, sy);
                    },
                    [&](int row, int col, float v, float res) {
        fp_st_tag(hout + (size_t)row * MQ_H + 16 * hb_tile + col, res + v, tag);
      }, hb_lo, tag, sy);
    }
  }
  // final RMSNorm of the last position (fp32, prefill_mk_final_norm, :601-650) + LM head argmax,
  // from the last layer's residual stream (or the embeddings), polled
  {
    const float* hl = hbuf(2 * p.num_layers) + (size_t)(n - 1) * MQ_H;
    lds[LDS_IN + 2 * t] = fp_poll1(hl + 2 * t, tag, sy);
    lds[LDS_IN + 2 * t + 1] = fp_poll1(hl + 2 * t + 1, tag, sy);
  }
  __syncthreads();
  lm_head_run(p, wg, G, lds, f.tok_out, f.logits, n - 1, false, false);
}

// ---------------------------------------------------------------------- state kernels
__global__ void mq_fill_state_kernel(MqState* st, int pos, int clear_err) {
  const int t = threadIdx.x;
  if (t == 0) {
    st->sync.done.v = 0;
    if (clear_err) {
      st->sync.err.v = 0;
      st->xep.v = 0;
    }
    st->sync.argmax.v = 0;
    st->pos.v = (uint32_t)pos;
    st->steps.v = 0;
  }
  if (t < MQ_GROUPS) st->place[t].v = 0;
}
// Debug: the exchange-epoch base (validated by the caller: xep < MQ_XEP_PERIOD).
__global__ void mq_set_xep_kernel(MqState* st, uint32_t xep) {
  if (threadIdx.x == 0) st->xep.v = xep;
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

size_t mq_fused_activation_bytes(int num_layers) {
  const size_t L = (size_t)(num_layers > 0 ? num_layers : 0);
  return (size_t)MQ_FUSED_MAX_N * 4 *
         ((2 * L + 1) * MQ_H + L * (MQ_QDIM + 2 * MQ_KVDIM + MQ_QDIM + MQ_I));
}
size_t mq_fused_workspace_bytes(int num_layers) {
  return mq_fused_activation_bytes(num_layers) + FP_SYNC_WORDS * 4;
}
void mq_fused_bind(MqFusedArgs* f, char* base, int num_layers) {
  const size_t L = (size_t)(num_layers > 0 ? num_layers : 0);
  float* q = reinterpret_cast<float*>(base);
  f->h = q;
  f->qkv = f->h + (2 * L + 1) * MQ_FUSED_MAX_N * MQ_H;
  f->att = f->qkv + L * MQ_FUSED_MAX_N * (MQ_QDIM + 2 * MQ_KVDIM);
  f->m = f->att + L * MQ_FUSED_MAX_N * MQ_QDIM;
  f->bar = reinterpret_cast<uint32_t*>(f->m + L * MQ_FUSED_MAX_N * MQ_I);
}
static int g_fused_blocks_per_cu = -1;
int mq_launch_prefill_fused(const MqDecodeParams& p, const MqFusedArgs& f, int grid,
                            hipStream_t stream) {
  if (device_info() != 0) return -1;
  if (g_fused_blocks_per_cu < 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void*>(mq_prefill_fused_kernel), MQ_THREADS, 0) !=
        hipSuccess)
      nb = 0;
    g_fused_blocks_per_cu = nb;
  }
  if (!g_coop_ok || g_fused_blocks_per_cu < 1 || grid > g_cu_count * g_fused_blocks_per_cu)
    return -2;
  if (grid < 256 || f.n < 1 || f.n > MQ_FUSED_MAX_N || f.tag < 1 || f.tag > 3) return -3;
  if (grid / MQ_GROUPS > 32) return -3;   // an XCD's 32 workgroups take the 32 q|k|v tiles of its head
  const int rc = mq_launch_zero(f.bar, FP_SYNC_WORDS * 4, stream);
  if (rc != 0) return rc;
  MqDecodeParams pc = p;
  MqFusedArgs fc = f;
  void* args[] = {&pc, &fc};
  hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(mq_prefill_fused_kernel),
                                            dim3(grid), dim3(MQ_THREADS), args, 0, stream);
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

int mq_launch_clear_state(MqState* st, MqExchange* x, hipStream_t stream) {
  const int rc = mq_launch_zero(x, sizeof(MqExchange), stream);
  if (rc != 0) return rc;
  return mq_launch_fill_state(st, 0, stream, true);
}

int mq_launch_set_position(MqState* st, MqExchange* x, int pos, hipStream_t stream) {
  const int rc = mq_launch_zero(&x->part[0][0], sizeof(x->part), stream);
  if (rc != 0) return rc;
  return mq_launch_fill_state(st, pos, stream);
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

int mq_launch_set_xep(MqState* st, uint32_t xep, hipStream_t stream) {
  if (xep >= MQ_XEP_PERIOD) return -3;
  mq_set_xep_kernel<<<1, 64, 0, stream>>>(st, xep);
  return launch_status();
}

int mq_read_xep(MqState* st, hipStream_t stream, uint32_t* xep_out) {
  uint32_t v = 0;
  if (hipMemcpyAsync(&v, &st->xep.v, 4, hipMemcpyDeviceToHost, stream) != hipSuccess) return -1;
  if (hipStreamSynchronize(stream) != hipSuccess) return -1;
  *xep_out = v;
  return 0;
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
// The split is capped at MQ_MAX_CHUNKS chunks per kv head (mq_attn_nchunks) and MqScratch.part
// holds that many, so every cache length the entry point accepts ([1, max_seq_len]) fits: the
// array's size does not depend on the input.
static_assert(sizeof(MqScratch::part) ==
                  sizeof(float) * MQ_NKV * MQ_MAX_CHUNKS * MQ_GQA * MQ_PART_STRIDE,
              "one partial slot per chunk the split can produce");

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
