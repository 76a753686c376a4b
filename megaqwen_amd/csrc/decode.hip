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
#define MQ_LDS_FLOATS 4608

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
      }
    }
  }

  template <class RowPtr, class Out>
  MQ_DEV void compute(RowPtr rowptr, int nr, const float* __restrict__ x, Out out) const {
    const int lane = lane_id(), wave = wave_id();
    if (wave >= MQ_CWAVES) return;
    const int nitems = nr * S;
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int it = wave + j * MQ_CWAVES;
      if (it < nitems) {
        const float* xs = x + (it % S) * KS + lane * 8;
        float acc = 0.f;
#pragma unroll
        for (int l = 0; l < NL; ++l) acc = dot8_lds(w[j][l], xs + l * 512, acc);
        acc = wave_sum(acc);
        if (lane == 0) out(it, acc);
      }
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
  const uint32_t wv = reinterpret_cast<const uint32_t*>(w)[t];
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
#define ALDS_KN 768       // [128] new-position k (bf16 values)
#define ALDS_VN 896       // [128] new-position v (bf16 values)
#define ALDS_SC 1024      // [2][MQ_ATT_BLOCK] scores / probabilities
#define ALDS_STAT (ALDS_SC + 2 * MQ_ATT_BLOCK)   // m[2], l[2], alpha[2]
#define ALDS_ORED (ALDS_STAT + 16)               // [MQ_CWAVES][256] per-wave partial outputs
// The merge runs after this item's partial has been published, so it reuses the score area.
#define ALDS_MW ALDS_SC                          // merge: (m, l)[2][64] then weights [2][64]
#define ALDS_MSUM (ALDS_MW + 512)                // merge: [4][2][128] partial sums
static_assert(ALDS_ORED + MQ_CWAVES * 256 <= MQ_LDS_FLOATS, "attention LDS carve");
static_assert(ALDS_MSUM + 1024 <= MQ_LDS_FLOATS, "attention merge LDS carve");

// q/k RMSNorm over one head held as (lane, lane + 64) of one wave, then rotate-half RoPE with
// the bf16 table row (fused_decode_ldg_common.inl:268-394):
//   o_i = x_i c_i - x_{i+64} s_i,  o_{i+64} = x_i s_{i+64} + x_{i+64} c_{i+64}.
MQ_DEV void head_norm_rope(float& lo, float& hi, const bf16_t* __restrict__ nw,
                           const bf16_t* __restrict__ cs, const bf16_t* __restrict__ sn) {
  const int lane = lane_id();
  const float ss = wave_sum(lo * lo + hi * hi);
  const float r = rsqrtf(ss * (1.0f / MQ_D) + MQ_EPS);
  const float a = lo * r * bf16_to_f32(nw[lane]);
  const float b = hi * r * bf16_to_f32(nw[lane + 64]);
  const float c_lo = bf16_to_f32(cs[lane]), c_hi = bf16_to_f32(cs[lane + 64]);
  const float s_lo = bf16_to_f32(sn[lane]), s_hi = bf16_to_f32(sn[lane + 64]);
  lo = a * c_lo - b * s_lo;
  hi = a * s_hi + b * c_hi;
}

MQ_DEV float* part_ptr(float* part, int h, int c, int j) {
  return part + ((size_t)(h * MQ_MAX_CHUNKS + c) * MQ_GQA + j) * MQ_PART_STRIDE;
}

// Sync-wave input of an attention item: raw q of query heads 2h, 2h+1, k and v of kv head h.
MQ_DEV void attn_input(const float* qkv, int h, float* lds) {
  const int lane = lane_id();
  float2 v[4];
  v[0] = ld_coh2(qkv + 2 * h * MQ_D + 2 * lane);
  v[1] = ld_coh2(qkv + 2 * h * MQ_D + 128 + 2 * lane);
  v[2] = ld_coh2(qkv + MQ_QDIM + h * MQ_D + 2 * lane);
  v[3] = ld_coh2(qkv + MQ_QDIM + MQ_KVDIM + h * MQ_D + 2 * lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) reinterpret_cast<float2*>(lds + ALDS_RAW)[lane + 64 * i] = v[i];
}

// Prologue of an attention item for kv head h at decode position `pos` (raw inputs in LDS):
// q-hat of query heads 2h, 2h+1; k-hat and v of the new position rounded to bf16 (kept as fp32)
// and, when `write_cache`, stored into the cache row `pos`.  Waves 0..3 each own one head.
MQ_DEV void attn_prologue(const MqDecodeParams& p, int layer, const MqLayerW& w, int h, int pos,
                          bool write_cache, float* lds) {
  const int lane = lane_id(), wave = wave_id();
  const float* raw = lds + ALDS_RAW;
  const bf16_t* cs = p.cos + (size_t)pos * MQ_D;
  const bf16_t* sn = p.sin + (size_t)pos * MQ_D;
  const size_t row = (((size_t)layer * MQ_NKV + h) * p.max_seq + pos) * MQ_D;
  if (wave < 2) {
    float lo = raw[wave * MQ_D + lane], hi = raw[wave * MQ_D + 64 + lane];
    head_norm_rope(lo, hi, w.q_norm, cs, sn);
    lds[ALDS_QS + wave * MQ_D + lane] = lo;
    lds[ALDS_QS + wave * MQ_D + 64 + lane] = hi;
  } else if (wave == 2) {
    float lo = raw[256 + lane], hi = raw[256 + 64 + lane];
    head_norm_rope(lo, hi, w.k_norm, cs, sn);
    const bf16_t blo = f32_to_bf16(lo), bhi = f32_to_bf16(hi);
    lds[ALDS_KN + lane] = bf16_to_f32(blo);
    lds[ALDS_KN + 64 + lane] = bf16_to_f32(bhi);
    if (write_cache) {
      p.kc[row + lane] = blo;
      p.kc[row + 64 + lane] = bhi;
    }
  } else if (wave == 3) {
    const bf16_t blo = f32_to_bf16(raw[384 + lane]), bhi = f32_to_bf16(raw[384 + 64 + lane]);
    lds[ALDS_VN + lane] = bf16_to_f32(blo);
    lds[ALDS_VN + 64 + lane] = bf16_to_f32(bhi);
    if (write_cache) {
      p.vc[row + lane] = blo;
      p.vc[row + 64 + lane] = bhi;
    }
  }
}

// K/V of up to MQ_ATT_BLOCK positions: position blk + k*28 + wave*4 + (lane/16) goes to compute
// wave `wave`, row lane/16, each lane holding 8 of the 128 dims (16 bytes).
struct KvBlock {
  uint4 k[MQ_ATT_NK], v[MQ_ATT_NK];
};
MQ_DEV void kv_block_load(KvBlock& b, const bf16_t* Kb, const bf16_t* Vb, int blk, int bend) {
  const int lane = lane_id(), wave = wave_id();
  if (wave >= MQ_CWAVES) return;
#pragma unroll
  for (int k = 0; k < MQ_ATT_NK; ++k) {
    const int pp = blk + k * 4 * MQ_CWAVES + wave * 4 + (lane >> 4);
    if (pp < bend) {
      b.k[k] = ld16(Kb + (size_t)pp * MQ_D);
      b.v[k] = ld16(Vb + (size_t)pp * MQ_D);
    } else {
      b.k[k] = b.v[k] = make_uint4(0, 0, 0, 0);
    }
  }
}
MQ_DEV const bf16_t* kv_base(const bf16_t* cache, const MqDecodeParams& p, int layer, int h) {
  return cache + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D + (lane_id() & 15) * 8;
}

MQ_DEV void attn_stat_init(float* lds) {
  if (tid() < 2) {
    lds[ALDS_STAT + tid()] = -INFINITY;
    lds[ALDS_STAT + 2 + tid()] = 0.f;
  }
}

// Core of one attention item: kv head h, cache positions [p0, p1), first block already in `b`.
// Rotated queries in ALDS_QS; position `pos_new` (if inside the range) takes its K/V from
// ALDS_KN/ALDS_VN instead of the cache.  Per block: q.K for 4 positions per wave-instruction
// (16 lanes x 8 dims, DPP row sums), max/exp pass in LDS, p * V accumulated in registers; blocks
// are merged with the running max.  Leaves m[2], l[2] in ALDS_STAT and the unnormalised o[2][128]
// in ALDS_ORED[0..255] (reference: fused_decode_ldg_common.inl:417-602; split-K precedent
// split_decode_gemm.cu:748-904).
MQ_DEV void attn_core(const MqDecodeParams& p, int layer, int h, int p0, int p1, int pos_new,
                      KvBlock& b, float* lds) {
  const float* qs = lds + ALDS_QS;
  const float* kn = lds + ALDS_KN;
  const float* vn = lds + ALDS_VN;
  float* sc = lds + ALDS_SC;
  float* stat = lds + ALDS_STAT;
  float* ored = lds + ALDS_ORED;
  const int lane = lane_id(), wave = wave_id();
  const bool cw = wave < MQ_CWAVES;
  const int g = lane >> 4, sub = lane & 15;
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

  for (int blk = p0; blk < p1; blk += MQ_ATT_BLOCK) {
    const int bend = min(p1, blk + MQ_ATT_BLOCK);
    if (blk != p0) kv_block_load(b, Kb, Vb, blk, bend);
    if (cw) {
#pragma unroll
      for (int k = 0; k < MQ_ATT_NK; ++k) {
        const int pp = blk + k * 4 * MQ_CWAVES + wave * 4 + g;
        float kv[8];
        unpack8(b.k[k], kv);
        if (pp == pos_new) {
#pragma unroll
          for (int e = 0; e < 8; ++e) kv[e] = kn[sub * 8 + e];
        }
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s0 = fmaf(q0[e], kv[e], s0);
          s1 = fmaf(q1[e], kv[e], s1);
        }
        s0 = row16_sum(s0);
        s1 = row16_sum(s1);
        if (pp < bend && sub == 0) {
          sc[pp - blk] = s0 * p.scale_log2;
          sc[MQ_ATT_BLOCK + pp - blk] = s1 * p.scale_log2;
        }
      }
    }
    __syncthreads();
    if (wave < 2) {
      float* s = sc + wave * MQ_ATT_BLOCK;
      const int nb = bend - blk;
      float mx = -INFINITY;
      for (int i = lane; i < nb; i += 64) mx = fmaxf(mx, s[i]);
      mx = wave_max(mx);
      const float m_old = stat[wave];
      const float m_new = fmaxf(m_old, mx);
      const float alpha = exp2f(m_old - m_new);
      float ls = 0.f;
      for (int i = lane; i < nb; i += 64) {
        const float e = exp2f(s[i] - m_new);
        s[i] = e;
        ls += e;
      }
      ls = wave_sum(ls);
      if (lane == 0) {
        stat[wave] = m_new;
        stat[2 + wave] = stat[2 + wave] * alpha + ls;
        stat[4 + wave] = alpha;
      }
    }
    __syncthreads();
    if (cw) {
      const float al0 = stat[4], al1 = stat[5];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc0[e] *= al0;
        acc1[e] *= al1;
      }
#pragma unroll
      for (int k = 0; k < MQ_ATT_NK; ++k) {
        const int pp = blk + k * 4 * MQ_CWAVES + wave * 4 + g;
        if (pp < bend) {
          float vv[8];
          unpack8(b.v[k], vv);
          if (pp == pos_new) {
#pragma unroll
            for (int e = 0; e < 8; ++e) vv[e] = vn[sub * 8 + e];
          }
          const float w0 = sc[pp - blk], w1 = sc[MQ_ATT_BLOCK + pp - blk];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc0[e] = fmaf(w0, vv[e], acc0[e]);
            acc1[e] = fmaf(w1, vv[e], acc1[e]);
          }
        }
      }
    }
    __syncthreads();
  }
  // reduce the 4 position rows of each compute wave, then the compute waves
  if (cw) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc0[e] += xor_lane(acc0[e], 16);
      acc0[e] += xor_lane(acc0[e], 32);
      acc1[e] += xor_lane(acc1[e], 16);
      acc1[e] += xor_lane(acc1[e], 32);
    }
    if (g == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ored[wave * 256 + sub * 8 + e] = acc0[e];
        ored[wave * 256 + MQ_D + sub * 8 + e] = acc1[e];
      }
    }
  }
  __syncthreads();
  if (tid() < 256) {
    float o = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < MQ_CWAVES; ++w8) o += ored[w8 * 256 + tid()];
    ored[tid()] = o;   // each thread rewrites only the slot it alone read last
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
MQ_DEV void attn_merge_head(const float* part, int h, int nch, float* att, float* lds) {
  float* mw = lds + ALDS_MW;      // (m, l) pairs [2][64] -> weights [2][64] at +256
  float* msum = lds + ALDS_MSUM;  // [4][2][128]
  const int t = tid();
  const int j = t >> 8, pr = (t >> 2) & 63, q = t & 3;
  float* pbase = const_cast<float*>(part);
  float2 ml = make_float2(0.f, 0.f);
  if (t < 2 * nch) ml = ld_coh2(part_ptr(pbase, h, t % nch, t / nch));
  float2 o2[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = q + 4 * i;
    o2[i] = c < nch ? ld_coh2(part_ptr(pbase, h, c, j) + 4 + 2 * pr) : make_float2(0.f, 0.f);
  }
  if (t < 2 * nch) reinterpret_cast<float2*>(mw)[(t / nch) * 64 + t % nch] = ml;
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
    st_coh(att + (2 * h + jj) * MQ_D + d, o);
  }
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

// P2 for an active item (inputs already in LDS, first K/V block in `kv`).  With one chunk per
// head the item normalises and writes att directly; otherwise it publishes its partial and the
// last chunk of the head to arrive (per-head counter, monotone within the step) merges them.
MQ_DEV void attn_run(const MqDecodeParams& p, int layer, const MqLayerW& w, int pos, int nch,
                     const AttnItem& it, KvBlock& kv, float* lds) {
  const int cache_len = pos + 1;
  float* s_att = p.s->att;
  attn_prologue(p, layer, w, it.h, pos, it.p1 == cache_len, lds);
  attn_stat_init(lds);
  __syncthreads();
  attn_core(p, layer, it.h, it.p0, it.p1, pos, kv, lds);
  if (nch == 1) {
    if (tid() < 256)
      st_coh(s_att + 2 * it.h * MQ_D + tid(),
             lds[ALDS_ORED + tid()] / lds[ALDS_STAT + 2 + (tid() >> 7)]);
    return;
  }
  attn_write_partial(p.s->part, it.h, it.c, lds);
  wait_all_memory();
  __syncthreads();
  __shared__ int s_last;
  if (tid() == 0) {
    const uint32_t old = __hip_atomic_fetch_add(&p.st->sync.attn[it.h].v, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    s_last = (old == (uint32_t)((layer + 1) * nch - 1));
  }
  __syncthreads();
  if (s_last) attn_merge_head(p.s->part, it.h, nch, s_att, lds);
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
                        float* logits, int pos, bool advance_pos, bool round_norm = false) {
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
      *tok_out = (int)argmax_key_index(kk);
      __hip_atomic_store(&sy->argmax.v, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int i = 0; i < MQ_BAR_STRIPES; ++i)
        __hip_atomic_store(&sy->bar[i].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int i = 0; i < MQ_NKV; ++i)
        __hip_atomic_store(&sy->attn[i].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (advance_pos)
        __hip_atomic_store(&p.st->pos.v, (uint32_t)(pos + 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sy->done.v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------------------------- kernels
// Reads and validates the step's position and input token.  The result is identical in every
// workgroup, so an invalid step makes all of them return before the first barrier.
MQ_DEV bool step_inputs(const MqDecodeParams& p, int& pos, int& tok) {
  pos = (int)__hip_atomic_load(&p.st->pos.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  tok = *p.tok_in;
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

__global__ void __launch_bounds__(MQ_THREADS) mq_decode_persistent_kernel(MqDecodeParams p) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  const int G = gridDim.x, wg = blockIdx.x;
  int pos, tok;
  if (!step_inputs(p, pos, tok)) return;
  const int nch = mq_attn_nchunks(pos + 1, G);
  const AttnItem item = attn_item(wg, nch, pos + 1);
  MqSync* sy = &p.st->sync;
  MqScratch* s = p.s;
  const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
  int r0h, nrh;
  row_range(MQ_H, wg, G, r0h, nrh);
  // residual of this workgroup's hidden rows, held by sync-wave lane t for row r0h + t
  float res = lane_id() < nrh ? bf16_to_f32(xe[r0h + lane_id()]) : 0.f;
  uint32_t nbar = 0;
  QkvSet wq;
  OSet wo;
  GateUpSet wgu;
  DownSet wd;
  KvBlock kv;
  if (p.num_layers > 0) qkv_load(wq, p.layers[0], wg, G);
  phase_sync(sy, 0, false, MQ_NOTHING, [&] { wave_copy_bf16_1024(lds + LDS_IN, xe); });
  for (int l = 0; l < p.num_layers; ++l) {
    const MqLayerW w = p.layers[l];
    stamp(p, wg, l, 0);
    qkv_run(wq, w, wg, G, lds);
    stamp(p, wg, l, 1);
    if (item.active)
      kv_block_load(kv, kv_base(p.kc, p, l, item.h), kv_base(p.vc, p, l, item.h), item.p0,
                    min(item.p1, item.p0 + MQ_ATT_BLOCK));
    phase_sync(sy, (++nbar) * (uint32_t)G, true, [&] { qkv_publish(s->qkv, wg, G, lds); },
               [&] { if (item.active) attn_input(s->qkv, item.h, lds); });
    stamp(p, wg, l, 2);
    if (item.active) {
      attn_run(p, l, w, pos, nch, item, kv, lds);
      wait_all_memory();
    }
    stamp(p, wg, l, 3);
    o_load(wo, w, wg, G);
    phase_sync(sy, (++nbar) * (uint32_t)G, true, MQ_NOTHING,
               [&] { wave_copy_coh<MQ_QDIM>(lds + LDS_IN, s->att); });
    stamp(p, wg, l, 4);
    o_run(wo, w, wg, G, lds);
    stamp(p, wg, l, 5);
    gu_load(wgu, w, wg, G);
    phase_sync(sy, (++nbar) * (uint32_t)G, true, [&] { o_publish(s->a, wg, G, lds, res); },
               [&] { wave_copy_coh<MQ_H>(lds + LDS_IN, s->a); });
    stamp(p, wg, l, 6);
    gu_run(wgu, w, wg, G, lds);
    stamp(p, wg, l, 7);
    down_load(wd, w, wg, G);
    phase_sync(sy, (++nbar) * (uint32_t)G, true, [&] { gu_publish(s->mlp, wg, G, lds); },
               [&] { wave_copy_coh<MQ_I>(lds + LDS_IN, s->mlp); });
    stamp(p, wg, l, 8);
    down_run(wd, w, wg, G, lds);
    stamp(p, wg, l, 9);
    if (l + 1 < p.num_layers) qkv_load(wq, p.layers[l + 1], wg, G);
    phase_sync(sy, (++nbar) * (uint32_t)G, true,
               [&] { down_publish(wg, G, lds, res, [&](int r, float v) { hidden_out(p, l, r, v); }); },
               [&] { wave_copy_coh<MQ_H>(lds + LDS_IN, s->hidden); });
    stamp(p, wg, l, 10);
  }
  lm_head_run(p, wg, G, lds, p.tok_out, p.logits, pos, true);
}

// One kernel per phase (kernel boundaries replace the grid barriers; residuals are re-read).
template <int PH>
__global__ void __launch_bounds__(MQ_THREADS) mq_decode_phase_kernel(MqDecodeParams p, int l) {
  __shared__ __align__(16) float lds[MQ_LDS_FLOATS];
  const int G = gridDim.x, wg = blockIdx.x;
  int pos, tok;
  if (!step_inputs(p, pos, tok)) return;
  MqScratch* s = p.s;
  MqSync* sy = &p.st->sync;
  const bf16_t* xe = p.embed + (size_t)tok * MQ_H;
  int r0h, nrh;
  row_range(MQ_H, wg, G, r0h, nrh);
  const int t = lane_id();
  if constexpr (PH == 5) {
    phase_sync(sy, 0, false, MQ_NOTHING, [&] {
      if (p.num_layers == 0) wave_copy_bf16_1024(lds + LDS_IN, xe);
      else wave_copy_coh<MQ_H>(lds + LDS_IN, s->hidden);
    });
    lm_head_run(p, wg, G, lds, p.tok_out, p.logits, pos, true);
  } else {
    const MqLayerW w = p.layers[l];
    const int nch = mq_attn_nchunks(pos + 1, G);
    if constexpr (PH == 0) {
      QkvSet ws;
      qkv_load(ws, w, wg, G);
      phase_sync(sy, 0, false, MQ_NOTHING, [&] {
        if (l == 0) wave_copy_bf16_1024(lds + LDS_IN, xe);
        else wave_copy_coh<MQ_H>(lds + LDS_IN, s->hidden);
      });
      qkv_run(ws, w, wg, G, lds);
      phase_finish([&] { qkv_publish(s->qkv, wg, G, lds); });
    }
    if constexpr (PH == 1) {
      const AttnItem item = attn_item(wg, nch, pos + 1);
      if (item.active) {
        KvBlock kv;
        kv_block_load(kv, kv_base(p.kc, p, l, item.h), kv_base(p.vc, p, l, item.h), item.p0,
                      min(item.p1, item.p0 + MQ_ATT_BLOCK));
        phase_sync(sy, 0, false, MQ_NOTHING, [&] { attn_input(s->qkv, item.h, lds); });
        attn_run(p, l, w, pos, nch, item, kv, lds);
      }
    }
    if constexpr (PH == 2) {
      OSet ws;
      o_load(ws, w, wg, G);
      float res = 0.f;
      if (t < nrh) res = l == 0 ? bf16_to_f32(xe[r0h + t]) : ld_coh(s->hidden + r0h + t);
      phase_sync(sy, 0, false, MQ_NOTHING,
                 [&] { wave_copy_coh<MQ_QDIM>(lds + LDS_IN, s->att); });
      o_run(ws, w, wg, G, lds);
      phase_finish([&] { o_publish(s->a, wg, G, lds, res); });
    }
    if constexpr (PH == 3) {
      GateUpSet ws;
      gu_load(ws, w, wg, G);
      phase_sync(sy, 0, false, MQ_NOTHING, [&] { wave_copy_coh<MQ_H>(lds + LDS_IN, s->a); });
      gu_run(ws, w, wg, G, lds);
      phase_finish([&] { gu_publish(s->mlp, wg, G, lds); });
    }
    if constexpr (PH == 4) {
      DownSet ws;
      down_load(ws, w, wg, G);
      float res = t < nrh ? ld_coh(s->a + r0h + t) : 0.f;
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
  __shared__ __align__(16) float lds[1024];
  const int h = blockIdx.x;
  phase_sync(&p.st->sync, 0, false, MQ_NOTHING, [&] { attn_input(p.s->qkv, h, lds); });
  attn_prologue(p, l, p.layers[l], h, pos, true, lds);
  __syncthreads();
  if (tid() < 256) q_out[2 * h * MQ_D + tid()] = lds[ALDS_QS + tid()];
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
                min(it.p1, it.p0 + MQ_ATT_BLOCK));
  if (tid() < 256) lds[ALDS_QS + tid()] = q_hat[2 * it.h * MQ_D + tid()];
  attn_stat_init(lds);
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
__global__ void mq_fill_state_kernel(MqState* st, int pos) {
  const int t = threadIdx.x;
  if (t < MQ_BAR_STRIPES) st->sync.bar[t].v = 0;
  if (t < MQ_NKV) st->sync.attn[t].v = 0;
  if (t == 0) {
    st->sync.done.v = 0;
    st->sync.err.v = 0;
    st->sync.argmax.v = 0;
    st->pos.v = (uint32_t)pos;
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
          &nb, reinterpret_cast<const void*>(mq_decode_persistent_kernel), MQ_THREADS, 0) !=
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
  *grid_out = g_cu_count;  // one 512-thread workgroup per CU
  return 0;
}

static int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -(int)e - 1000;
}

int mq_launch_decode(const MqDecodeParams& p, int mode, int grid, hipStream_t stream) {
  if (grid < 64 || grid > 4096) return -3;
  if (mode == MQ_MODE_PERSISTENT) {
    MqDecodeParams pc = p;
    void* args[] = {&pc};
    hipError_t e = hipLaunchCooperativeKernel(
        reinterpret_cast<const void*>(mq_decode_persistent_kernel), dim3(grid), dim3(MQ_THREADS),
        args, 0, stream);
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

int mq_launch_fill_state(MqState* st, int pos, hipStream_t stream) {
  mq_fill_state_kernel<<<1, 64, 0, stream>>>(st, pos);
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
