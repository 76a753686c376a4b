// Device-side building blocks for the gfx950 (CDNA4) decode/prefill kernels.
//
// Everything here is written for wave64: reductions use DPP row operations inside a 16-lane
// row and cross-row swizzles, never 32-lane warp shuffles.  bf16 values are carried as raw
// 16-bit patterns (uint16_t) and widened with a shift, so no vendor bf16 type is involved.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq_config.h"

typedef uint16_t bf16_t;

#define MQ_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------- bf16 <-> fp32
MQ_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
MQ_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
MQ_DEV float bf16_to_f32(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Round-to-nearest-even fp32 -> bf16 (the rounding torch and __float2bfloat16 use): gfx950's
// v_cvt_pk_bf16_f32 under the default rounding mode (a NaN stays a NaN).
MQ_DEV bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }
MQ_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---------------------------------------------------------------------------- loads
// Weights are streamed once per token and never fit in the 256 MB MALL next to the KV cache,
// so they are loaded non-temporally (no L2 allocation priority).
// Every pointer these helpers take is global memory.  They load through the global address
// space explicitly: a pointer whose origin the compiler cannot trace (the weight table is read
// from LDS) would otherwise be loaded with FLAT instructions, which also count in lgkmcnt, so the
// next LDS wait or barrier of the wave would wait for the whole weight prefetch to land.
#define MQ_GLOBAL __attribute__((address_space(1)))
typedef unsigned int mq_u32x4 __attribute__((ext_vector_type(4)));
template <class T>
MQ_DEV const MQ_GLOBAL T* gptr(const void* p) {
  return (const MQ_GLOBAL T*)(p);
}
MQ_DEV uint4 ld_nt16(const void* p) {
  const mq_u32x4 v = __builtin_nontemporal_load(gptr<mq_u32x4>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
MQ_DEV uint4 ld16(const void* p) {
  const mq_u32x4 v = *gptr<mq_u32x4>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
MQ_DEV uint32_t ld32(const void* p) { return *gptr<uint32_t>(p); }

// dot of 8 bf16 (one 16-byte load) with 8 fp32 values
MQ_DEV float dot8(uint4 w, const float* x, float acc) {
  acc = fmaf(bf16_lo(w.x), x[0], acc);
  acc = fmaf(bf16_hi(w.x), x[1], acc);
  acc = fmaf(bf16_lo(w.y), x[2], acc);
  acc = fmaf(bf16_hi(w.y), x[3], acc);
  acc = fmaf(bf16_lo(w.z), x[4], acc);
  acc = fmaf(bf16_hi(w.z), x[5], acc);
  acc = fmaf(bf16_lo(w.w), x[6], acc);
  acc = fmaf(bf16_hi(w.w), x[7], acc);
  return acc;
}
MQ_DEV float dot8_lds(uint4 w, const float* x_lds, float acc) {
  float4 a = *reinterpret_cast<const float4*>(x_lds);
  float4 b = *reinterpret_cast<const float4*>(x_lds + 4);
  float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return dot8(w, xs, acc);
}
// Eight bf16-exact fp32 values (e.g. from LDS) packed back into 16 bytes of bf16.
MQ_DEV uint4 pack8_bf16(const float* x) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    u[i] = (__float_as_uint(x[2 * i]) >> 16) | (__float_as_uint(x[2 * i + 1]) & 0xffff0000u);
  return make_uint4(u[0], u[1], u[2], u[3]);
}
MQ_DEV void unpack8(uint4 w, float* o) {
  o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x);
  o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
  o[4] = bf16_lo(w.z); o[5] = bf16_hi(w.z);
  o[6] = bf16_lo(w.w); o[7] = bf16_hi(w.w);
}

// ---------------------------------------------------------------------------- wave64 reductions
// DPP control words (GCN/CDNA encoding).
#define MQ_DPP_QUAD_XOR1 0xB1   // quad_perm [1,0,3,2]
#define MQ_DPP_QUAD_XOR2 0x4E   // quad_perm [2,3,0,1]
#define MQ_DPP_ROW_HALF_MIRROR 0x141
#define MQ_DPP_ROW_MIRROR 0x140

template <int CTRL>
MQ_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over each 16-lane row; every lane of the row receives the row total.
MQ_DEV float row16_sum(float v) {
  v += dpp_f<MQ_DPP_QUAD_XOR1>(v);
  v += dpp_f<MQ_DPP_QUAD_XOR2>(v);
  v += dpp_f<MQ_DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f<MQ_DPP_ROW_MIRROR>(v);
  return v;
}
MQ_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f<MQ_DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_f<MQ_DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_f<MQ_DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<MQ_DPP_ROW_MIRROR>(v));
  return v;
}
// Arbitrary lane exchange through ds_bpermute (LDS crossbar, no LDS storage).
MQ_DEV float xor_lane(float v, int mask) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}
// Cross-row steps with the gfx950 row swaps (VALU, no LDS round trip).  With both operands x,
// v_permlane16_swap returns (rows 0,0,2,2 of x ; rows 1,1,3,3 of x) and v_permlane32_swap returns
// (lanes 0-31 twice ; lanes 32-63 twice), so the pair's sum (or max) is the value combined with
// lane ^ 16 (^ 32), identical in both lanes of a pair.
MQ_DEV float2 swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
MQ_DEV float2 swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Totals of four per-lane partial sums a0..a3 over the 64 lanes, with two row exchanges per
// step instead of one per value: v_permlane32_swap(a, b) yields (a_lo | b_lo, a_hi | b_hi), so
// one swap + add folds a over lanes ^32 into lanes 0-31 and b into lanes 32-63; then
// v_permlane16_swap of the two folds leaves value j folded over lanes ^16 and ^32 in lanes
// 16j..16j+15, and a DPP row sum finishes it.  Lanes 16j..16j+15 receive the total of aj.
MQ_DEV float sum4_rows(float a0, float a1, float a2, float a3) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0), __float_as_uint(a2), false,
                                                  false);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(a1), __float_as_uint(a3), false,
                                                  false);
  const float x0 = __uint_as_float(p[0]) + __uint_as_float(p[1]);   // a0 | a2
  const float x1 = __uint_as_float(q[0]) + __uint_as_float(q[1]);   // a1 | a3
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x0), __float_as_uint(x1), false,
                                                  false);
  return row16_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}
// Totals over 32-lane halves of two values (a0: lanes 0-31 | lanes 32-63 are two sums, same for
// a1): lanes 0-15 receive a0's low-half total, 16-31 a1's low-half total, 32-47 a0's high-half
// total, 48-63 a1's high-half total.
MQ_DEV float sum2_halves(float a0, float a1) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a0), __float_as_uint(a1), false,
                                                  false);
  return row16_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}
MQ_DEV float sum_xor16(float v) { const float2 p = swap16(v); return p.x + p.y; }
MQ_DEV float sum_xor32(float v) { const float2 p = swap32(v); return p.x + p.y; }
MQ_DEV float max_xor16(float v) { const float2 p = swap16(v); return fmaxf(p.x, p.y); }
MQ_DEV float max_xor32(float v) { const float2 p = swap32(v); return fmaxf(p.x, p.y); }
// Sum over all 64 lanes; every lane receives the total.
MQ_DEV float wave_sum(float v) {
  return sum_xor32(sum_xor16(row16_sum(v)));
}
MQ_DEV float wave_max(float v) {
  return max_xor32(max_xor16(row16_max(v)));
}

// Workgroup sum of one value per thread; `red` is MQ_WAVES floats of LDS.  All threads
// receive the total.  Contains two __syncthreads.
MQ_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < MQ_WAVES; ++i) t += red[i];
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------- argmax keys
// (value, index) packed so that unsigned 64-bit max picks the largest value and, among equal
// values, the LOWEST index.  Monotone float->uint map: flip all bits of negatives, set the sign
// bit of non-negatives.
MQ_DEV uint64_t argmax_key(float v, uint32_t idx) {
  uint32_t u = __float_as_uint(v);
  uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - idx);
}
MQ_DEV uint32_t argmax_key_index(uint64_t k) { return 0xffffffffu - (uint32_t)(k & 0xffffffffu); }

MQ_DEV uint64_t u64_max(uint64_t a, uint64_t b) { return a > b ? a : b; }
MQ_DEV uint64_t wave_max_u64(uint64_t k) {
  int lane = __lane_id();
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    uint32_t olo = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, lo);
    uint32_t ohi = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, hi);
    k = u64_max(k, ((uint64_t)ohi << 32) | olo);
  }
  return k;
}

// ---------------------------------------------------------------------------- coherent exchange
// Activations crossing workgroups are written and read with agent-scope relaxed atomics, which
// gfx950 lowers to single `sc1` loads/stores that are coherent across the 8 XCD-private L2s.
// No release/acquire fences are used: those lower to whole-L2 writeback/invalidate
// (buffer_wbl2 / buffer_inv) and cost ~7 us per grid barrier on MI355X.  Ordering instead comes
// from words that carry their own epoch (a value and its epoch are one store and one load), and,
// for the one counter that remains (the LM head's completion count, which ends a step), from
// waiting for every outstanding memory operation of the wave (s_waitcnt 0) before the arrival
// atomic and issuing the dependent loads only after the count has been observed.
MQ_DEV void st_coh(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
MQ_DEV float ld_coh(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
}
MQ_DEV float2 ld_coh2(const float* p) {
  const uint64_t u = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}
MQ_DEV uint64_t ld_coh64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MQ_DEV void st_coh64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MQ_DEV void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// ------------------------------------------------------------------ XCD-local exchange
// Values exchanged only among workgroups of one XCD are stored with plain stores (no cache-
// bypass bits): the per-CU vector L1 is write-through, so the store lands in the XCD's L2 and
// stays there; the readers' agent-scope (sc1) loads above miss their own L1 and are served by
// that L2.  A device-scope (sc1) store also writes through to memory, which the reader does not
// need: measured on 256 co-resident workgroups exchanging one word per round inside their XCD,
// 0.49 us per round against 0.79 us with sc1 stores (512 words per group: 1.6 against 3.4 us).
// Readers on another XCD would not see these stores (their L2 may hold the line and the data
// never reaches memory before the kernel ends), so the kernels that use them assign workgroup
// roles from the hardware XCD index (xcc_id).  Workgroup-scope (sc0) loads are no substitute
// for the sc1 loads: they are served by the reader's own L1 and never observe another CU's
// stores.  The stores are single 64-bit (or 32-bit) instructions, so a word and its epoch or
// tag arrive together.
MQ_DEV void st_local64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
MQ_DEV void st_local32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
// Hardware XCD index of the executing workgroup (HW_REG_XCC_ID, bits 3:0).
MQ_DEV int xcc_id() { return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11)) & 15; }

// ---------------------------------------------------------------------------- sync state
// Sync state lives in its own 128-byte lines (one L2 line each on gfx950).
struct alignas(128) MqLine {
  uint32_t v;
  uint32_t pad[31];
};
struct alignas(128) MqLine64 {
  unsigned long long v;
  uint32_t pad[30];
};
struct MqSync {
  MqLine done;                 // LM-head completion counter
  MqLine err;                  // nonzero after a wait timed out or a bound was violated
  MqLine64 argmax;             // packed (value, index) key of the running vocabulary argmax
};

// Spin bound: every wave leaves a wait (an exchange poll) after at most this many polls even if
// some workgroup never publishes (then `err` is set and later waits end at once).
#define MQ_SPIN_LIMIT (1u << 23)

