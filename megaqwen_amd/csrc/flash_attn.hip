// flash_attn.hip — unmasked multi-head attention over contiguous [B, H, T, 64] fp16 / bf16
// tensors: out = softmax(scale * q k^T) v per (batch, head).  This is the audio tower's
// self-attention (Qwen3-ASR-0.6B: 14 heads of 64 dims, T ~ 1500 frames), the operation of
// flash_attn_bhwd (megaqwen/triton_flash_attn.py:27-171, kernel body :63-129).
//
// Organisation (gfx950, v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulation):
//   * a workgroup is one (batch*head, 32-query block), XCD-major (see the item mapping in the
//     kernel); its 4 waves split the key tiles (32 keys each) into contiguous ranges and merge their (max, sum, O) partials through LDS at the
//     end, so a 1500-key row costs every wave ~12 tiles instead of 47;
//   * S^T = K Q^T: rows are keys, so each lane holds the scores of ONE query (lanes l and l+32
//     split its 32 keys), and the softmax max / sum need one lane swap;
//   * K tile row r carries key fa_key_perm(r) (bits 2 and 3 of r swapped).  That makes score
//     accumulator element j of lane l the key 16 (j / 8) + 8 (l / 32) + j % 8, which is the
//     B-operand layout of two 16-key MFMA steps: O^T += V^T P^T takes P^T from registers;
//   * K and V^T are first copied (fa_pack_kernel, into the caller's workspace) into per-tile
//     operand order: each 16-byte operand register of a wave is one contiguous 1 KB load.  Read
//     from the [T, 64] rows directly, an operand load touches 16-32 cache lines and the loads
//     bound the kernel;
//   * the scores are exact fp32 dot products of the 16-bit inputs (up to accumulation order),
//     the softmax is fp32, and P enters the MFMA as a hi + lo pair of the input type (two
//     MFMAs), ~16 bits more than one rounding of P; the output is o / l rounded to nearest-even
//     in the input type (triton_flash_attn.py:126-127).
// Keys >= T (the last tile) get score -inf and zero V^T entries (the pack writes zeros for
// them); queries >= T read row T-1 and store nothing.  All loads stay inside the tensors and the
// workspace.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mq_device.h"
#include "mq_flash.h"

#define FA_D 64           // head dim
#define FA_QB 32          // queries per workgroup
#define FA_KT 32          // keys per tile
#define FA_WAVES 4        // waves per workgroup (split of the key tiles)
#define FA_RESCALE 8.0f   // exponent headroom of the lazily raised softmax reference point

typedef float fa_f32x16 __attribute__((ext_vector_type(16)));
typedef float fa_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 fa_bf16x2 __attribute__((ext_vector_type(2)));

template <bool F16> struct FaType;
template <> struct FaType<false> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 scalar;
  static __device__ __forceinline__ fa_f32x16 mfma(v8 a, v8 b, fa_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct FaType<true> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 scalar;
  static __device__ __forceinline__ fa_f32x16 mfma(v8 a, v8 b, fa_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

MQ_DEV int fa_key_perm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

template <bool F16> MQ_DEV uint32_t fa_pack2(float a, float b) {
  if constexpr (F16) {
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) |
           ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
  } else {
    return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  }
}

// Operand copies of one (batch * head, 32-key tile), 4 KB each, in the workspace:
//   K' [bh][tile][s 0..3][lane 0..63] (16 bytes): K[32 t + fa_key_perm(lane % 32)][16 s + 8 (lane / 32) ..+8]
//   V' [bh][tile][2 nt + s][lane] (16 bytes): V[32 t + 16 s + 8 (lane / 32) + e][32 nt + lane % 32], e = 0..7
// Keys >= T are zero in both.
__global__ void __launch_bounds__(256) fa_pack_kernel(const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ v, uint4* kp,
                                                      uint4* vp, int T, int ntiles) {
  __shared__ uint16_t sv[FA_KT][FA_D + 8];
  const int t = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const size_t base = (size_t)bh * T * FA_D;
  const size_t tile = ((size_t)bh * ntiles + t) * 256;
  const int lane = tid & 63, s = tid >> 6;
  {
    const int key = t * FA_KT + fa_key_perm(lane & 31);
    kp[tile + tid] = key < T ? ld16(k + base + (size_t)key * FA_D + 16 * s + 8 * (lane >> 5))
                             : make_uint4(0u, 0u, 0u, 0u);
  }
  {
    const int r = tid >> 3, c = tid & 7, key = t * FA_KT + r;
    const uint4 w = key < T ? ld16(v + base + (size_t)key * FA_D + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(&sv[r][8 * c]) = w;
  }
  __syncthreads();
  {
    const int nt = s >> 1, ss = s & 1, dim = 32 * nt + (lane & 31), k0 = 16 * ss + 8 * (lane >> 5);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)sv[k0 + 2 * e][dim] | ((uint32_t)sv[k0 + 2 * e + 1][dim] << 16);
    vp[tile + tid] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// CPOS: the scale is >= 0 (the softmax max is taken over the raw scores; otherwise their min),
// a compile-time choice so that a tile carries neither the other extreme nor selects between them
template <bool F16, bool CPOS>
__global__ void __launch_bounds__(64 * FA_WAVES) __attribute__((amdgpu_waves_per_eu(3)))
fa_bhwd_kernel(const uint16_t* __restrict__ q, const uint4* __restrict__ kp,
               const uint4* __restrict__ vp, uint16_t* __restrict__ out, int T,
               float scale_log2, int nqb, int items, int per_xcd) {
  typedef FaType<F16> Ty;
  typedef typename Ty::v8 v8;
  // LDS: the workgroup's Q^T operand (shared by its waves, 4 KB) during the key loop; the
  // partials of waves 1.. (o: 32 per lane, m, l) afterwards.
  union FaLds {
    struct {
      uint4 q[4][64];
    } loop;
    float red[FA_WAVES - 1][34][64];
  };
  __shared__ __attribute__((aligned(16))) FaLds lds;

  // Work item = (batch * head, query block), head-major.  Workgroups are dealt to the 8 XCDs
  // round robin (linear id % 8), so XCD x is given the contiguous items [x * per_xcd, ..): the
  // workgroups resident on one XCD share one or two heads' K and V, which its L2 then holds,
  // instead of every XCD streaming every head's K and V from HBM once per query block.
  const int item = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (item >= items) return;                       // grid padding (uniform per workgroup)
  const int bh = item / nqb, qb = item - bh * nqb;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 31, hh = lane >> 5;
  const size_t base = (size_t)bh * T * FA_D;
  const uint16_t* Q = q + base;
  const int qi = qb * FA_QB + fr;                  // this lane's query
  const int ntiles = (T + FA_KT - 1) / FA_KT;
  const int t0 = ntiles * wave / FA_WAVES, t1 = ntiles * (wave + 1) / FA_WAVES;

  // Q^T operand in LDS, read by every wave at every tile (registers are the scarcer resource):
  // lds.loop.q[s][lane] = query q0 + lane % 32 (rows >= T read row T-1, never stored), dims
  // 16 s + 8 (lane / 32) .. + 8; wave w loads step s = w
  {
    const int qrow = min(qb * FA_QB + fr, T - 1);
    lds.loop.q[wave][lane] = ld16(Q + (size_t)qrow * FA_D + 16 * wave + 8 * hh);
  }
  __syncthreads();
  // Operands of the key tiles from the operand copies, loaded ahead of their use (contiguous
  // 1 KB per wave instruction).  The loads are unconditional: a load under a branch makes the
  // compiler wait for every outstanding load at the next use of any of them.
  const uint4* KP = kp + (size_t)bh * ntiles * 256 + lane;
  const uint4* VP = vp + (size_t)bh * ntiles * 256 + lane;
  uint4 kr[4];
  auto load_k = [&](int t) {
#pragma unroll
    for (int s = 0; s < 4; ++s) kr[s] = ld16(KP + (size_t)t * 256 + 64 * s);
  };
  auto load_v = [&](int t, uint4 (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ld16(VP + (size_t)t * 256 + 64 * i);
  };
  // S^T of the tile whose K operand is in kr
  auto scores = [&]() {
    fa_f32x16 acc;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = Ty::mfma(__builtin_bit_cast(v8, kr[s]), __builtin_bit_cast(v8, lds.loop.q[s][lane]), acc);
    return acc;
  };

  fa_f32x16 o[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[nt][j] = 0.f;
  // m: the reference point of the exponentials (log2 units), raised only when a score exceeds
  // it by more than FA_RESCALE (every weight is <= 2^FA_RESCALE, and o, l are rescaled rarely
  // instead of at every new maximum); l: the sum of the weights
  float m = -INFINITY, l = 0.f;
  // max_j (s_j * c) is max_j(s_j) * c for c >= 0 and min_j(s_j) * c for c < 0 (rounding is
  // monotonic), so the extreme is taken over the raw scores

  // Software pipeline: the MFMAs of tile t + 1's scores are issued before tile t's softmax, so
  // they run while the softmax's VALU work issues, and the next tiles' operands are loaded a full
  // step before their use.  The last iteration recomputes its own tile's scores (unused) rather
  // than branch.
  // vcur: this tile's V^T operands; vnext receives the next tile's (the two register sets
  // alternate with the unrolled steps, so no operand is copied)
  auto step = [&](int t, fa_f32x16& sv, fa_f32x16& snext, const uint4 (&vcur)[4],
                  uint4 (&vnext)[4]) {
    snext = scores();
    // keys >= T exist only in the row's last tile
    const bool masked = t == ntiles - 1 && T % FA_KT != 0;
    load_k(min(t + 2, t1 - 1));
    load_v(min(t + 1, t1 - 1), vnext);
    if (__builtin_expect(masked, false)) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (t * FA_KT + 16 * (j >> 3) + 8 * hh + (j & 7) >= T) sv[j] = CPOS ? -INFINITY : INFINITY;
    }
    float mr;
    if constexpr (CPOS) {
      mr = fmaxf(sv[0], sv[1]);
#pragma unroll
      for (int j = 2; j < 16; j += 2) mr = fmaxf(mr, fmaxf(sv[j], sv[j + 1]));
      mr = max_xor32(mr);
    } else {
      mr = fminf(sv[0], sv[1]);
#pragma unroll
      for (int j = 2; j < 16; j += 2) mr = fminf(mr, fminf(sv[j], sv[j + 1]));
      const float2 pr = swap32(mr);
      mr = fminf(pr.x, pr.y);
    }
    const float mt = mr * scale_log2;
    float alpha = 1.0f;
    if (mt > m + FA_RESCALE) {
      alpha = __builtin_amdgcn_exp2f(m - mt);
      m = mt;
    }
    // sv becomes the exponent s * c - m of each weight
#pragma unroll
    for (int j = 0; j < 16; ++j) sv[j] = fmaf(sv[j], scale_log2, -m);
    if (__builtin_expect(masked, false)) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (t * FA_KT + 16 * (j >> 3) + 8 * hh + (j & 7) >= T) sv[j] = -INFINITY;
    }
    // weights, and P as hi + lo 16-bit parts: hi truncates (bf16: the upper half of the fp32
    // word; fp16: round toward zero), lo is the exact fp32 remainder rounded once
    float ls = 0.f;
    uint32_t phw[8], plw[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const float p0 = __builtin_amdgcn_exp2f(sv[2 * w]);
      const float p1 = __builtin_amdgcn_exp2f(sv[2 * w + 1]);
      ls += p0 + p1;
      if constexpr (F16) {
        const auto hw = __builtin_amdgcn_cvt_pkrtz(p0, p1);
        const auto lw = __builtin_amdgcn_cvt_pkrtz(p0 - (float)hw[0], p1 - (float)hw[1]);
        phw[w] = __builtin_bit_cast(uint32_t, hw);
        plw[w] = __builtin_bit_cast(uint32_t, lw);
      } else {
        const float h0 = __uint_as_float(__float_as_uint(p0) & 0xffff0000u);
        const float h1 = __uint_as_float(__float_as_uint(p1) & 0xffff0000u);
        phw[w] = __builtin_amdgcn_perm(__float_as_uint(p1), __float_as_uint(p0), 0x07060302u);
        const fa_f32x2 lo = {p0 - h0, p1 - h1};
        plw[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, fa_bf16x2));
      }
    }
    l = l * alpha + ls;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[nt][j] *= alpha;
    }
    // O^T += V^T P^T; V^T operand (nt, s): dim 32 nt + fr, keys 16 s + 8 hh .. + 8
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const v8 ph = __builtin_bit_cast(v8, make_uint4(phw[4 * s], phw[4 * s + 1], phw[4 * s + 2], phw[4 * s + 3]));
      const v8 pl = __builtin_bit_cast(v8, make_uint4(plw[4 * s], plw[4 * s + 1], plw[4 * s + 2], plw[4 * s + 3]));
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const v8 vb = __builtin_bit_cast(v8, vcur[2 * nt + s]);
        o[nt] = Ty::mfma(vb, ph, o[nt]);
        o[nt] = Ty::mfma(vb, pl, o[nt]);
      }
    }
  };
  if (t0 < t1) {
    uint4 va[4], vb[4];
    load_k(t0);
    load_v(t0, va);
    fa_f32x16 sa = scores(), sb;
    load_k(min(t0 + 1, t1 - 1));
    // unrolled by two so that the two score buffers and the two V^T sets alternate without copies
    for (int t = t0; t < t1; t += 2) {
      step(t, sa, sb, va, vb);
      if (t + 1 < t1) step(t + 1, sb, sa, vb, va);
    }
  }

  // merge the key ranges in wave order (a wave without tiles has m = -inf and adds 0; at least
  // one wave has a tile, so the common max is finite)
  __syncthreads();                                 // every wave is done with the Q^T operand
  if (wave > 0) {
    float* r = &lds.red[wave - 1][0][lane];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) r[(16 * nt + j) * 64] = o[nt][j];
    r[32 * 64] = m;
    r[33 * 64] = l;
  }
  __syncthreads();
  if (wave > 0) return;
  float mt = m;
#pragma unroll
  for (int w = 1; w < FA_WAVES; ++w) mt = fmaxf(mt, lds.red[w - 1][32][lane]);
  {
    const float a = __builtin_amdgcn_exp2f(m - mt);
    l *= a;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[nt][j] *= a;
  }
#pragma unroll
  for (int w = 1; w < FA_WAVES; ++w) {
    const float a = __builtin_amdgcn_exp2f(lds.red[w - 1][32][lane] - mt);
    l = fmaf(lds.red[w - 1][33][lane], a, l);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[nt][j] = fmaf(lds.red[w - 1][16 * nt + j][lane], a, o[nt][j]);
  }
  l = sum_xor32(l);                                // lanes l, l+32 summed different keys
  if (qi < T) {
    uint16_t* dst = out + base + (size_t)qi * FA_D;
    // O^T accumulator element j of tile nt: dim 32 nt + 8 (j / 4) + 4 hh + j % 4
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        uint2 w;
        w.x = fa_pack2<F16>(o[nt][4 * jg] / l, o[nt][4 * jg + 1] / l);
        w.y = fa_pack2<F16>(o[nt][4 * jg + 2] / l, o[nt][4 * jg + 3] / l);
        *reinterpret_cast<uint2*>(dst + 32 * nt + 8 * jg + 4 * hh) = w;
      }
  }
}

size_t mq_flash_attn_workspace(int bh, int T) {
  return (size_t)2 * bh * ((T + FA_KT - 1) / FA_KT) * FA_KT * FA_D * 2;
}

int mq_launch_flash_attn_bhwd(const void* q, const void* k, const void* v, void* out, int bh,
                              int T, bool f16, float scale_log2, void* workspace,
                              hipStream_t stream) {
  const int nqb = (T + FA_QB - 1) / FA_QB, ntiles = (T + FA_KT - 1) / FA_KT;
  const long long items = (long long)nqb * bh, per = (items + 7) / 8;
  if (8 * per > 0x7fffffffLL) return -1;
  const uint16_t* qq = static_cast<const uint16_t*>(q);
  const uint16_t* kk = static_cast<const uint16_t*>(k);
  const uint16_t* vv = static_cast<const uint16_t*>(v);
  uint4* kp = static_cast<uint4*>(workspace);
  uint4* vp = kp + (size_t)bh * ntiles * 256;
  uint16_t* oo = static_cast<uint16_t*>(out);
  hipLaunchKernelGGL(fa_pack_kernel, dim3(ntiles, bh), dim3(256), 0, stream, kk, vv, kp, vp, T,
                     ntiles);
  const dim3 grid((unsigned)(8 * per)), block(64 * FA_WAVES);
  const bool cpos = scale_log2 >= 0.f;
  if (f16 && cpos)
    hipLaunchKernelGGL((fa_bhwd_kernel<true, true>), grid, block, 0, stream, qq, kp, vp, oo, T,
                       scale_log2, nqb, (int)items, (int)per);
  else if (f16)
    hipLaunchKernelGGL((fa_bhwd_kernel<true, false>), grid, block, 0, stream, qq, kp, vp, oo, T,
                       scale_log2, nqb, (int)items, (int)per);
  else if (cpos)
    hipLaunchKernelGGL((fa_bhwd_kernel<false, true>), grid, block, 0, stream, qq, kp, vp, oo, T,
                       scale_log2, nqb, (int)items, (int)per);
  else
    hipLaunchKernelGGL((fa_bhwd_kernel<false, false>), grid, block, 0, stream, qq, kp, vp, oo, T,
                       scale_log2, nqb, (int)items, (int)per);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
