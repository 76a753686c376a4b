// Prefill of n tokens at positions 0..n-1 on gfx950 (launch_prefill_float,
// csrc/megakernel/fused_prefill_launch.inl:71-731, with the kernels of fused_prefill_kernels.inl).
//
// The reference keeps bf16 intermediates and rounds after every GEMM and elementwise op; so does
// this path.  Per layer:
//   xn  = bf16(RMSNorm(h) * w_in)                                   row kernel
//   qkv = bf16(xn Wq|Wk|Wv^T)                                       MFMA GEMM  (n x 4096 x 1024)
//   q,k = bf16(RoPE(RMSNorm_head(.) * w)); k, v -> KV cache rows    head kernel
//   att = bf16(causal GQA softmax(q k^T / sqrt(128)) v)             MFMA flash attention
//   h   = bf16(bf16(att Wo^T) + h)                                  MFMA GEMM + residual epilogue
//   xn  = bf16(RMSNorm(h) * w_post)
//   m   = bf16(silu(bf16(xn Wg^T)) * bf16(xn Wu^T))                 dual MFMA GEMM + SwiGLU
//   h   = bf16(bf16(m Wd^T) + h)                                    MFMA GEMM + residual epilogue
// then the last row's final norm (bf16) and the LM-head argmax (fused_prefill_kernels.inl:655-824).
//
// GEMMs are C[M,N] = A[M,K] B[N,K]^T ("NT": activations and weights both K-contiguous) on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation: 64x64 workgroup tiles, 4 waves of 32x32,
// K staged through double-buffered LDS in steps of 32.  Consecutive workgroups walk N first, so
// with N/64 a multiple of 8 all M tiles of one weight tile land on one XCD and share its L2.
#include "mq_prefill.h"

#include <math.h>

typedef __bf16 mq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mq_f32x16 __attribute__((ext_vector_type(16)));

MQ_DEV mq_bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(mq_bf16x8, v); }
MQ_DEV float silu_f(float x) { return x / (1.0f + expf(-x)); }

// ------------------------------------------------------------------------- row kernels
__global__ void __launch_bounds__(128) pf_embed_kernel(const bf16_t* __restrict__ embed,
                                                       const int32_t* __restrict__ tokens,
                                                       bf16_t* __restrict__ h) {
  const int row = blockIdx.x;
  const int tok = tokens[row];
  reinterpret_cast<uint4*>(h + (size_t)row * MQ_H)[threadIdx.x] =
      reinterpret_cast<const uint4*>(embed + (size_t)tok * MQ_H)[threadIdx.x];
}

// y = bf16(x * rsqrt(mean(x^2) + eps) * w) for one 1024-wide row per workgroup
// (prefill_rmsnorm_kernel, fused_prefill_kernels.inl:52-105).
__global__ void __launch_bounds__(128) pf_rmsnorm_kernel(const bf16_t* __restrict__ x,
                                                         const bf16_t* __restrict__ w,
                                                         bf16_t* __restrict__ y) {
  __shared__ float red[2];
  const int row = blockIdx.x, t = threadIdx.x;
  const uint4 xv = reinterpret_cast<const uint4*>(x + (size_t)row * MQ_H)[t];
  float v[8];
  unpack8(xv, v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((red[0] + red[1]) * (1.0f / MQ_H) + MQ_EPS);
  float wv[8];
  unpack8(reinterpret_cast<const uint4*>(w)[t], wv);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (uint32_t)f32_to_bf16(v[2 * e] * r * wv[2 * e]) |
           ((uint32_t)f32_to_bf16(v[2 * e + 1] * r * wv[2 * e + 1]) << 16);
  reinterpret_cast<uint4*>(y + (size_t)row * MQ_H)[t] = make_uint4(o[0], o[1], o[2], o[3]);
}

// Per-(position, head) q/k RMSNorm + rotate-half RoPE, rounded to bf16 in place; k and v rows go
// to the KV cache of `layer` (prefill_qk_norm_rope_kernel, fused_prefill_kernels.inl:112-258).
// One wave per (position, head); heads 0..15 are q, 16..23 are k (with v).
__global__ void __launch_bounds__(64) pf_qk_norm_rope_kernel(MqDecodeParams p, int layer,
                                                             bf16_t* __restrict__ qkv) {
  const int pos = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  const MqLayerW w = p.layers[layer];
  const bf16_t* cs = p.cos + (size_t)pos * MQ_D;
  const bf16_t* sn = p.sin + (size_t)pos * MQ_D;
  bf16_t* row = qkv + (size_t)pos * MQ_QKV;
  const bool is_q = head < MQ_NQ;
  const int h = is_q ? head : head - MQ_NQ;
  bf16_t* x = row + (is_q ? h * MQ_D : MQ_QDIM + h * MQ_D);
  float lo = bf16_to_f32(x[lane]), hi = bf16_to_f32(x[lane + 64]);
  const bf16_t* nw = is_q ? w.q_norm : w.k_norm;
  const float ss = wave_sum(lo * lo + hi * hi);
  const float r = rsqrtf(ss * (1.0f / MQ_D) + MQ_EPS);
  const float a = lo * r * bf16_to_f32(nw[lane]);
  const float b = hi * r * bf16_to_f32(nw[lane + 64]);
  const bf16_t olo = f32_to_bf16(a * bf16_to_f32(cs[lane]) - b * bf16_to_f32(sn[lane]));
  const bf16_t ohi = f32_to_bf16(a * bf16_to_f32(sn[lane + 64]) + b * bf16_to_f32(cs[lane + 64]));
  x[lane] = olo;
  x[lane + 64] = ohi;
  if (!is_q) {
    const size_t crow = (((size_t)layer * MQ_NKV + h) * p.max_seq + pos) * MQ_D;
    p.kc[crow + lane] = olo;
    p.kc[crow + lane + 64] = ohi;
    const bf16_t* v = row + MQ_QDIM + MQ_KVDIM + h * MQ_D;
    p.vc[crow + lane] = v[lane];
    p.vc[crow + lane + 64] = v[lane + 64];
  }
}

// ------------------------------------------------------------------------------ GEMM
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

struct GemmArgs {
  const bf16_t* A;   // [M, K]
  int lda;
  const bf16_t* B0;  // rows [0, n0) of B (weights [rows, K])
  const bf16_t* B1;  // rows [n0, n1)
  const bf16_t* B2;  // rows [n1, N)
  int n0, n1;
  const bf16_t* Bu;  // EPI_SWIGLU: the up-projection weights (same shape as B0)
  bf16_t* C;         // [M, N]
  int ldc;
  const bf16_t* R;   // EPI_RESID: residual [M, N] (may alias C)
  int ldr;
  int M, N, K;
};

#define GEMM_BM 64
#define GEMM_BN 64
#define GEMM_BK 32
#define GEMM_LDS_STRIDE 40   // bf16 per LDS row: 32 + 8 padding

template <int EPI>
__global__ void __launch_bounds__(256) pf_gemm_kernel(GemmArgs g) {
  constexpr int NB = EPI == EPI_SWIGLU ? 2 : 1;
  __shared__ __align__(16) bf16_t As[2][GEMM_BM * GEMM_LDS_STRIDE];
  __shared__ __align__(16) bf16_t Bs[2][NB][GEMM_BN * GEMM_LDS_STRIDE];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n_base = blockIdx.x * GEMM_BN, m_base = blockIdx.y * GEMM_BM;
  const bf16_t* B;
  if (n_base < g.n0) B = g.B0 + (size_t)n_base * g.K;
  else if (n_base < g.n1) B = g.B1 + (size_t)(n_base - g.n0) * g.K;
  else B = g.B2 + (size_t)(n_base - g.n1) * g.K;
  const bf16_t* Bu = (EPI == EPI_SWIGLU) ? g.Bu + (size_t)n_base * g.K : nullptr;

  // global -> register staging: thread t moves 16 bytes of row t/4, k offset (t%4)*8
  const int lr = t >> 2, lk = (t & 3) * 8;
  const int am = m_base + lr;
  const bool a_ok = am < g.M;
  const bf16_t* a_src = g.A + (size_t)(a_ok ? am : g.M - 1) * g.lda + lk;
  const bf16_t* b_src = B + (size_t)lr * g.K + lk;
  const bf16_t* u_src = (EPI == EPI_SWIGLU) ? Bu + (size_t)lr * g.K + lk : nullptr;

  uint4 ra = a_ok ? ld16(a_src) : make_uint4(0, 0, 0, 0);
  uint4 rb[NB];
  rb[0] = ld_nt16(b_src);
  if (NB == 2) rb[NB - 1] = ld_nt16(u_src);
  *reinterpret_cast<uint4*>(&As[0][lr * GEMM_LDS_STRIDE + lk]) = ra;
#pragma unroll
  for (int b = 0; b < NB; ++b) *reinterpret_cast<uint4*>(&Bs[0][b][lr * GEMM_LDS_STRIDE + lk]) = rb[b];
  __syncthreads();

  mq_f32x16 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[b][j] = 0.f;

  const int fr = lane & 31, fk = (lane >> 5) * 8;   // MFMA operand row and k offset of a lane
  int cur = 0;
  for (int k0 = 0; k0 < g.K; k0 += GEMM_BK) {
    const bool more = k0 + GEMM_BK < g.K;
    if (more) {
      ra = a_ok ? ld16(a_src + k0 + GEMM_BK) : make_uint4(0, 0, 0, 0);
      rb[0] = ld_nt16(b_src + k0 + GEMM_BK);
      if (NB == 2) rb[NB - 1] = ld_nt16(u_src + k0 + GEMM_BK);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const mq_bf16x8 af = as_bf16x8(
          *reinterpret_cast<const uint4*>(&As[cur][(wm * 32 + fr) * GEMM_LDS_STRIDE + 16 * s + fk]));
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const mq_bf16x8 bf = as_bf16x8(*reinterpret_cast<const uint4*>(
            &Bs[cur][b][(wn * 32 + fr) * GEMM_LDS_STRIDE + 16 * s + fk]));
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc[b], 0, 0, 0);
      }
    }
    if (more) {
      *reinterpret_cast<uint4*>(&As[cur ^ 1][lr * GEMM_LDS_STRIDE + lk]) = ra;
#pragma unroll
      for (int b = 0; b < NB; ++b)
        *reinterpret_cast<uint4*>(&Bs[cur ^ 1][b][lr * GEMM_LDS_STRIDE + lk]) = rb[b];
    }
    __syncthreads();
    cur ^= 1;
  }

  // epilogue: acc[j] is C[row][col] with row = 8*(j/4) + 4*(lane/32) + j%4, col = lane%32
  const int col = n_base + wn * 32 + (lane & 31);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int row = m_base + wm * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
    if (row < g.M) {
      float v;
      if (EPI == EPI_STORE) {
        v = acc[0][j];
      } else if (EPI == EPI_RESID) {
        v = round_bf16(acc[0][j]) + bf16_to_f32(g.R[(size_t)row * g.ldr + col]);
      } else {
        const float gv = round_bf16(acc[0][j]), uv = round_bf16(acc[NB - 1][j]);
        v = silu_f(gv) * uv;
      }
      g.C[(size_t)row * g.ldc + col] = f32_to_bf16(v);
    }
  }
}

// --------------------------------------------------------------------- causal attention
// Flash-style causal GQA attention of one kv head over 32 query positions per workgroup
// (2 waves: query heads 2h and 2h+1 share every K/V tile).  Per 32-key tile: S = Q K^T with
// v_mfma_f32_32x32x16_bf16 (q and k are bf16, so the fp32 scores are exact up to accumulation
// order), online softmax in fp32 on the accumulator layout, then O += P V where P is split into
// bf16 hi + lo parts (two MFMAs) so the weights keep ~16 bits more than bf16, close to the
// reference's fp32 softmax (prefill_causal_attention_kernel, fused_prefill_kernels.inl:265-342).
#define ATT_KT 32
#define ATT_KSTR 136     // K tile row stride (bf16): 128 + 8
#define ATT_VSTR 40      // transposed V tile row stride (bf16): 32 + 8
#define ATT_PSTR 36      // P tile row stride (fp32): 32 + 4

__global__ void __launch_bounds__(128) pf_attn_kernel(MqDecodeParams p, int layer,
                                                      const bf16_t* __restrict__ qkv,
                                                      bf16_t* __restrict__ att, int n) {
  __shared__ __align__(16) bf16_t Ks[ATT_KT * ATT_KSTR];
  __shared__ __align__(16) bf16_t Vt[MQ_D * ATT_VSTR];
  __shared__ __align__(16) float Ps[2][32 * ATT_PSTR];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = blockIdx.y, qh = 2 * h + wave;
  const int q0 = blockIdx.x * 32;
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  const bf16_t* Kc = p.kc + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D;
  const bf16_t* Vc = p.vc + ((size_t)layer * MQ_NKV + h) * p.max_seq * MQ_D;

  // Q fragments: query row q0 + lane%32, dims 16s + 8*(lane/32) .. +8
  mq_bf16x8 qf[8];
  {
    const int qr = q0 + fr;
    const bf16_t* src = qkv + (size_t)(qr < n ? qr : n - 1) * MQ_QKV + qh * MQ_D + fk;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = as_bf16x8(qr < n ? ld16(src + 16 * s) : make_uint4(0, 0, 0, 0));
  }
  mq_f32x16 o[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[nt][j] = 0.f;
  float m[16], l[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
  }
  const float scale = p.scale_log2;
  const int q_last = min(n, q0 + 32) - 1;
  float* P = Ps[wave];
  for (int k0 = 0; k0 <= q_last; k0 += ATT_KT) {
    // K tile row-major, V tile transposed (dim-major) into LDS; 128 threads x 4 x 16 bytes each
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = t + 128 * i;          // 0..255: key idx/8, dim chunk (idx%8)*16 ... as 16B units
      const int key = idx >> 3, dc = (idx & 7) * 16;
      const int kk = k0 + key;
      const bool ok = kk < n;
      uint4 kv0 = ok ? ld16(Kc + (size_t)kk * MQ_D + dc) : make_uint4(0, 0, 0, 0);
      uint4 kv1 = ok ? ld16(Kc + (size_t)kk * MQ_D + dc + 8) : make_uint4(0, 0, 0, 0);
      uint4 vv0 = ok ? ld16(Vc + (size_t)kk * MQ_D + dc) : make_uint4(0, 0, 0, 0);
      uint4 vv1 = ok ? ld16(Vc + (size_t)kk * MQ_D + dc + 8) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&Ks[key * ATT_KSTR + dc]) = kv0;
      *reinterpret_cast<uint4*>(&Ks[key * ATT_KSTR + dc + 8]) = kv1;
      const uint32_t vw[8] = {vv0.x, vv0.y, vv0.z, vv0.w, vv1.x, vv1.y, vv1.z, vv1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Vt[(dc + 2 * e) * ATT_VSTR + key] = (bf16_t)(vw[e] & 0xffffu);
        Vt[(dc + 2 * e + 1) * ATT_VSTR + key] = (bf16_t)(vw[e] >> 16);
      }
    }
    __syncthreads();
    // S = Q K^T  (rows: queries, cols: keys)
    mq_f32x16 sacc;
#pragma unroll
    for (int j = 0; j < 16; ++j) sacc[j] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const mq_bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(&Ks[fr * ATT_KSTR + 16 * s + fk]));
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[s], kf, sacc, 0, 0, 0);
    }
    // mask, online softmax (row j of this lane: query q0 + rowj, key k0 + lane%32)
    const int key = k0 + fr;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int qrow = q0 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
      float sv = (key <= qrow && key < n) ? sacc[j] * scale : -INFINITY;
      float mx = row16_max(sv);
      mx = fmaxf(mx, xor_lane(mx, 16));
      const float m_new = fmaxf(m[j], mx);
      const float alpha = exp2f(m[j] - m_new);
      const float pv = exp2f(sv - m_new);
      float ps = row16_sum(pv);
      ps += xor_lane(ps, 16);
      l[j] = l[j] * alpha + ps;
      m[j] = m_new;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) o[nt][j] *= alpha;
      P[(8 * (j >> 2) + 4 * (lane >> 5) + (j & 3)) * ATT_PSTR + fr] = pv;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // O += P V with P = hi + lo (bf16 each)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float pr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pr[e] = P[fr * ATT_PSTR + 16 * s + fk + e];
      mq_bf16x8 phi, plo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const __bf16 hb = (__bf16)pr[e];
        phi[e] = hb;
        plo[e] = (__bf16)(pr[e] - (float)hb);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const mq_bf16x8 vf = as_bf16x8(
            *reinterpret_cast<const uint4*>(&Vt[(nt * 32 + fr) * ATT_VSTR + 16 * s + fk]));
        o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(phi, vf, o[nt], 0, 0, 0);
        o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(plo, vf, o[nt], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // normalise and store bf16: O[row][dim] with dim = 32*nt + lane%32
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int qrow = q0 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
    if (qrow < n) {
      const float inv = 1.0f / l[j];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        att[(size_t)qrow * MQ_QDIM + qh * MQ_D + nt * 32 + fr] = f32_to_bf16(o[nt][j] * inv);
    }
  }
}

// -------------------------------------------------------------------------- host side
static size_t pf_align(size_t v) { return (v + 255) / 256 * 256; }

size_t mq_prefill_workspace_bytes(int max_n) {
  if (max_n <= 0) return 0;
  const size_t n = (size_t)max_n;
  return pf_align(n * MQ_H * 2) * 2 + pf_align(n * MQ_QKV * 2) + pf_align(n * MQ_QDIM * 2) +
         pf_align(n * MQ_I * 2);
}

void mq_prefill_bind(MqPrefillBuffers* b, char* base, int max_n) {
  b->max_n = max_n;
  if (max_n <= 0) {
    b->h = b->xn = b->qkv = b->att = b->m = nullptr;
    return;
  }
  const size_t n = (size_t)max_n;
  char* c = base;
  b->h = reinterpret_cast<bf16_t*>(c);   c += pf_align(n * MQ_H * 2);
  b->xn = reinterpret_cast<bf16_t*>(c);  c += pf_align(n * MQ_H * 2);
  b->qkv = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QKV * 2);
  b->att = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QDIM * 2);
  b->m = reinterpret_cast<bf16_t*>(c);
}

template <int EPI>
static void gemm(const GemmArgs& g, hipStream_t s) {
  dim3 grid(g.N / GEMM_BN, (g.M + GEMM_BM - 1) / GEMM_BM);
  pf_gemm_kernel<EPI><<<grid, 256, 0, s>>>(g);
}

int mq_launch_prefill(const MqDecodeParams& p, const MqLayerW* hl, const MqPrefillBuffers& b,
                      const int32_t* tokens, int n, int32_t* tok_out, float* logits, int grid,
                      hipStream_t stream) {
  if (n <= 0 || n > b.max_n || n > p.max_seq) return -3;
  pf_embed_kernel<<<n, 128, 0, stream>>>(p.embed, tokens, b.h);
  for (int l = 0; l < p.num_layers; ++l) {
    const MqLayerW& w = hl[l];
    pf_rmsnorm_kernel<<<n, 128, 0, stream>>>(b.h, w.in_ln, b.xn);
    GemmArgs g{};
    g.A = b.xn; g.lda = MQ_H;
    g.B0 = w.wq; g.B1 = w.wk; g.B2 = w.wv; g.n0 = MQ_QDIM; g.n1 = MQ_QDIM + MQ_KVDIM;
    g.C = b.qkv; g.ldc = MQ_QKV; g.M = n; g.N = MQ_QKV; g.K = MQ_H;
    gemm<EPI_STORE>(g, stream);
    pf_qk_norm_rope_kernel<<<dim3(n, MQ_NQ + MQ_NKV), 64, 0, stream>>>(p, l, b.qkv);
    pf_attn_kernel<<<dim3((n + 31) / 32, MQ_NKV), 128, 0, stream>>>(p, l, b.qkv, b.att, n);
    g = GemmArgs{};
    g.A = b.att; g.lda = MQ_QDIM;
    g.B0 = g.B1 = g.B2 = w.wo; g.n0 = g.n1 = MQ_H;
    g.C = b.h; g.ldc = MQ_H; g.R = b.h; g.ldr = MQ_H; g.M = n; g.N = MQ_H; g.K = MQ_QDIM;
    gemm<EPI_RESID>(g, stream);
    pf_rmsnorm_kernel<<<n, 128, 0, stream>>>(b.h, w.post_ln, b.xn);
    g = GemmArgs{};
    g.A = b.xn; g.lda = MQ_H;
    g.B0 = g.B1 = g.B2 = w.wg; g.n0 = g.n1 = MQ_I; g.Bu = w.wu;
    g.C = b.m; g.ldc = MQ_I; g.M = n; g.N = MQ_I; g.K = MQ_H;
    gemm<EPI_SWIGLU>(g, stream);
    g = GemmArgs{};
    g.A = b.m; g.lda = MQ_I;
    g.B0 = g.B1 = g.B2 = w.wd; g.n0 = g.n1 = MQ_H;
    g.C = b.h; g.ldc = MQ_H; g.R = b.h; g.ldr = MQ_H; g.M = n; g.N = MQ_H; g.K = MQ_I;
    gemm<EPI_RESID>(g, stream);
  }
  // last row: final norm rounded to bf16, LM head argmax (fused_prefill_kernels.inl:655-824)
  return mq_launch_lm_head_bf16norm(p, b.h + (size_t)(n - 1) * MQ_H, tok_out, logits, grid,
                                    stream);
}
