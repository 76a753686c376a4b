// Prefill of n tokens at positions 0..n-1 on gfx950 (launch_prefill_float,
// csrc/megakernel/fused_prefill_launch.inl:71-731, with the kernels of fused_prefill_kernels.inl).
//
// The reference keeps bf16 intermediates and rounds after every GEMM and elementwise op; so does
// this path.  Per layer:
//   xn  = bf16(RMSNorm(h) * w_in)                                   row kernel
//   qkv = bf16(xn Wq|Wk|Wv^T)                                       MFMA GEMM  (n x 4096 x 1024)
//   q,k = bf16(RoPE(RMSNorm_head(.) * w)); k, v -> KV cache rows    the same GEMM's epilogue
//   att = bf16(causal GQA softmax(q k^T / sqrt(128)) v)             MFMA flash attention
//   h   = bf16(bf16(att Wo^T) + h)                                  MFMA GEMM + residual epilogue
//   xn  = bf16(RMSNorm(h) * w_post)
//   m   = bf16(silu(bf16(xn Wg^T)) * bf16(xn Wu^T))                 dual MFMA GEMM + SwiGLU
//   h   = bf16(bf16(m Wd^T) + h)                                    MFMA GEMM + residual epilogue
// then the last row's final norm (bf16) and the LM-head argmax (fused_prefill_kernels.inl:655-824).
//
// GEMMs are C[M,N] = A[M,K] B[N,K]^T ("NT": activations and weights both K-contiguous) on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation: 128x128, 128x64, 64x64 or 32x64 workgroup
// tiles (by M and N), K staged through double-buffered LDS in steps of 64 (128 for 32-row tiles), fed by a
// register ring of global loads.  Consecutive workgroups walk N first, so with N/BN a multiple
// of 8 all M tiles of one weight tile land on one XCD and share its L2.
#include "mq_prefill.h"

#include <math.h>

#include <type_traits>

typedef __bf16 mq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mq_f32x16 __attribute__((ext_vector_type(16)));

MQ_DEV mq_bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(mq_bf16x8, v); }
MQ_DEV float silu_f(float x) { return x / (1.0f + expf(-x)); }
typedef float mq_pf_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 mq_pf_bf16x2 __attribute__((ext_vector_type(2)));
// Two values rounded to bf16 (nearest even) by one v_cvt_pk_bf16_f32; a in the low half.
MQ_DEV uint32_t pack_bf16x2(float a, float b) {
  const mq_pf_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, mq_pf_bf16x2));
}

// ------------------------------------------------------------ attention operand layouts
// The causal attention reads K and V^T as MFMA operands, 16 bytes per lane.  Both are kept, per
// kv head and 32-key tile, in the exact order the operand registers take them, so every operand
// load of the attention is one contiguous 1 KB wave load (the KV cache rows stay [pos][128] for
// decode; these are prefill-only copies).
//   K  (A operand of S^T = K Q^T):   [h][tile][s 0..7][lane][8];  lane = row + 32 hh holds key
//       32 tile + att_key_perm(row), dims 16 s + 8 hh .. + 8
//   V^T (A operand of O^T += V^T P^T): [h][tile][nt 0..3][s 0..1][lane][8];  lane = c + 32 hh
//       holds dim 32 nt + c, keys 32 tile + 16 s + 8 hh .. + 8
// att_key_perm swaps bits 2 and 3 of a tile row (an involution); the reason is given at the
// attention kernel.
MQ_DEV int att_key_perm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
MQ_DEV size_t kt_index(int h, int ntiles, int key, int d) {
  const int t = key >> 5, row = att_key_perm(key & 31), s = d >> 4, hh = (d >> 3) & 1;
  return ((((size_t)h * ntiles + t) * 8 + s) * 64 + row + 32 * hh) * 8 + (d & 7);
}
MQ_DEV size_t vt_index(int h, int ntiles, int key, int d) {
  const int t = key >> 5, kk = key & 31, s = kk >> 4, hh = (kk >> 3) & 1, nt = d >> 5;
  return (((((size_t)h * ntiles + t) * 4 + nt) * 2 + s) * 64 + (d & 31) + 32 * hh) * 8 + (kk & 7);
}

// ------------------------------------------------------------------------- row kernels
// Embedding gather (prefill_embed_kernel, fused_prefill_kernels.inl:3-20); rows
// [patch_start, patch_start + patch_len) take the caller's bf16 rows instead (the audio span of
// prefill_patch_audio_kernel, fused_prefill_kernels.inl:28-45, fused into the gather).
// A token id outside [0, vocab) reads row 0 instead and sets the error flag to 2 (as the decode
// kernels do for their input token), so a bad id never reads outside the embedding table.
__global__ void __launch_bounds__(128) pf_embed_kernel(const bf16_t* __restrict__ embed,
                                                       const int32_t* __restrict__ tokens,
                                                       bf16_t* __restrict__ h,
                                                       const bf16_t* __restrict__ patch,
                                                       int patch_start, int patch_len, int vocab,
                                                       uint32_t* err) {
  const int row = blockIdx.x;
  const int pr = row - patch_start;
  const bool patched = pr >= 0 && pr < patch_len;
  int tok = patched ? 0 : tokens[row];
  if (tok < 0 || tok >= vocab) {
    if (threadIdx.x == 0)
      __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tok = 0;
  }
  const bf16_t* src = patched ? patch + (size_t)pr * MQ_H : embed + (size_t)tok * MQ_H;
  reinterpret_cast<uint4*>(h + (size_t)row * MQ_H)[threadIdx.x] =
      reinterpret_cast<const uint4*>(src)[threadIdx.x];
}

// y = bf16(x * rsqrt(mean(x^2) + eps) * w) for one 1024-wide row per workgroup
// (prefill_rmsnorm_kernel, fused_prefill_kernels.inl:52-105).
__global__ void __launch_bounds__(128) pf_rmsnorm_kernel(const bf16_t* __restrict__ x,
                                                         const bf16_t* __restrict__ w,
                                                         bf16_t* __restrict__ y) {
  __shared__ float red[2];
  const int row = blockIdx.x, t = threadIdx.x;
  const uint4 xv = reinterpret_cast<const uint4*>(x + (size_t)row * MQ_H)[t];
  const uint4 wq = reinterpret_cast<const uint4*>(w)[t];   // loaded with x: one round trip
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
  unpack8(wq, wv);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (uint32_t)f32_to_bf16(v[2 * e] * r * wv[2 * e]) |
           ((uint32_t)f32_to_bf16(v[2 * e + 1] * r * wv[2 * e + 1]) << 16);
  reinterpret_cast<uint4*>(y + (size_t)row * MQ_H)[t] = make_uint4(o[0], o[1], o[2], o[3]);
}

// ------------------------------------------------------------------------------ GEMM
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3 };

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
  bf16_t* Vt;        // EPI_STORE / QKV: columns [n1, N) (V) also stored as V^T operand tiles
  int vt_tiles;      // 32-row tiles per kv head in Vt (and Kt)
  // EPI_QKV (the q|k|v projection, N = 4096, one 128-column head per tile; rows are positions
  // 0 .. M - 1): q/k heads get their RMSNorm (qn / kn weights) and RoPE (cs / sn tables) in the
  // epilogue, k heads also go to the K cache (kcl, this layer's [8][max_seq][128]) and the K
  // operand tiles (Kt, kt_index); v heads also go to the V cache (vcl)
  const bf16_t* qn;
  const bf16_t* kn;
  const bf16_t* cs;
  const bf16_t* sn;
  bf16_t* kcl;
  bf16_t* vcl;
  bf16_t* Kt;
  int max_seq;
  int M, N, K;
  // split-K (gridDim.z = sk > 1): every split writes its fp32 partial tile to `part` with
  // device-coherent stores; the last split of a tile to arrive (counter `cnt[tile]`, reset by
  // it to 0) sums the sk partials in split order and runs the epilogue, so the result does not
  // depend on which split finishes last
  int sk;
  float* part;       // [tiles][sk][elements per thread][threads]
  uint32_t* cnt;     // [tiles], 0 between uses
};

#define GEMM_BK 64           // K per step of 64- and 128-row tiles (32-row tiles: 128)
#define GEMM_STAGES 4        // K steps whose global loads are in flight in registers (64-row and
                             // 32-row tiles)
#define GEMM_STAGES_BIG 4    // the same for 128-row tiles (172-177 VGPRs: still two waves per
                             // SIMD); 2 stages measured ~1% slower per 4096-token prefill
static_assert(512 / GEMM_BK % GEMM_STAGES == 0 && 512 / GEMM_BK % GEMM_STAGES_BIG == 0,
              "every K (a multiple of 512) is a whole number of register-ring rounds");

// One BM x BN tile of C per workgroup of 4 waves, K in steps of 64.  The global loads of step
// k + S are issued while step k is multiplied: a ring of S register slots (GEMM_STAGES, or
// GEMM_STAGES_BIG for 128-row tiles) feeds a double-buffered LDS tile.
//   BM = 64 / 128: waves form a 2 x 2 grid of (BM / 2) x (BN / 2) tiles, each made of 32 x 32
//            MFMA blocks (128 x 128 tiles halve the L2 traffic per flop of 64 x 64 ones and are
//            used when there are enough of them to fill the CUs).
//   BM = 32 (BN = 64): waves 0/1 and 2/3 compute the same two 32 x 32 blocks over the first and
//            the second half of every K step; the halves are added in LDS before the epilogue
//            (this doubles the workgroups of the N = 1024 GEMMs at M = 512).
// Epilogue of a q or k head tile of the q|k|v GEMM (the work of prefill_qk_norm_rope_kernel,
// fused_prefill_kernels.inl:112-258): the bf16-rounded tile goes through LDS (row stride 136
// bf16), then 16 threads per position take dims 4i .. 4i + 3 and their RoPE partners
// 64 + 4i .. 64 + 4i + 3: RMSNorm over the head, weight, rotate-half RoPE, bf16; the result
// replaces the head in C, and a k head also goes to the K cache and the K operand tiles.
template <int BM, int BN, int MB, int NBK>
MQ_DEV void qk_head_epilogue(const GemmArgs& g, const mq_f32x16 (&acc)[MB][NBK],
                             unsigned char* smem, int m_base, int n_base, int row0, int col0) {
  constexpr int TS = BN + 8;
  constexpr int NR = BM / 16;                       // positions per thread group of 16
  bf16_t* T = reinterpret_cast<bf16_t*>(smem);
  static_assert(TS <= 2 * (GEMM_BK + 8), "the tile fits the A staging buffers (2 x BM rows)");
  const int t = threadIdx.x, lane = t & 63;
  const int i = t & 15, d0 = 4 * i;
  // the RoPE table entries of every position this thread handles, issued before the tile goes
  // through LDS (inside the position loop each position waited for its own: 4096-token prefill
  // 9.19 against 9.31 ms)
  uint2 cl[NR], ch[NR], sl[NR], sh[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const int pos = min(m_base + (t >> 4) + 16 * k, g.M - 1);
    cl[k] = *reinterpret_cast<const uint2*>(g.cs + (size_t)pos * MQ_D + d0);
    ch[k] = *reinterpret_cast<const uint2*>(g.cs + (size_t)pos * MQ_D + 64 + d0);
    sl[k] = *reinterpret_cast<const uint2*>(g.sn + (size_t)pos * MQ_D + d0);
    sh[k] = *reinterpret_cast<const uint2*>(g.sn + (size_t)pos * MQ_D + 64 + d0);
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = row0 + mb * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        T[r * TS + col0 + nb * 32 + (lane & 31)] = f32_to_bf16(acc[mb][nb][j]);
      }
  __syncthreads();
  const bool is_q = n_base < g.n0;
  const int h = (is_q ? n_base : n_base - g.n0) >> 7;
  const bf16_t* nw = is_q ? g.qn : g.kn;
  const uint2 nl = *reinterpret_cast<const uint2*>(nw + d0);
  const uint2 nh = *reinterpret_cast<const uint2*>(nw + 64 + d0);
  const float nwl[4] = {bf16_lo(nl.x), bf16_hi(nl.x), bf16_lo(nl.y), bf16_hi(nl.y)};
  const float nwh[4] = {bf16_lo(nh.x), bf16_hi(nh.x), bf16_lo(nh.y), bf16_hi(nh.y)};
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const int r = (t >> 4) + 16 * k, pos = m_base + r;
    if (pos >= g.M) break;     // whole 16-lane groups leave together
    const uint2 xl = *reinterpret_cast<const uint2*>(T + r * TS + d0);
    const uint2 xh = *reinterpret_cast<const uint2*>(T + r * TS + 64 + d0);
    const float lo[4] = {bf16_lo(xl.x), bf16_hi(xl.x), bf16_lo(xl.y), bf16_hi(xl.y)};
    const float hi[4] = {bf16_lo(xh.x), bf16_hi(xh.x), bf16_lo(xh.y), bf16_hi(xh.y)};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += lo[e] * lo[e] + hi[e] * hi[e];
    ss = row16_sum(ss);
    const float rs = rsqrtf(ss * (1.0f / MQ_D) + MQ_EPS);
    const float cosl[4] = {bf16_lo(cl[k].x), bf16_hi(cl[k].x), bf16_lo(cl[k].y), bf16_hi(cl[k].y)};
    const float cosh_[4] = {bf16_lo(ch[k].x), bf16_hi(ch[k].x), bf16_lo(ch[k].y), bf16_hi(ch[k].y)};
    const float sinl[4] = {bf16_lo(sl[k].x), bf16_hi(sl[k].x), bf16_lo(sl[k].y), bf16_hi(sl[k].y)};
    const float sinh_[4] = {bf16_lo(sh[k].x), bf16_hi(sh[k].x), bf16_lo(sh[k].y), bf16_hi(sh[k].y)};
    bf16_t olo[4], ohi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = lo[e] * rs * nwl[e], b = hi[e] * rs * nwh[e];
      olo[e] = f32_to_bf16(a * cosl[e] - b * sinl[e]);
      ohi[e] = f32_to_bf16(a * sinh_[e] + b * cosh_[e]);
    }
    const uint2 ol = make_uint2((uint32_t)olo[0] | ((uint32_t)olo[1] << 16),
                                (uint32_t)olo[2] | ((uint32_t)olo[3] << 16));
    const uint2 oh = make_uint2((uint32_t)ohi[0] | ((uint32_t)ohi[1] << 16),
                                (uint32_t)ohi[2] | ((uint32_t)ohi[3] << 16));
    bf16_t* x = g.C + (size_t)pos * g.ldc + n_base;
    *reinterpret_cast<uint2*>(x + d0) = ol;
    *reinterpret_cast<uint2*>(x + 64 + d0) = oh;
    if (!is_q) {
      bf16_t* kr = g.kcl + ((size_t)h * g.max_seq + pos) * MQ_D;
      *reinterpret_cast<uint2*>(kr + d0) = ol;
      *reinterpret_cast<uint2*>(kr + 64 + d0) = oh;
      *reinterpret_cast<uint2*>(g.Kt + kt_index(h, g.vt_tiles, pos, d0)) = ol;
      *reinterpret_cast<uint2*>(g.Kt + kt_index(h, g.vt_tiles, pos, 64 + d0)) = oh;
    }
  }
}

template <int EPI, int BM, int BN>
__global__ void __launch_bounds__(256) pf_gemm_kernel(GemmArgs g) {
  constexpr int NB = EPI == EPI_SWIGLU ? 2 : 1;   // weight tiles per step (gate and up)
  constexpr int KG = BM == 32 ? 2 : 1;            // wave groups splitting each K step
  constexpr int WM = KG == 2 ? 32 : BM / 2;       // rows of a wave's tile
  constexpr int WN = BN / 2;                      // columns of a wave's tile
  constexpr int MB = WM / 32, NBK = WN / 32;      // 32 x 32 MFMA blocks per wave tile
  constexpr int BK = BM == 32 ? 128 : GEMM_BK;    // K per step (32-row tiles: fewer, longer steps)
  constexpr int LDSS = BK + 8;                    // bf16 per LDS row (16-byte chunk c of row r at
                                                  // (BK / 8 + 1) r + c: conflict-free reads)
  constexpr int CPR = BK / 8;                     // 16-byte chunks per tile row and step
  constexpr int RPP = 256 / CPR;                  // rows staged per pass of the 256 threads
  constexpr int NA = BM / RPP;                    // 16-byte A loads per thread per step
  constexpr int NL = BN / RPP;                    // 16-byte loads per weight tile per thread
  constexpr int KQ = BK / 16;                     // MFMA k-steps per step
  constexpr int S = BM == 128 ? GEMM_STAGES_BIG : GEMM_STAGES;
  static_assert(BM == 32 || BM == 64 || BM == 128, "tile rows");
  static_assert(BN == 64 || BN == 128, "tile columns");
  static_assert(KG == 1 || BN == 64, "the K-split layout covers 32 x 64 tiles");
  __shared__ __align__(16) bf16_t As[2][BM * LDSS];
  __shared__ __align__(16) bf16_t Bs[2][NB][BN * LDSS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wn = wave & 1;
  const int wm = KG == 1 ? (wave >> 1) : 0;
  const int wk = KG == 2 ? (wave >> 1) : 0;
  const int n_base = blockIdx.x * BN, m_base = blockIdx.y * BM;
  const int kslice = g.K / g.sk, k_first = (int)blockIdx.z * kslice;   // this split's K range
  const bf16_t* B;
  if (n_base < g.n0) B = g.B0 + (size_t)n_base * g.K;
  else if (n_base < g.n1) B = g.B1 + (size_t)(n_base - g.n0) * g.K;
  else B = g.B2 + (size_t)(n_base - g.n1) * g.K;
  const bf16_t* Bu = (EPI == EPI_SWIGLU) ? g.Bu + (size_t)n_base * g.K : B;

  // global -> register staging: thread t moves 16-byte chunk t % CPR of rows t / CPR + RPP i.
  // Rows past M read row M - 1 (their results are never stored).
  const int sr = t / CPR, sk = (t % CPR) * 8;
  const bf16_t* a_src[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int am = min(m_base + sr + RPP * i, g.M - 1);
    a_src[i] = g.A + (size_t)am * g.lda + k_first + sk;
  }
  const bf16_t* b_src[NB];
  b_src[0] = B + (size_t)sr * g.K + k_first + sk;
  if (NB == 2) b_src[NB - 1] = Bu + (size_t)sr * g.K + k_first + sk;

  uint4 ra[S][NA], rb[S][NB][NL];
  auto load_step = [&](int k, uint4 (&a)[NA], uint4 (&b)[NB][NL]) {
    const int k0 = k * BK;
#pragma unroll
    for (int i = 0; i < NA; ++i) a[i] = ld16(a_src[i] + k0);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < NL; ++i) b[j][i] = ld16(b_src[j] + (size_t)(RPP * i) * g.K + k0);
  };
  auto store_step = [&](int buf, const uint4 (&a)[NA], const uint4 (&b)[NB][NL]) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
      *reinterpret_cast<uint4*>(&As[buf][(sr + RPP * i) * LDSS + sk]) = a[i];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < NL; ++i)
        *reinterpret_cast<uint4*>(&Bs[buf][j][(sr + RPP * i) * LDSS + sk]) = b[j][i];
  };

  mq_f32x16 acc[NB][MB][NBK];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[b][mb][nb][j] = 0.f;

  // EPI_RESID: the residual values of this lane's accumulator elements, loaded now so that the
  // epilogue does not start with a memory round trip (element (mb, nb, j): row 32 mb + 8 (j / 4) +
  // 4 (lane / 32) + j % 4, column 32 nb + lane % 32 of the wave's tile; rows past M read row M - 1)
  // (64-row and smaller tiles; the 128-row tiles have no registers to spare)
  constexpr bool RPRE = EPI == EPI_RESID && BM <= 64;
  bf16_t rres[RPRE ? MB : 1][RPRE ? NBK : 1][16];
  if constexpr (RPRE) {
    if (KG == 1 || wk == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb) {
          const int col = n_base + wn * WN + nb * 32 + (lane & 31);
          const int rbase = m_base + wm * WM + mb * 32;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int row = min(rbase + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3), g.M - 1);
            rres[mb][nb][j] = *gptr<bf16_t>(g.R + (size_t)row * g.ldr + col);
          }
        }
    }
  }
  const int fr = lane & 31, fk = (lane >> 5) * 8;   // MFMA operand row and k offset of a lane
  auto mma_step = [&](int buf) {
#pragma unroll
    for (int q = 0; q < KQ / KG; ++q) {
      const int kofs = 16 * (q + wk * (KQ / KG)) + fk;
      mq_bf16x8 af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = as_bf16x8(*reinterpret_cast<const uint4*>(
            &As[buf][(wm * WM + mb * 32 + fr) * LDSS + kofs]));
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb) {
          const mq_bf16x8 bf = as_bf16x8(*reinterpret_cast<const uint4*>(
              &Bs[buf][b][(wn * WN + nb * 32 + fr) * LDSS + kofs]));
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[b][mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], bf, acc[b][mb][nb],
                                                                     0, 0, 0);
        }
    }
  };

  // Schedule (all slot and buffer indices compile-time, so each step is straight-line code and
  // the loads of a slot are waited for only when that slot is stored): step k stores slot
  // (k + 1) % S into LDS buffer (k + 1) % 2, refills slot k % S with step k + S and multiplies
  // buffer k % 2.  The split's K / BK is a multiple of S (the launcher picks sk so).
  const int nk = kslice / BK;
#pragma unroll
  for (int s = 0; s < S; ++s) load_step(s, ra[s], rb[s]);
  store_step(0, ra[0], rb[0]);
  __syncthreads();
  for (int kb = 0; kb < nk - S; kb += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      store_step((s + 1) & 1, ra[(s + 1) % S], rb[(s + 1) % S]);
      load_step(kb + s + S, ra[s], rb[s]);
      mma_step(s & 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s + 1 < S) store_step((s + 1) & 1, ra[s + 1], rb[s + 1]);
    mma_step(s & 1);
    __syncthreads();
  }

  if (KG == 2) {
    // waves 2/3 hand their half-K sums to waves 0/1 through LDS (the last loop step synced)
    float* red = reinterpret_cast<float*>(&As[0][0]);
    if (wk == 1) {
#pragma unroll
      for (int j = 0; j < 16; ++j) red[(wn * 16 + j) * 64 + lane] = acc[0][0][0][j];
    }
    __syncthreads();
    if (wk == 1) return;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[0][0][0][j] += red[(wn * 16 + j) * 64 + lane];
  }

  if (g.sk > 1) {
    // split-K fixup (the waves left after the K-group merge: 128 or 256 threads)
    constexpr int E = NB * MB * NBK * 16;
    constexpr int NT = KG == 2 ? 128 : 256;
    __shared__ uint32_t is_last;
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    float* mine = g.part + ((size_t)tile * g.sk + blockIdx.z) * E * NT + t;
    {
      int e = 0;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
            for (int j = 0; j < 16; ++j, ++e) st_coh(mine + (size_t)e * NT, acc[b][mb][nb][j]);
    }
    wait_all_memory();            // this thread's partial is stored ...
    __syncthreads();              // ... and every other thread's
    if (t == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(g.cnt + tile, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      is_last = prev + 1 == (uint32_t)g.sk;
      if (is_last) __hip_atomic_store(g.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;
    const float* base = g.part + (size_t)tile * g.sk * E * NT + t;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[b][mb][nb][j] = 0.f;
    for (int sp = 0; sp < g.sk; ++sp) {
      const float* src = base + (size_t)sp * E * NT;
      int e = 0;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
            for (int j = 0; j < 16; ++j, ++e) acc[b][mb][nb][j] += ld_coh(src + (size_t)e * NT);
    }
  }

  if constexpr (EPI == EPI_QKV) {
    static_assert(BN == 128 && KG == 1, "one head per tile");
    if (n_base < g.n1) {
      qk_head_epilogue<BM, BN, MB, NBK>(g, acc[0], reinterpret_cast<unsigned char*>(&As[0][0]),
                                        m_base, n_base, wm * WM, wn * WN);
      return;
    }
  }

  // epilogue: acc[.][mb][nb][j] is C[row][col] with row = 32 mb + 8 (j / 4) + 4 (lane / 32) +
  // j % 4, col = 32 nb + lane % 32 within the wave's tile
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb) {
      const int col = n_base + wn * WN + nb * 32 + (lane & 31);
      const int rbase = m_base + wm * WM + mb * 32;
      // the 16 bf16 results of this lane's column, then 32-bit stores of column pairs: lanes 2c
      // and 2c + 1 exchange their values (DPP), the even lane stores rows j < 8 of the pair and
      // the odd lane rows j >= 8
      uint32_t vb[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = rbase + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        float v;
        if (EPI == EPI_STORE || EPI == EPI_QKV) {
          v = acc[0][mb][nb][j];
        } else if (EPI == EPI_RESID) {
          const bf16_t r = RPRE ? rres[RPRE ? mb : 0][RPRE ? nb : 0][j]
                                : g.R[(size_t)min(row, g.M - 1) * g.ldr + col];
          v = round_bf16(acc[0][mb][nb][j]) + bf16_to_f32(r);
        } else {
          const float gv = round_bf16(acc[0][mb][nb][j]), uv = round_bf16(acc[NB - 1][mb][nb][j]);
          v = silu_f(gv) * uv;
        }
        vb[j] = f32_to_bf16(v);
      }
      const bool odd = lane & 1;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(
            0, (int)vb[j], MQ_DPP_QUAD_XOR1, 0xF, 0xF, true);
        const int row = rbase + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        if ((j < 8) != odd && row < g.M) {
          const uint32_t pair = odd ? (other | (vb[j] << 16)) : (vb[j] | (other << 16));
          *reinterpret_cast<uint32_t*>(g.C + (size_t)row * g.ldc + (col & ~1)) = pair;
          if (EPI == EPI_QKV) {
            // v heads (the q/k tiles returned before the loop): the V cache row too
            const int d = (col & ~1) - g.n1;
            *reinterpret_cast<uint32_t*>(
                g.vcl + ((size_t)(d >> 7) * g.max_seq + row) * MQ_D + (d & 127)) = pair;
          }
        }
      }
      if ((EPI == EPI_STORE || EPI == EPI_QKV) && g.Vt != nullptr && n_base >= g.n1) {
        // V^T operand tiles: accumulator elements 4 jg .. 4 jg + 3 are 4 consecutive keys (rows),
        // which are 4 consecutive bf16 of one V^T lane slot
        const int d = col - g.n1, h = d >> 7, dd = d & 127;
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) {
          const int row = rbase + 8 * jg + 4 * (lane >> 5);
          bf16_t* dst = g.Vt + vt_index(h, g.vt_tiles, row, dd);
          if (row + 3 < g.M) {
            uint2 w;
            w.x = pack_bf16x2(acc[0][mb][nb][4 * jg], acc[0][mb][nb][4 * jg + 1]);
            w.y = pack_bf16x2(acc[0][mb][nb][4 * jg + 2], acc[0][mb][nb][4 * jg + 3]);
            *reinterpret_cast<uint2*>(dst) = w;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (row + e < g.M) dst[e] = f32_to_bf16(acc[0][mb][nb][4 * jg + e]);
          }
        }
      }
    }
}


// --------------------------------------------------------------------- causal attention
// Flash-style causal GQA attention (prefill_causal_attention_kernel,
// fused_prefill_kernels.inl:265-342), one wave per (32 query positions, query head), keys in
// tiles of 32, on v_mfma_f32_32x32x16_bf16:
//   S^T = K Q^T      rows are keys, so every lane holds the 16 scores of ONE query (its lane
//                    pair holds the other 16): the softmax max needs one lane swap per tile and
//                    the row sum none until the end;
//   O^T += V^T P^T   P^T is the score accumulator itself.  K tile row r carries key
//                    att_key_perm(r) (bits 2 and 3 of r swapped), which makes accumulator element
//                    j of lane l the key 16 (j / 8) + 8 (l / 32) + j % 8: exactly the B-operand
//                    layout of two 16-key MFMA steps, so P never leaves the registers.
// q and k are bf16, so the fp32 scores are exact up to accumulation order; the softmax is fp32
// and P enters the MFMA as bf16 hi + lo parts (two MFMAs), keeping ~16 more bits than bf16,
// close to the reference's fp32 weights.  V^T (dims x keys) is written by the QKV GEMM epilogue.
#define ATT_KT 32


// A workgroup is one (query head, 32-query block); its blockDim.x / 64 waves (<= ATT_SPLIT) split
// the block's key tiles into contiguous ranges and merge their (max, sum, O) partials through LDS
// at the end, in wave order.  Query blocks are dispatched longest first (blockIdx.y = 0 is the
// last block).  The kernel is held to 256 registers so that two waves share each SIMD: one
// wave's softmax (VALU) runs while the other's MFMAs run.  K is loaded one tile ahead.
#define ATT_SPLIT 4
#define ATT_LAZY 8.0f          // running-max slack (log2 units): weights stay below 2^8
#ifndef ATT_P_SPLIT
#define ATT_P_SPLIT 1
#endif

__global__ void __launch_bounds__(64 * ATT_SPLIT) __attribute__((amdgpu_waves_per_eu(2)))
pf_attn_kernel(MqDecodeParams p, int layer, const bf16_t* __restrict__ qkv,
               const bf16_t* __restrict__ kop, const bf16_t* __restrict__ vop, int ntiles,
               bf16_t* __restrict__ att, int n) {
  __shared__ float red[ATT_SPLIT - 1][66][64];     // waves 1.. : o (64 per lane), m, l
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // kv head h = blockIdx.x % 8 is the XCD the workgroup runs on (workgroups are dealt to the 8
  // XCDs round robin and gridDim.x = 16), so each XCD's L2 holds the K/V^T of one kv head only
  const int h = blockIdx.x & 7, qh = 2 * h + (blockIdx.x >> 3);   // q heads 2h, 2h+1 share h
  const int qb = gridDim.y - 1 - blockIdx.y;
  const int q0 = qb * 32;
  const int fr = lane & 31, hh = lane >> 5;
  const int q = q0 + fr;                           // this lane's query position
  const int t0 = (qb + 1) * wave / nw, t1 = (qb + 1) * (wave + 1) / nw;   // key tiles of this wave
  // this kv head's operand tiles (see kt_index / vt_index): tile t starts at 4096 * t
  const bf16_t* Kt = kop + (size_t)h * ntiles * 4096 + lane * 8;
  const bf16_t* Vt = vop + (size_t)h * ntiles * 4096 + lane * 8;

  // Q^T operand: query q, dims 16 s + 8 hh .. + 8 (rows past n read row n - 1, never stored)
  mq_bf16x8 qf[8];
  {
    const bf16_t* src = qkv + (size_t)min(q, n - 1) * MQ_QKV + qh * MQ_D + 8 * hh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = as_bf16x8(ld16(src + 16 * s));
  }
  // K operand of tile t: key 32 t + att_key_perm(fr), dims 16 s + 8 hh .. + 8 (slots of keys
  // >= n hold stale values; their scores are masked)
  uint4 kf[8];
  auto load_k = [&](int t) {
#pragma unroll
    for (int s = 0; s < 8; ++s) kf[s] = ld16(Kt + (size_t)t * 4096 + s * 512);
  };

  mq_f32x16 o[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[nt][j] = 0.f;
  float m = -INFINITY, l = 0.f;                    // running max (scaled, log2 units) and sum
  const float scale = p.scale_log2;
  // One key tile.  DIAG: the diagonal tile, the only one holding keys > q or keys >= n (its
  // masked variant is compiled separately so the other tiles carry no per-score selects).
  auto tile = [&](int kt, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const int k0 = kt * ATT_KT;
    // V^T operand: dim 32 nt + fr, keys k0 + 16 s + 8 hh .. + 8
    uint4 vf[4][2];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int s = 0; s < 2; ++s) vf[nt][s] = ld16(Vt + (size_t)kt * 4096 + (2 * nt + s) * 512);
    mq_f32x16 sacc;
#pragma unroll
    for (int j = 0; j < 16; ++j) sacc[j] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[s]), qf[s], sacc, 0, 0, 0);
    // unconditional (the last tile of the range reloads itself): a conditional load here made
    // the compiler's wait for V before the O^T MFMAs wait for these K loads as well
    load_k(min(kt + 1, t1 - 1));
    float raw[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = k0 + 16 * (j >> 3) + 8 * hh + (j & 7);
      raw[j] = (!DIAG || key <= q) ? sacc[j] : -INFINITY;
    }
    float mloc = fmaxf(fmaxf(raw[0], raw[1]), raw[2]);
#pragma unroll
    for (int j = 3; j < 15; j += 2) mloc = fmaxf(fmaxf(mloc, raw[j]), raw[j + 1]);
    mloc = fmaxf(mloc, raw[15]);
    // max(raw) * scale == max(raw * scale): rounding is monotonic and scale > 0
    const float mt = max_xor32(mloc) * scale;
    // Lazy running max: a lane takes the tile's max only when it exceeds the max its weights
    // use by more than ATT_LAZY (log2 units), so the weights stay below 2^ATT_LAZY and o and l are
    // rescaled only in the rare tiles where that happens (the result is the same softmax: o and l
    // always share one reference max).  The first tile sets it (m = -inf).
    if (__builtin_amdgcn_ballot_w64(mt > m + ATT_LAZY) != 0) {
      const float m_new = mt > m + ATT_LAZY ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[nt][j] *= alpha;
    }
    // weights p = 2^(s scale - m) as bf16 hi + lo: hi is p rounded to bf16, lo the remainder
    // p - hi (exact in fp32) rounded to bf16; two bf16 values per conversion
    float ls = 0.f;
    uint32_t ph[2][4];
#if ATT_P_SPLIT
    uint32_t pl[2][4];
#endif
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(raw[j], scale, -m));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(raw[j + 1], scale, -m));
      ls += p0;
      ls += p1;
      const uint32_t hp = pack_bf16x2(p0, p1);
      ph[j >> 3][(j & 7) >> 1] = hp;
#if ATT_P_SPLIT
      pl[j >> 3][(j & 7) >> 1] =
          pack_bf16x2(p0 - __uint_as_float(hp << 16), p1 - __uint_as_float(hp & 0xffff0000u));
#endif
    }
    l += ls;
    mq_bf16x8 phi[2];
#if ATT_P_SPLIT
    mq_bf16x8 plo[2];
#endif
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      phi[s] = as_bf16x8(make_uint4(ph[s][0], ph[s][1], ph[s][2], ph[s][3]));
#if ATT_P_SPLIT
      plo[s] = as_bf16x8(make_uint4(pl[s][0], pl[s][1], pl[s][2], pl[s][3]));
#endif
    }
    if (DIAG && k0 + ATT_KT > n) {
      // keys >= n: their weights are 0, but the V^T padding may hold anything (0 * NaN)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int kbase = k0 + 16 * s + 8 * hh;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          uint32_t w[4] = {vf[nt][s].x, vf[nt][s].y, vf[nt][s].z, vf[nt][s].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (kbase + 2 * e >= n) w[e] &= 0xffff0000u;
            if (kbase + 2 * e + 1 >= n) w[e] &= 0x0000ffffu;
          }
          vf[nt][s] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const mq_bf16x8 vb = as_bf16x8(vf[nt][s]);
        o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, phi[s], o[nt], 0, 0, 0);
#if ATT_P_SPLIT
        o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, plo[s], o[nt], 0, 0, 0);
#endif
      }
  };
  if (t0 < t1) load_k(t0);
  const int tend = min(t1, qb);                    // tiles below the diagonal
  for (int kt = t0; kt < tend; ++kt) tile(kt, std::false_type{});
  if (t1 == qb + 1) tile(qb, std::true_type{});
  // merge the key ranges: wave 0 rescales every partial to the common max (a wave with no tiles
  // has m = -inf and contributes 0; the wave holding the diagonal tile always has a finite m)
  if (wave > 0) {
    float* r = &red[wave - 1][0][lane];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) r[(16 * nt + j) * 64] = o[nt][j];
    r[64 * 64] = m;
    r[65 * 64] = l;
  }
  __syncthreads();
  if (wave > 0) return;
  float mt = m;
  for (int w = 1; w < nw; ++w) mt = fmaxf(mt, red[w - 1][64][lane]);
  {
    const float a = __builtin_amdgcn_exp2f(m - mt);
    l *= a;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[nt][j] *= a;
  }
  for (int w = 1; w < nw; ++w) {
    const float a = __builtin_amdgcn_exp2f(red[w - 1][64][lane] - mt);
    l = fmaf(red[w - 1][65][lane], a, l);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[nt][j] = fmaf(red[w - 1][16 * nt + j][lane], a, o[nt][j]);
  }
  // each lane of a pair summed its own 16 keys of every tile
  l = sum_xor32(l);
  if (q < n) {
    const float inv = 1.0f / l;
    bf16_t* dst = att + (size_t)q * MQ_QDIM + qh * MQ_D;
    // O^T accumulator element j of tile nt: dim 32 nt + 8 (j / 4) + 4 hh + j % 4
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        uint2 w;
        w.x = pack_bf16x2(o[nt][4 * jg] * inv, o[nt][4 * jg + 1] * inv);
        w.y = pack_bf16x2(o[nt][4 * jg + 2] * inv, o[nt][4 * jg + 3] * inv);
        *reinterpret_cast<uint2*>(dst + 32 * nt + 8 * jg + 4 * hh) = w;
      }
  }
}

// -------------------------------------------------------------------------- host side
static size_t pf_align(size_t v) { return (v + 255) / 256 * 256; }

// 32-key tiles per kv head of the K / V^T operand copies
static int pf_tiles(int max_n) { return (max_n + 31) / 32; }

static void pf_split_sizes(int max_n, size_t& part_bytes, size_t& tiles);

size_t mq_prefill_workspace_bytes(int max_n) {
  if (max_n <= 0) return 0;
  const size_t n = (size_t)max_n;
  size_t part, tiles;
  pf_split_sizes(max_n, part, tiles);
  return pf_align(n * MQ_H * 2) * 2 + pf_align(n * MQ_QKV * 2) + pf_align(n * MQ_QDIM * 2) +
         pf_align(n * MQ_I * 2) + 2 * pf_align((size_t)MQ_NKV * pf_tiles(max_n) * 4096 * 2) +
         pf_align(part) + pf_align(tiles * 4);
}

void mq_prefill_bind(MqPrefillBuffers* b, char* base, int max_n) {
  b->max_n = max_n;
  if (max_n <= 0) {
    b->h = b->xn = b->qkv = b->att = b->m = b->vt = nullptr;
    b->kt = nullptr;
    b->ntiles = 0;
    b->part = nullptr;
    b->cnt = nullptr;
    b->cnt_bytes = 0;
    return;
  }
  const size_t n = (size_t)max_n;
  char* c = base;
  b->h = reinterpret_cast<bf16_t*>(c);   c += pf_align(n * MQ_H * 2);
  b->xn = reinterpret_cast<bf16_t*>(c);  c += pf_align(n * MQ_H * 2);
  b->qkv = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QKV * 2);
  b->att = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QDIM * 2);
  b->m = reinterpret_cast<bf16_t*>(c);    c += pf_align(n * MQ_I * 2);
  b->vt = reinterpret_cast<bf16_t*>(c);
  b->ntiles = pf_tiles(max_n);
  c += pf_align((size_t)MQ_NKV * b->ntiles * 4096 * 2);
  b->kt = reinterpret_cast<bf16_t*>(c);
  c += pf_align((size_t)MQ_NKV * b->ntiles * 4096 * 2);
  size_t part, tiles;
  pf_split_sizes(max_n, part, tiles);
  b->part = reinterpret_cast<float*>(c);
  c += pf_align(part);
  b->cnt = reinterpret_cast<uint32_t*>(c);
  b->cnt_bytes = pf_align(tiles * 4);
}

// K must be a multiple of 512 and N of 128 (every Qwen3-0.6B projection is).
static_assert(MQ_H % 512 == 0 && MQ_QDIM % 512 == 0 && MQ_I % 512 == 0, "GEMM K steps");
// Tile choice:
// 128 x 128 (128 x 64 for the two SwiGLU matrices) when that still gives >= 512 workgroups
// (two per CU; large M); for the N = 1024 GEMMs (O, down) 128 x 64 when that gives >= 512
// (M >= 4096: the 64 x 64 tiles' waves wait on LDS issue, three LDS instructions per MFMA;
// 4096-token prefill 9.6 -> 9.4 ms with the 4-stage ring above); otherwise 64 x 64, or 32 x 64
// when even 64-row tiles would leave CUs idle (M <= 1024).
//
// Tile and split plan of one GEMM (shared by the launcher and the workspace sizing).
struct GemmPlan {
  int bm, bn, gx, gy, sk, nb;
};
// Smallest split of K that gives >= 480 workgroups (about two per CU), else the largest
// allowed: a split's K must hold a whole ring of steps (BK x S).
static int pick_sk(int tiles, int K, int bk, int stages) {
  const int cands[] = {1, 2, 3, 4, 6, 8};
  int best = 1;
  for (int sk : cands) {
    if (K % sk != 0 || (K / sk) % (bk * stages) != 0) continue;
    best = sk;
    if (tiles * sk >= 480) break;
  }
  return best;
}
template <int EPI>
static GemmPlan gemm_plan(int M, int N, int K) {
  const int mt128 = (M + 127) / 128;
  GemmPlan pl{64, 64, N / 64, (M + 63) / 64, 1, EPI == EPI_SWIGLU ? 2 : 1};
  if constexpr (EPI == EPI_SWIGLU) {
    if ((N / 64) * mt128 >= 512) pl = GemmPlan{128, 64, N / 64, mt128, 1, 2};
  } else if constexpr (EPI == EPI_QKV) {
    // one 128-column head per tile
    if ((N / 128) * mt128 >= 512) pl = GemmPlan{128, 128, N / 128, mt128, 1, 1};
    else pl = GemmPlan{64, 128, N / 128, (M + 63) / 64, 1, 1};
  } else {
    if ((N / 128) * mt128 >= 512) pl = GemmPlan{128, 128, N / 128, mt128, 1, 1};
    else if ((N / 64) * mt128 >= 512) pl = GemmPlan{128, 64, N / 64, mt128, 1, 1};
    else if ((N / 64) * ((M + 63) / 64) < 256) pl = GemmPlan{32, 64, N / 64, (M + 31) / 32, 1, 1};
  }
  // K is split only for the 32 x 64 tiles of short prompts (fewer than 128 tiles, so at most
  // half the CUs busy): there a split's partial is 8 KB and the fixup costs less than the
  // longer K loop it removes (O and down at 16 tokens: 11.8 -> 9.5-10 us).  Larger tiles pay
  // more for the partial round trip than they save (q|k|v and gate|up at 16 tokens 12-12.4 ->
  // 12.9-13.5 us with 4 splits; every GEMM at 512 tokens slower with 2 splits, e.g. gate|up
  // 18.0 -> 23.9 us).
  if (pl.bm == 32 && pl.gx * pl.gy < 128) pl.sk = pick_sk(pl.gx * pl.gy, K, 128, GEMM_STAGES);
  return pl;
}
// fp32 partial bytes of a plan (0 without a split)
static size_t plan_part_bytes(const GemmPlan& pl) {
  return pl.sk > 1 ? (size_t)pl.gx * pl.gy * pl.sk * pl.bm * pl.bn * pl.nb * 4 : 0;
}

template <int EPI>
static void gemm(GemmArgs g, const MqPrefillBuffers& b, hipStream_t s) {
  const GemmPlan pl = gemm_plan<EPI>(g.M, g.N, g.K);
  g.sk = pl.sk;
  g.part = b.part;
  g.cnt = b.cnt;
  const dim3 grid(pl.gx, pl.gy, pl.sk);
  if (pl.bm == 128 && pl.bn == 64) {
    if constexpr (EPI != EPI_QKV) pf_gemm_kernel<EPI, 128, 64><<<grid, 256, 0, s>>>(g);
  } else if (pl.bm == 128) {
    if constexpr (EPI != EPI_SWIGLU) pf_gemm_kernel<EPI, 128, 128><<<grid, 256, 0, s>>>(g);
  } else if (pl.bm == 64 && pl.bn == 128) {
    if constexpr (EPI == EPI_QKV) pf_gemm_kernel<EPI, 64, 128><<<grid, 256, 0, s>>>(g);
  } else if (pl.bm == 32) {
    if constexpr (EPI != EPI_QKV && EPI != EPI_SWIGLU)
      pf_gemm_kernel<EPI, 32, 64><<<grid, 256, 0, s>>>(g);
  } else {
    if constexpr (EPI != EPI_QKV) pf_gemm_kernel<EPI, 64, 64><<<grid, 256, 0, s>>>(g);
  }
}

// Largest split-K partial area and tile count over every prompt length up to max_n.
static void pf_split_sizes(int max_n, size_t& part_bytes, size_t& tiles) {
  part_bytes = 0;
  tiles = 0;
  for (int m = 1; m <= max_n; m = (m < 32 ? 32 : m + 32)) {
    const int mm = m > max_n ? max_n : m;
    const GemmPlan ps[] = {gemm_plan<EPI_QKV>(mm, MQ_QKV, MQ_H),
                           gemm_plan<EPI_RESID>(mm, MQ_H, MQ_QDIM),
                           gemm_plan<EPI_SWIGLU>(mm, MQ_I, MQ_H),
                           gemm_plan<EPI_RESID>(mm, MQ_H, MQ_I)};
    for (const GemmPlan& pl : ps) {
      part_bytes = part_bytes > plan_part_bytes(pl) ? part_bytes : plan_part_bytes(pl);
      const size_t t = (size_t)pl.gx * pl.gy;
      tiles = tiles > t ? tiles : t;
    }
    if (mm == max_n) break;
  }
}

int mq_launch_prefill(const MqDecodeParams& p, const MqLayerW* hl, const MqPrefillBuffers& b,
                      const int32_t* tokens, int n, int32_t* tok_out, float* logits, int grid,
                      hipStream_t stream, const bf16_t* patch, int patch_start, int patch_len,
                      bf16_t* trace) {
  if (n <= 0 || n > b.max_n || n > p.max_seq) return -3;
  if (patch != nullptr && (patch_len <= 0 || patch_start < 0 || patch_start + patch_len > n))
    return -3;
  if (patch == nullptr) patch_len = 0;
  pf_embed_kernel<<<n, 128, 0, stream>>>(p.embed, tokens, b.h, patch, patch_start, patch_len,
                                         p.vocab, &p.st->sync.err.v);
  for (int l = 0; l < p.num_layers; ++l) {
    const MqLayerW& w = hl[l];
    pf_rmsnorm_kernel<<<n, 128, 0, stream>>>(b.h, w.in_ln, b.xn);
    GemmArgs g{};
    g.A = b.xn; g.lda = MQ_H;
    g.B0 = w.wq; g.B1 = w.wk; g.B2 = w.wv; g.n0 = MQ_QDIM; g.n1 = MQ_QDIM + MQ_KVDIM;
    g.C = b.qkv; g.ldc = MQ_QKV; g.M = n; g.N = MQ_QKV; g.K = MQ_H;
    g.Vt = b.vt; g.vt_tiles = b.ntiles;
    g.qn = w.q_norm; g.kn = w.k_norm; g.cs = p.cos; g.sn = p.sin; g.max_seq = p.max_seq;
    g.kcl = p.kc + (size_t)l * MQ_NKV * p.max_seq * MQ_D;
    g.vcl = p.vc + (size_t)l * MQ_NKV * p.max_seq * MQ_D;
    g.Kt = b.kt;
    gemm<EPI_QKV>(g, b, stream);
    pf_attn_kernel<<<dim3(MQ_NQ, (n + 31) / 32), 64 * ATT_SPLIT, 0, stream>>>(
        p, l, b.qkv, b.kt, b.vt, b.ntiles, b.att, n);
    g = GemmArgs{};
    g.A = b.att; g.lda = MQ_QDIM;
    g.B0 = g.B1 = g.B2 = w.wo; g.n0 = g.n1 = MQ_H;
    g.C = b.h; g.ldc = MQ_H; g.R = b.h; g.ldr = MQ_H; g.M = n; g.N = MQ_H; g.K = MQ_QDIM;
    gemm<EPI_RESID>(g, b, stream);
    pf_rmsnorm_kernel<<<n, 128, 0, stream>>>(b.h, w.post_ln, b.xn);
    g = GemmArgs{};
    g.A = b.xn; g.lda = MQ_H;
    g.B0 = g.B1 = g.B2 = w.wg; g.n0 = g.n1 = MQ_I; g.Bu = w.wu;
    g.C = b.m; g.ldc = MQ_I; g.M = n; g.N = MQ_I; g.K = MQ_H;
    gemm<EPI_SWIGLU>(g, b, stream);
    g = GemmArgs{};
    g.A = b.m; g.lda = MQ_I;
    g.B0 = g.B1 = g.B2 = w.wd; g.n0 = g.n1 = MQ_H;
    g.C = b.h; g.ldc = MQ_H; g.R = b.h; g.ldr = MQ_H; g.M = n; g.N = MQ_H; g.K = MQ_I;
    gemm<EPI_RESID>(g, b, stream);
    if (trace != nullptr &&
        hipMemcpyAsync(trace + (size_t)l * n * MQ_H, b.h, (size_t)n * MQ_H * sizeof(bf16_t),
                       hipMemcpyDeviceToDevice, stream) != hipSuccess)
      return -4;
  }
  // last row: final norm rounded to bf16, LM head argmax (fused_prefill_kernels.inl:655-824)
  return mq_launch_lm_head_bf16norm(p, b.h + (size_t)(n - 1) * MQ_H, tok_out, logits, grid,
                                    stream);
}
