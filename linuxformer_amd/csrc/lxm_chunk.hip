// The stock forward's chunked delta rule (torch_chunk_gated_delta_rule, transformers qwen3_5
// :249-327) for one chunk of <= 64 positions, on MI355X's matrix cores.
//
// One workgroup (4 waves) per (value head, 32 state columns). Everything a chunk needs sits in
// LDS as fp32 (the keys and queries over the live key dims, the state's 32 columns, the values
// times beta), and every matrix product is a sequence of v_mfma_f32_16x16x4_f32 (a 16 x 16 tile
// += 16 x 4 times 4 x 16; lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds
// D[4 (l / 16) + r][l % 16], r = 0..3):
//   A2 = (q k^T) * Gamma,   Gamma[i][j] = exp(gc_i - gc_j) for j <= i, else 0  (gc: cumsum g)
//   O1 = (q exp(gc)) S
//   L  = (k beta k^T) * Gamma below the diagonal;  T = (I + L)^-1  (the stock loop's result + I)
//   W  = T (k beta exp(gc));  U = T (v beta);  v_new = U - W S
//   o  = O1 + A2 v_new;  S <- S exp(g_last) + (k exp(g_last - gc))^T v_new
// T is formed by blocks of 16: each diagonal block by forward substitution on one wave, then the
// blocks below it one block row at a time, T_ij = -T_ii (sum_{k=j}^{i-1} L_ik T_kj), on MFMA.
// The workgroups of a head repeat the head's Gram matrices and inverse (they are small) and each
// takes its own 32 columns of the state, so the grid has no dependency between workgroups.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lxm_chunk.h"
#include "lxm_math.h"

using namespace lxm;

namespace {

constexpr int CT = 256;       // threads per workgroup (4 waves)
constexpr int C = 64;         // positions per chunk
constexpr int KL = 128;       // live key dims at most
constexpr int VD = 128;
constexpr int VT = 32;        // state columns per workgroup
constexpr int SK = KL + 4;    // row strides in floats (LDS padding)
constexpr int SC = C + 4;
constexpr int SV = VT + 4;
constexpr int ST = 16 + 1;

struct ChunkLds {
  float k[C][SK];             // keys (rows past n and dims past kl: 0)
  float qw[C][SK];            // queries, then W = T (k beta exp(gc))
  float a2[C][SC];            // (q k^T) * Gamma
  float lp[C][SC];            // L = (k beta k^T) * Gamma, strictly lower; later v_new
  float tt[C][SC];            // T = (I + L)^-1
  float s[KL][SV];            // the state's columns
  float vb[C][SV];            // v beta
  float pt[4][16][ST];        // per-wave 16 x 16 scratch (the block inverse)
  float gc[C], eg[C], f[C], beta[C];
  float misc[4];
};
static_assert(sizeof(ChunkLds) <= 160 * 1024, "one workgroup's LDS");

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// the tile's lane coordinates: A/B operand row (or column) a_i and k index a_k; D rows d_i + r
struct Lane {
  int a_i, a_k, d_i, d_j;
  __device__ Lane() {
    const int l = threadIdx.x & 63;
    a_i = l & 15;
    a_k = l >> 4;
    d_i = 4 * (l >> 4);
    d_j = l & 15;
  }
};

// dispatch of one of the four waves' rows of a 16 x 16 output tile
__device__ __forceinline__ int wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

}  // namespace

__global__ __launch_bounds__(CT) void lxm_chunk_k(lxm_chunk_io io) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  ChunkLds& l = *reinterpret_cast<ChunkLds*>(smem_raw);
  const int t = threadIdx.x, w = wave(), h = blockIdx.x, c0 = blockIdx.y * VT;
  const int n = io.n, kl = io.kl, kh = h / io.rl;
  const Lane ln;
  float* Sg = io.S + ((size_t)kh * io.rfull + h % io.rl) * 256 * VD;

  // ---- inputs into LDS (zero past n positions and kl dims)
  for (int idx = t; idx < C * KL; idx += CT) {
    const int i = idx / KL, d = idx % KL;
    float kv = 0.0f, qv = 0.0f;
    if (i < n && d < kl) {
      kv = io.k[(int64_t)i * io.qk_ts + (int64_t)kh * io.qk_hs + d];
      qv = io.q[(int64_t)i * io.qk_ts + (int64_t)kh * io.qk_hs + d];
    }
    l.k[i][d] = kv;
    l.qw[i][d] = qv;
  }
  if (t < C) {
    float b = 0.0f, g = 0.0f;
    if (t < n) {
      b = io.beta[(int64_t)t * io.g_ts + (int64_t)h * io.g_hs];
      g = io.g[(int64_t)t * io.gl_ts + h];
    }
    l.beta[t] = b;
    l.gc[t] = g;
  }
  for (int idx = t; idx < KL * VT; idx += CT) {
    const int d = idx / VT, c = idx % VT;
    l.s[d][c] = d < kl ? Sg[(size_t)d * VD + c0 + c] : 0.0f;
  }
  __syncthreads();
  if (t == 0) {  // cumsum of g: binary64 accumulation, each prefix rounded (ATen's CPU cumsum)
    double acc = 0.0;
    for (int i = 0; i < C; i++) {
      acc += (double)l.gc[i];
      l.gc[i] = (float)acc;
    }
  }
  for (int idx = t; idx < C * VT; idx += CT) {
    const int i = idx / VT, c = idx % VT;
    l.vb[i][c] = (i < n ? io.v[(int64_t)i * io.v_ts + (int64_t)h * VD + c0 + c] : 0.0f) * l.beta[i];
  }
  __syncthreads();
  if (t < C) {
    const float glast = l.gc[C - 1];
    l.eg[t] = cr_exp(l.gc[t]);
    l.f[t] = cr_exp(glast - l.gc[t]);
    if (t == 0) l.misc[0] = cr_exp(glast);
  }
  __syncthreads();

  // ---- A2 = (q k^T) * Gamma and L = (k beta k^T) * Gamma (strictly lower): wave w takes row
  // block w, column blocks 0..w (the rest are zero); O1 = (q exp(gc)) S on the wave's row block
  v4f o1[VT / 16];
  {
    const int ti = w;
    for (int tj = 0; tj < 4; tj++) {
      v4f aq = {0.0f, 0.0f, 0.0f, 0.0f}, ak = {0.0f, 0.0f, 0.0f, 0.0f};
      if (tj <= ti) {
        const int ia = 16 * ti + ln.a_i, jb = 16 * tj + ln.a_i;
        const float bi = l.beta[ia];
        for (int d0 = 0; d0 < kl; d0 += 4) {
          const float kb = l.k[jb][d0 + ln.a_k];  // B[d][j] = k[j][d]
          aq = mfma4(l.qw[ia][d0 + ln.a_k], kb, aq);
          ak = mfma4(l.k[ia][d0 + ln.a_k] * bi, kb, ak);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int i = 16 * ti + ln.d_i + r, j = 16 * tj + ln.d_j;
        const float gm = j <= i ? cr_exp(l.gc[i] - l.gc[j]) : 0.0f;
        l.a2[i][j] = aq[r] * gm;
        l.lp[i][j] = j < i ? ak[r] * gm : 0.0f;
      }
    }
#pragma unroll
    for (int tc = 0; tc < VT / 16; tc++) {
      v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
      const int ia = 16 * ti + ln.a_i;
      const float e = l.eg[ia];
      for (int d0 = 0; d0 < kl; d0 += 4)
        a = mfma4(l.qw[ia][d0 + ln.a_k] * e, l.s[d0 + ln.a_k][16 * tc + ln.a_i], a);
      o1[tc] = a;
    }
  }
  __syncthreads();

  // ---- T = (I + L)^-1: diagonal block w by forward substitution on wave w (lanes 0..15 are
  // the columns: T[i][j] = -sum_{m=j}^{i-1} L[i][m] T[m][j], T[i][i] = 1)
  {
    const int b0 = 16 * w, j = t & 63;
    if (j < 16) l.tt[b0][b0 + j] = j == 0 ? 1.0f : 0.0f;
    __builtin_amdgcn_wave_barrier();
    for (int i = 1; i < 16; i++) {
      if (j < 16) {
        float s = 0.0f;
        for (int m = j; m < i; m++) s = s + l.lp[b0 + i][b0 + m] * l.tt[b0 + m][b0 + j];
        l.tt[b0 + i][b0 + j] = j < i ? -s : (j == i ? 1.0f : 0.0f);
      }
      __builtin_amdgcn_wave_barrier();
    }
    // the blocks above the diagonal are zero
    if (j < 16)
      for (int jb = w + 1; jb < 4; jb++)
        for (int i = 0; i < 16; i++) l.tt[b0 + i][16 * jb + j] = 0.0f;
  }
  __syncthreads();
  // block rows 1..3: T_ij = -T_ii P, P = sum_{k=j}^{i-1} L_ik T_kj; block (i, j) on wave j
  for (int bi = 1; bi < 4; bi++) {
    if (w < bi) {
      const int bj = w;
      v4f p = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int bk = bj; bk < bi; bk++)
        for (int m0 = 0; m0 < 16; m0 += 4)
          p = mfma4(l.lp[16 * bi + ln.a_i][16 * bk + m0 + ln.a_k],
                    l.tt[16 * bk + m0 + ln.a_k][16 * bj + ln.a_i], p);
#pragma unroll
      for (int r = 0; r < 4; r++) l.pt[w][ln.d_i + r][ln.d_j] = p[r];
      __builtin_amdgcn_wave_barrier();
      v4f q = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m0 = 0; m0 < 16; m0 += 4)
        q = mfma4(l.tt[16 * bi + ln.a_i][16 * bi + m0 + ln.a_k], l.pt[w][m0 + ln.a_k][ln.a_i], q);
#pragma unroll
      for (int r = 0; r < 4; r++) l.tt[16 * bi + ln.d_i + r][16 * bj + ln.d_j] = -q[r];
    }
    __syncthreads();
  }

  // ---- W = T (k beta exp(gc)) into qw (the queries are no longer read): wave w takes column
  // blocks 2w, 2w + 1 of every row block (T is lower triangular: k blocks <= the row block)
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const int tc = 2 * w + cb;
    if (16 * tc >= kl) continue;
    for (int ti = 0; ti < 4; ti++) {
      v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m0 = 0; m0 < 16 * (ti + 1); m0 += 4) {
        const int m = m0 + ln.a_k;
        a = mfma4(l.tt[16 * ti + ln.a_i][m], (l.k[m][16 * tc + ln.a_i] * l.beta[m]) * l.eg[m], a);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) l.qw[16 * ti + ln.d_i + r][16 * tc + ln.d_j] = a[r];
    }
  }
  __syncthreads();

  // ---- v_new = T (v beta) - W S on the wave's row block, into lp (L is no longer read)
  {
    const int ti = w;
#pragma unroll
    for (int tc = 0; tc < VT / 16; tc++) {
      v4f u = {0.0f, 0.0f, 0.0f, 0.0f}, vp = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m0 = 0; m0 < 16 * (ti + 1); m0 += 4)
        u = mfma4(l.tt[16 * ti + ln.a_i][m0 + ln.a_k], l.vb[m0 + ln.a_k][16 * tc + ln.a_i], u);
      for (int d0 = 0; d0 < kl; d0 += 4)
        vp = mfma4(l.qw[16 * ti + ln.a_i][d0 + ln.a_k], l.s[d0 + ln.a_k][16 * tc + ln.a_i], vp);
#pragma unroll
      for (int r = 0; r < 4; r++) l.lp[16 * ti + ln.d_i + r][16 * tc + ln.d_j] = u[r] - vp[r];
    }
  }
  __syncthreads();

  // ---- o = O1 + A2 v_new on the wave's row block (A2 is lower triangular)
  {
    const int ti = w;
#pragma unroll
    for (int tc = 0; tc < VT / 16; tc++) {
      v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m0 = 0; m0 < 16 * (ti + 1); m0 += 4)
        a = mfma4(l.a2[16 * ti + ln.a_i][m0 + ln.a_k], l.lp[m0 + ln.a_k][16 * tc + ln.a_i], a);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int i = 16 * ti + ln.d_i + r, c = 16 * tc + ln.d_j;
        if (i < n) {
          const float v = o1[tc][r] + a[r];
          io.o[(int64_t)i * io.o_ts + (int64_t)h * VD + c0 + c] = io.o_bf16 ? bf16r(v) : v;
        }
      }
    }
  }
  // ---- S <- S exp(g_last) + (k f)^T v_new: rows d of the state (kl of them), wave w takes
  // row blocks w, w + 4 (only those below kl)
  {
    const float el = l.misc[0];
    for (int rb = w; rb < KL / 16; rb += 4) {
      if (16 * rb >= kl) continue;
#pragma unroll
      for (int tc = 0; tc < VT / 16; tc++) {
        v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int m0 = 0; m0 < C; m0 += 4) {
          const int m = m0 + ln.a_k;
          a = mfma4(l.k[m][16 * rb + ln.a_i] * l.f[m], l.lp[m][16 * tc + ln.a_i], a);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int d = 16 * rb + ln.d_i + r, c = 16 * tc + ln.d_j;
          Sg[(size_t)d * VD + c0 + c] = l.s[d][c] * el + a[r];
        }
      }
    }
  }
}

extern "C" int lxm_gdn_chunk(const lxm_chunk_io* io, void* stream) {
  if (!io || io->n < 1 || io->n > C || io->kl < 1 || io->kl > KL || io->kl % 16 != 0 ||
      io->n_slots < 1 || io->rl < 1 || io->rfull < io->rl)
    return (int)hipErrorInvalidValue;
  const int lds = (int)sizeof(ChunkLds);
  hipError_t e = hipFuncSetAttribute((const void*)lxm_chunk_k,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(lxm_chunk_k, dim3(io->n_slots, VD / VT), dim3(CT), lds,
                     (hipStream_t)stream, *io);
  return (int)hipGetLastError();
}
