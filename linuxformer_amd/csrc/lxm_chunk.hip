// The stock forward's chunked delta rule (torch_chunk_gated_delta_rule, transformers qwen3_5
// :249-327) for one chunk of <= 64 positions, on MI355X's matrix cores.
//
// One workgroup (8 waves) per (value head, 32 state columns). Everything a chunk needs sits in
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

constexpr int CT = 512;       // threads per workgroup (8 waves: two per SIMD)
constexpr int NWV = CT / 64;
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

__device__ __forceinline__ int wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// acc += A B over k blocks kb0 .. kb1 - 1 of 16 (k = 16 kb + 4 j + a_k): fa(k) and fb(k) give
// this lane's A and B elements. Each block's 8 operands are read before the previous block's 4
// MFMAs issue, so the LDS reads overlap the matrix core.
template <class FA, class FB>
__device__ __forceinline__ v4f tile_mm(int kb0, int kb1, const Lane& ln, FA fa, FB fb, v4f acc) {
  if (kb0 >= kb1) return acc;
  float a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    a[j] = fa(16 * kb0 + 4 * j + ln.a_k);
    b[j] = fb(16 * kb0 + 4 * j + ln.a_k);
  }
  for (int kb = kb0; kb < kb1; kb++) {
    float an[4], bn[4];
    const int kn = kb + 1 < kb1 ? kb + 1 : kb;  // (the last block reads its own operands again)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      an[j] = fa(16 * kn + 4 * j + ln.a_k);
      bn[j] = fb(16 * kn + 4 * j + ln.a_k);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) acc = mfma4(a[j], b[j], acc);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      a[j] = an[j];
      b[j] = bn[j];
    }
  }
  return acc;
}

}  // namespace

__global__ __launch_bounds__(CT) void lxm_chunk_k(lxm_chunk_io io) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  ChunkLds& l = *reinterpret_cast<ChunkLds*>(smem_raw);
  const int t = threadIdx.x, w = wave(), h = blockIdx.x, c0 = blockIdx.y * VT;
  const int n = io.n, kl = io.kl, kh = h / io.rl;
  const Lane ln;
  float* Sg = io.S + ((size_t)kh * io.rfull + h % io.rl) * 256 * VD;
  constexpr int NKB = KL / 16;  // k blocks over the key dims (zeros past kl add nothing)

  // ---- inputs into LDS (zero past n positions and kl dims), four values per load
  for (int idx = t; idx < C * KL / 4; idx += CT) {
    const int i = idx / (KL / 4), d = 4 * (idx % (KL / 4));
    v4f kv = {0.0f, 0.0f, 0.0f, 0.0f}, qv = kv;
    if (i < n && d < kl) {
      const int64_t o = (int64_t)i * io.qk_ts + (int64_t)kh * io.qk_hs + d;
      kv = *reinterpret_cast<const v4f*>(io.k + o);
      qv = *reinterpret_cast<const v4f*>(io.q + o);
    }
    *reinterpret_cast<v4f*>(&l.k[i][d]) = kv;
    *reinterpret_cast<v4f*>(&l.qw[i][d]) = qv;
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
  for (int idx = t; idx < KL * VT / 4; idx += CT) {
    const int d = idx / (VT / 4), c = 4 * (idx % (VT / 4));
    v4f sv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (d < kl) sv = *reinterpret_cast<const v4f*>(Sg + (size_t)d * VD + c0 + c);
    *reinterpret_cast<v4f*>(&l.s[d][c]) = sv;
  }
  __syncthreads();
  if (t == 0) {  // cumsum of g: binary64 accumulation, each prefix rounded (ATen's CPU cumsum)
    double acc = 0.0;
    for (int i = 0; i < C; i++) {
      acc += (double)l.gc[i];
      l.gc[i] = (float)acc;
    }
  }
  for (int idx = t; idx < C * VT / 4; idx += CT) {
    const int i = idx / (VT / 4), c = 4 * (idx % (VT / 4));
    v4f vv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (i < n) vv = *reinterpret_cast<const v4f*>(io.v + (int64_t)i * io.v_ts + (int64_t)h * VD + c0 + c);
    const float b = l.beta[i];
    *reinterpret_cast<v4f*>(&l.vb[i][c]) = v4f{vv.x * b, vv.y * b, vv.z * b, vv.w * b};
  }
  __syncthreads();
  if (t < C) {
    const float glast = l.gc[C - 1];
    l.eg[t] = cr_exp(l.gc[t]);
    l.f[t] = cr_exp(glast - l.gc[t]);
    if (t == 0) l.misc[0] = cr_exp(glast);
  }
  __syncthreads();

  // ---- A2 = (q k^T) * Gamma and L = (k beta k^T) * Gamma (strictly lower) on the 10 tiles on
  // or below the diagonal, dealt to the waves (tile p: row block ti, column block tj <= ti);
  // O1 = (q exp(gc)) S: wave w takes row block w % 4, column tile w / 4
  for (int p = w; p < 10; p += NWV) {
    const int ti = p < 1 ? 0 : p < 3 ? 1 : p < 6 ? 2 : 3;
    const int tj = p - ti * (ti + 1) / 2;
    const int ia = 16 * ti + ln.a_i, jb = 16 * tj + ln.a_i;
    const float bi = l.beta[ia];
    v4f aq = {0.0f, 0.0f, 0.0f, 0.0f}, ak = aq;
    float qa[4], ka[4], kb[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      qa[j] = l.qw[ia][4 * j + ln.a_k];
      ka[j] = l.k[ia][4 * j + ln.a_k] * bi;
      kb[j] = l.k[jb][4 * j + ln.a_k];
    }
    for (int d0 = 0; d0 < KL; d0 += 16) {
      float qn[4], kn[4], bn[4];
      const int dn = d0 + 16 < KL ? d0 + 16 : d0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        qn[j] = l.qw[ia][dn + 4 * j + ln.a_k];
        kn[j] = l.k[ia][dn + 4 * j + ln.a_k] * bi;
        bn[j] = l.k[jb][dn + 4 * j + ln.a_k];
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        aq = mfma4(qa[j], kb[j], aq);
        ak = mfma4(ka[j], kb[j], ak);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        qa[j] = qn[j];
        ka[j] = kn[j];
        kb[j] = bn[j];
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
  // the six tiles above the diagonal are zero in both
  for (int idx = t; idx < 6 * 256; idx += CT) {
    const int p = idx / 256, e = idx % 256;
    const int ti = p < 3 ? 0 : p < 5 ? 1 : 2, tj = p < 3 ? p + 1 : p < 5 ? p - 1 : 3;
    l.a2[16 * ti + e / 16][16 * tj + e % 16] = 0.0f;
    l.lp[16 * ti + e / 16][16 * tj + e % 16] = 0.0f;
  }
  const int ob = w & 3, oc = w >> 2;  // this wave's output tile of the (64, 32) products
  v4f o1 = {0.0f, 0.0f, 0.0f, 0.0f};
  {
    const int ia = 16 * ob + ln.a_i;
    const float e = l.eg[ia];
    o1 = tile_mm(0, NKB, ln, [&](int k) { return l.qw[ia][k] * e; },
                 [&](int k) { return l.s[k][16 * oc + ln.a_i]; }, o1);
  }
  __syncthreads();

  // ---- T = (I + L)^-1: diagonal block w (waves 0..3) by forward substitution (lanes 0..15
  // are the columns: T[i][j] = -sum_{m=j}^{i-1} L[i][m] T[m][j], T[i][i] = 1); blocks above
  // the diagonal are zero
  if (w < 4) {
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
  } else {
    for (int idx = t - 256; idx < 6 * 256; idx += 256) {
      const int p = idx / 256, e = idx % 256;
      const int ti = p < 3 ? 0 : p < 5 ? 1 : 2, tj = p < 3 ? p + 1 : p < 5 ? p - 1 : 3;
      l.tt[16 * ti + e / 16][16 * tj + e % 16] = 0.0f;
    }
  }
  __syncthreads();
  // block rows 1..3: T_ij = -T_ii P, P = sum_{k=j}^{i-1} L_ik T_kj; block (i, j) on wave j
  for (int bi = 1; bi < 4; bi++) {
    if (w < bi) {
      const int bj = w;
      v4f p = {0.0f, 0.0f, 0.0f, 0.0f};
      p = tile_mm(bj, bi, ln, [&](int k) { return l.lp[16 * bi + ln.a_i][k]; },
                  [&](int k) { return l.tt[k][16 * bj + ln.a_i]; }, p);
#pragma unroll
      for (int r = 0; r < 4; r++) l.pt[w][ln.d_i + r][ln.d_j] = p[r];
      __builtin_amdgcn_wave_barrier();
      v4f q = {0.0f, 0.0f, 0.0f, 0.0f};
      q = tile_mm(0, 1, ln, [&](int k) { return l.tt[16 * bi + ln.a_i][16 * bi + k]; },
                  [&](int k) { return l.pt[w][k][ln.a_i]; }, q);
#pragma unroll
      for (int r = 0; r < 4; r++) l.tt[16 * bi + ln.d_i + r][16 * bj + ln.d_j] = -q[r];
    }
    __syncthreads();
  }

  // ---- W = T (k beta exp(gc)) into qw (the queries are no longer read): the 32 tiles (4 row
  // blocks x 8 column blocks) dealt to the waves; T is lower triangular (k blocks <= the row's)
  for (int p = w; p < 32; p += NWV) {
    const int ti = p & 3, tc = p >> 2;
    v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
    a = tile_mm(0, ti + 1, ln, [&](int k) { return l.tt[16 * ti + ln.a_i][k]; },
                [&](int k) { return (l.k[k][16 * tc + ln.a_i] * l.beta[k]) * l.eg[k]; }, a);
#pragma unroll
    for (int r = 0; r < 4; r++) l.qw[16 * ti + ln.d_i + r][16 * tc + ln.d_j] = a[r];
  }
  __syncthreads();

  // ---- v_new = T (v beta) - W S on the wave's output tile, into lp (L was last read by the
  // block stages, before the barriers above)
  {
    v4f u = {0.0f, 0.0f, 0.0f, 0.0f}, vp = u;
    u = tile_mm(0, ob + 1, ln, [&](int k) { return l.tt[16 * ob + ln.a_i][k]; },
                [&](int k) { return l.vb[k][16 * oc + ln.a_i]; }, u);
    vp = tile_mm(0, NKB, ln, [&](int k) { return l.qw[16 * ob + ln.a_i][k]; },
                 [&](int k) { return l.s[k][16 * oc + ln.a_i]; }, vp);
#pragma unroll
    for (int r = 0; r < 4; r++) l.lp[16 * ob + ln.d_i + r][16 * oc + ln.d_j] = u[r] - vp[r];
  }
  __syncthreads();

  // ---- o = O1 + A2 v_new on the wave's output tile (A2 is lower triangular)
  {
    v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
    a = tile_mm(0, ob + 1, ln, [&](int k) { return l.a2[16 * ob + ln.a_i][k]; },
                [&](int k) { return l.lp[k][16 * oc + ln.a_i]; }, a);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = 16 * ob + ln.d_i + r, c = 16 * oc + ln.d_j;
      if (i < n) {
        const float v = o1[r] + a[r];
        io.o[(int64_t)i * io.o_ts + (int64_t)h * VD + c0 + c] = io.o_bf16 ? bf16r(v) : v;
      }
    }
  }
  // ---- S <- S exp(g_last) + (k f)^T v_new: the state's 16 tiles (8 row blocks x 2 column
  // tiles) dealt to the waves (row blocks past kl skipped)
  {
    const float el = l.misc[0];
    for (int p = w; p < 2 * KL / 16; p += NWV) {
      const int rb = p >> 1, tc = p & 1;
      if (16 * rb >= kl) continue;
      v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
      a = tile_mm(0, C / 16, ln, [&](int m) { return l.k[m][16 * rb + ln.a_i] * l.f[m]; },
                  [&](int m) { return l.lp[m][16 * tc + ln.a_i]; }, a);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int d = 16 * rb + ln.d_i + r, c = 16 * tc + ln.d_j;
        Sg[(size_t)d * VD + c0 + c] = l.s[d][c] * el + a[r];
      }
    }
  }
}

// q, k, v and S are read four floats at a time: their pointers 16-byte aligned, and the strides
// between those reads multiples of 4 floats
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int lxm_gdn_chunk(const lxm_chunk_io* io, void* stream) {
  if (!io || io->n < 1 || io->n > C || io->kl < 1 || io->kl > KL || io->kl % 16 != 0 ||
      io->n_slots < 1 || io->rl < 1 || io->rfull < io->rl)
    return (int)hipErrorInvalidValue;
  if (!al16(io->q) || !al16(io->k) || !al16(io->v) || !al16(io->S) || io->qk_ts % 4 != 0 ||
      io->qk_hs % 4 != 0 || io->v_ts % 4 != 0)
    return (int)hipErrorInvalidValue;
  const int lds = (int)sizeof(ChunkLds);
  hipError_t e = hipFuncSetAttribute((const void*)lxm_chunk_k,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(lxm_chunk_k, dim3(io->n_slots, VD / VT), dim3(CT), lds,
                     (hipStream_t)stream, *io);
  return (int)hipGetLastError();
}
