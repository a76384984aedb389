// Greedy decode of the dense padded text-view stack on MI355X (gfx950).
//
// Per token: the embedding row; per layer the input norm, the projections (q, k, v, z, b, a of
// the live blocks), the conv and the delta rule of each live value head with its gated norm,
// out_proj and the residual, the post norm, SwiGLU, down_proj and the residual; then the final
// norm and the tied head's first maximum, fed back as the next input. Every projection is a set
// of dense rows streamed from HBM by one wave each: lane l sums its 64th of the row's entries in
// order from +0 (bf16 x bf16 products are exact in fp32, so each term is one fused op), the 64
// lane sums are combined by the wave's pairwise tree (offsets 32..1), and the result is rounded
// to bf16 once. The oracle restates exactly this order for dense matrices. The delta rule keeps
// the stock decode's (ATen's 16-row cascade for the state's row sums), as the sparse paths do.
// (Qwen3_5 decoder layer: transformers/models/qwen3_5/modeling_qwen3_5.py:168-545, :704-793.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lxm_dense.h"
#include "lxm_math.h"

using namespace lxm;

#define NT 512
#define NW (NT / 64)
#define KD 256
#define VD 128
static_assert(NT == KD + 2 * VD, "dn_gdn: one thread per query/key dim, per value and per z");
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// The 512-lane hidden sum of x * x over n <= 4096 values (thread t: its values 4t..4t+3, then
// 2048+4t..2048+4t+3; waves at offsets 32..1; the 8 wave totals at offsets 4, 2, 1).
__device__ __forceinline__ float hidden_sum(const float* x, int n, float* wsum) {
  const int t = threadIdx.x;
  float s = 0.0f;
#pragma unroll
  for (int half = 0; half < 2; half++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = half * 2048 + 4 * t + i;
      if (c < n) s = acc<true>(s, x[c], x[c]);
    }
  s = wave_tree(s);
  if ((t & 63) == 0) wsum[t >> 6] = s;
  __syncthreads();
  float w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}

// The step's input: forced[step] while forced tokens last, else the last prediction; its
// embedding row into h. The head's key is cleared for the step.
__global__ __launch_bounds__(NT) void dn_embed(const lxm_dn_params* __restrict__ pp) {
  const lxm_dn_params& p = *pp;
  const int step = *p.step;
  int tok = step < p.n_forced ? p.forced[step] : *p.tok;
  if (tok < 0 || tok >= p.vocab) {
    if (threadIdx.x == 0) *p.err = 1;
    tok = 0;
  }
  const uint16_t* e = p.embed + (int64_t)tok * p.hidden;
  const int G = p.hidden / 64;
  for (int c = threadIdx.x; c < p.hidden; c += NT) {
    // entry c is lane c / G's entry c % G (interleaved in 8-entry chunks when G >= 8)
    const int l = c / G, k = c % G;
    const int at = G < 8 ? c : ((k >> 3) * 64 + l) * 8 + (k & 7);
    p.h[c] = bf16f(e[at]);
  }
  if (threadIdx.x == 0) *p.keys = 0ull;
}

// out[c] = D((h[c] * r) * (1 + w[c])), r = rsqrt(mean(h^2) + eps) (TF:720-737). One workgroup.
__global__ __launch_bounds__(NT) void dn_norm(const lxm_dn_params* __restrict__ pp, const float* w,
                                              float eps) {
  __shared__ float wsum[NW];
  const lxm_dn_params& p = *pp;
  const int H = p.hidden;
  const float ss = hidden_sum(p.h, H, wsum);
  const float r = rsqrt_(ss / (float)H + eps);
  for (int c = threadIdx.x; c < H; c += NT) p.xn[c] = bf16r((p.h[c] * r) * (1.0f + w[c]));
}

// ---------------------------------------------------------------------------------------------
// Dense rows, one wave per row (grid-stride, rows ascending per wave). G = entries per lane (the
// row's length / 64). The lane's share of the input (bf16-exact values) stays in registers as
// bf16 pairs for every row the wave takes.
template <int G>
struct XChunk {
  static_assert(G % 4 == 0, "16-byte input loads");
  uint32_t v[G / 2];
  // x[lane G .. lane G + G), bf16-exact values
  __device__ __forceinline__ void load(const float* x, int lane) {
    const v4f* src = reinterpret_cast<const v4f*>(x + lane * G);
    v4f a[G / 4];
#pragma unroll
    for (int k = 0; k < G / 4; k++) a[k] = src[k];
#pragma unroll
    for (int k = 0; k < G / 4; k++) {
      v[2 * k] = (fbits(a[k].x) >> 16) | (fbits(a[k].y) & 0xffff0000u);
      v[2 * k + 1] = (fbits(a[k].z) >> 16) | (fbits(a[k].w) & 0xffff0000u);
    }
  }
};
// The lane's sum of its G entries of row w (bf16), in order from +0. A row is stored in 16-byte
// chunks lane-interleaved: chunk q (entries 8q..8q+7) of lane l at (q * 64 + l) * 16 bytes, so each
// of the wave's loads reads 1 KB in one piece (G = 4: lane l's 8 bytes at l * 8).
template <int G>
__device__ __forceinline__ float lane_dot(const uint16_t* w, int lane, const XChunk<G>& x) {
  static_assert(G % 8 == 0 || G == 4, "16-byte weight loads (or 8)");
  float s = 0.0f;
  if constexpr (G == 4) {
    const uint16_t* src = w + (int64_t)lane * G;
    const uint2 u = *reinterpret_cast<const uint2*>(src);
    const uint32_t wv[2] = {u.x, u.y};
#pragma unroll
    for (int k = 0; k < 2; k++) {
      s = __builtin_fmaf(bitsf(x.v[k] << 16), bitsf(wv[k] << 16), s);
      s = __builtin_fmaf(bitsf(x.v[k] & 0xffff0000u), bitsf(wv[k] & 0xffff0000u), s);
    }
  } else {
    v4u wv[G / 8];
#pragma unroll
    for (int q = 0; q < G / 8; q++) wv[q] = reinterpret_cast<const v4u*>(w)[q * 64 + lane];
#pragma unroll
    for (int q = 0; q < G / 8; q++)
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t xx = x.v[4 * q + k], ww = wv[q][k];
        s = __builtin_fmaf(bitsf(xx << 16), bitsf(ww << 16), s);
        s = __builtin_fmaf(bitsf(xx & 0xffff0000u), bitsf(ww & 0xffff0000u), s);
      }
  }
  return s;
}
// the row's sum in the dense order (lane 0 holds it)
template <int G>
__device__ __forceinline__ float row_dot(const uint16_t* w, int lane, const XChunk<G>& x) {
  return wave_tree(lane_dot<G>(w, lane, x));
}

// mode 0: out[row] = D(row . x); mode 1: out[row] = D(out[row] + D(row . x)) (the residual)
template <int G, int MODE>
__global__ __launch_bounds__(NT) void dn_rows(const uint16_t* __restrict__ W, int nrows,
                                              const float* __restrict__ x, float* out) {
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NW + (threadIdx.x >> 6), nwv = gridDim.x * NW;
  XChunk<G> xc;
  xc.load(x, lane);
  for (int r = wv; r < nrows; r += nwv) {
    const float s = row_dot<G>(W + (int64_t)r * 64 * G, lane, xc);
    if (lane == 0) {
      if constexpr (MODE == 0) out[r] = bf16r(s);
      else out[r] = bf16r(out[r] + bf16r(s));
    }
  }
}

// SwiGLU: unit u's gate and up rows, act[u] = D(D(silu(D(g))) * D(u)) (TF:704-717)
template <int G>
__global__ __launch_bounds__(NT) void dn_units(const uint16_t* __restrict__ Wg,
                                               const uint16_t* __restrict__ Wu, int nunits,
                                               const float* __restrict__ x, float* act) {
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NW + (threadIdx.x >> 6), nwv = gridDim.x * NW;
  XChunk<G> xc;
  xc.load(x, lane);
  for (int u = wv; u < nunits; u += nwv) {
    const float g = row_dot<G>(Wg + (int64_t)u * 64 * G, lane, xc);
    const float v = row_dot<G>(Wu + (int64_t)u * 64 * G, lane, xc);
    if (lane == 0) act[u] = bf16r(silu_bf16(bf16r(g)) * bf16r(v));
  }
}

// The head: logits D(row . x) over the vocabulary, the first maximum (ties to the lower index,
// NaN above everything: torch.argmax) folded into *keys by 64-bit atomic max. Each wave takes
// rows in ascending order and keeps its first strict maximum (and its first NaN apart).
template <int G>
__global__ __launch_bounds__(NT) void dn_head(const uint16_t* __restrict__ W, int nrows,
                                              const float* __restrict__ x,
                                              unsigned long long* keys) {
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NW + (threadIdx.x >> 6), nwv = gridDim.x * NW;
  XChunk<G> xc;
  xc.load(x, lane);
  float best = 0.0f;
  int bidx = -1, nanr = -1;
  for (int r = wv; r < nrows; r += nwv) {
    const float v = bf16r(row_dot<G>(W + (int64_t)r * 64 * G, lane, xc));
    if (v != v) {
      if (nanr < 0) nanr = r;
    } else if (bidx < 0 || v > best) {
      best = v;
      bidx = r;
    }
  }
  if (lane == 0) {
    unsigned long long k = bidx < 0 ? 0ull : argmax_key(best, bidx);
    if (nanr >= 0) {
      const unsigned long long kn = argmax_key(__builtin_nanf(""), nanr);
      k = kn > k ? kn : k;
    }
    if (k) atomicMax(keys, k);
  }
}

// the prediction, fed back; the step advanced
__global__ void dn_next(const lxm_dn_params* __restrict__ pp) {
  const lxm_dn_params& p = *pp;
  if (threadIdx.x == 0) {
    const int step = *p.step;
    const int pred = argmax_idx(*p.keys);
    if (step < p.n_steps) p.preds[step] = pred;
    *p.tok = pred;
    *p.step = step + 1;
  }
}

// ---------------------------------------------------------------------------------------------
// The GDN of one live value head per workgroup (vslot = kh x rl + r; value head kh x 8 + r):
// the key head's query and key (conv over the window [x(t-3), x(t-2), x(t-1), P], silu, TF:199-216;
// l2norm in the model dtype, the query times 1/16), the head's values, beta = sigmoid(b),
// g = -exp(A_log) softplus(a + dt_bias) (:497-499), the recurrent step (TF:330-380; the state
// tile in registers, thread = one of ATen's 16-row cascade blocks), the gated norm (TF:168-184)
// into on. The windows are advanced afterwards (dn_windows), once every head has read them.
__device__ __forceinline__ float conv_y(const uint16_t* cs, int64_t chan, const uint16_t* taps, float P) {
  float y = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float x = k < 3 ? bf16f(cs[chan * 4 + k + 1]) : P;
    y = __builtin_fmaf(bf16f(taps[k]), x, y);
  }
  return silu_bf16(bf16r(y));
}
__global__ __launch_bounds__(NT) void dn_gdn(const lxm_dn_params* __restrict__ pp, int L) {
  __shared__ __align__(16) float qd[KD], kd_[KD], qn[KD], kn[KD], vb[VD], zb[VD], dl[VD], ob[VD];
  __shared__ __align__(16) float bs[16 * VD];
  __shared__ float misc[4];
  const lxm_dn_params& p = *pp;
  const lxm_dn_layer& ly = p.layers[L];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nk = p.nk, kl = p.kl, rl = p.rl;
  const int vslot = blockIdx.x, kh = vslot / rl, rr = vslot % rl;
  const int R = p.nv / nk, vh = kh * R + rr;
  const int nq = nk * kl, nvr = nk * rl * VD;
  const float* P = p.P;
  // the state tile first (its loads overlap the inputs' work below)
  const int cg = t & 31, rb = t >> 5;
  v4f* S4 = reinterpret_cast<v4f*>(ly.rec + (size_t)vh * KD * VD);
  v4f s[16];
#pragma unroll
  for (int i = 0; i < 16; i++) s[i] = S4[(rb * 16 + i) * (VD / 4) + cg];
  // rows of P: q [0, nq), k [nq, 2nq), v [2nq, 2nq + nvr), z [.., + nvr), b [.., + nk rl), a
  if (t < KD) {
    float q = 0.0f, k = 0.0f;
    if (t < kl) {
      const int64_t cq = (int64_t)kh * KD + t, ck = (int64_t)nk * KD + kh * KD + t;
      q = conv_y(ly.conv, cq, ly.conv_qk + ((int64_t)kh * kl + t) * 4, P[kh * kl + t]);
      k = conv_y(ly.conv, ck, ly.conv_qk + ((int64_t)(nk + kh) * kl + t) * 4, P[nq + kh * kl + t]);
    }
    qd[t] = q;
    kd_[t] = k;
  } else if (t < KD + VD) {
    const int d = t - KD;
    const int64_t c = 2 * (int64_t)nk * KD + (int64_t)vh * VD + d;
    vb[d] = conv_y(ly.conv, c, ly.conv_v + ((int64_t)vslot * VD + d) * 4, P[2 * nq + vslot * VD + d]);
  } else {
    const int d = t - KD - VD;
    zb[d] = P[2 * nq + nvr + vslot * VD + d];
  }
  if (t == 0) {
    const float b = P[2 * nq + 2 * nvr + vslot], a = P[2 * nq + 2 * nvr + nk * rl + vslot];
    misc[0] = bf16r(sigmoid(b));
    misc[1] = cr_exp((-cr_exp(ly.A_log[vh])) * softplus(a + ly.dt_bias[vh]));
  }
  __syncthreads();
  // l2norm of the query (wave 0) and key (wave 1) in the model dtype; live: any nonzero
  if (wv < 2) {
    const float* x = wv ? kd_ : qd;
    float* o = wv ? kn : qn;
    float xs[4], s = 0.0f;
    bool nz = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xs[i] = x[lane + 64 * i];
      nz |= xs[i] != 0.0f;
      s = s + bf16r(xs[i] * xs[i]);
    }
    if (lane == 0) misc[2 + wv] = __ballot(nz) != 0ull ? 1.0f : 0.0f;
    s = bf16r(sum64(s));
    const float inv = bf16r(rsqrt_(bf16r(s + 1e-6f)));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v = bf16r(xs[i] * inv);
      if (!wv) v = v * 0.0625f;
      o[lane + 64 * i] = v;
    }
  }
  __syncthreads();
  const float beta = misc[0], e = misc[1];
  const bool live = misc[2] != 0.0f || misc[3] != 0.0f;
  if (e != 1.0f) {
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = s[i] * e;
  }
  if (live) {
    v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float f = kn[rb * 16 + i];
      if (f != 0.0f) a = v4f{a.x + s[i].x * f, a.y + s[i].y * f, a.z + s[i].z * f, a.w + s[i].w * f};
    }
    reinterpret_cast<v4f*>(bs + rb * VD)[cg] = a;
    __syncthreads();
    if (t < VD) {
      float kv = 0.0f;
#pragma unroll
      for (int q = 0; q < 16; q++) kv = kv + bs[q * VD + t];
      dl[t] = (vb[t] - kv) * beta;
    }
    __syncthreads();
    const v4f d = reinterpret_cast<const v4f*>(dl)[cg];
    v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float f = kn[rb * 16 + i];
      if (f != 0.0f) s[i] = v4f{s[i].x + f * d.x, s[i].y + f * d.y, s[i].z + f * d.z, s[i].w + f * d.w};
      const float g = qn[rb * 16 + i];
      if (g != 0.0f) o = v4f{o.x + s[i].x * g, o.y + s[i].y * g, o.z + s[i].z * g, o.w + s[i].w * g};
    }
    reinterpret_cast<v4f*>(bs + rb * VD)[cg] = o;
    __syncthreads();
    if (t < VD) {
      float q = 0.0f;
#pragma unroll
      for (int b = 0; b < 16; b++) q = q + bs[b * VD + t];
      ob[t] = bf16r(q);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 16; i++) S4[(rb * 16 + i) * (VD / 4) + cg] = s[i];
  // the gated norm: y = D(D(w * D(o * r)) * silu(z)); a head without a live query or key
  // outputs 0 (the oracle's proc 1)
  if (wv == 0) {
    float* y = p.on + vslot * VD;
    if (live) {
      float ss = 0.0f;
      for (int k = lane; k < VD; k += 64) ss = ss + ob[k] * ob[k];
      ss = sum64(ss);
      const float rr2 = rsqrt_(ss / (float)VD + p.geps);
      for (int k = lane; k < VD; k += 64)
        y[k] = bf16r(bf16r(ly.gnorm[k] * bf16r(ob[k] * rr2)) * silu(zb[k]));
    } else {
      for (int k = lane; k < VD; k += 64) y[k] = 0.0f;
    }
  }
}

// The windows after the step: [x(t-2), x(t-1), P] behind the oldest (causal_conv1d_update's
// shift), for the live channels (query/key of every key head's live dims, values of the live
// heads). One thread per channel.
__global__ void dn_windows(const lxm_dn_params* __restrict__ pp, int L) {
  const lxm_dn_params& p = *pp;
  const lxm_dn_layer& ly = p.layers[L];
  const int nk = p.nk, kl = p.kl, rl = p.rl, R = p.nv / nk;
  const int nq = nk * kl, nvr = nk * rl * VD;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= 2 * nq + nvr) return;
  int64_t chan;
  if (i < 2 * nq) {
    const int part = i / nq, j = i % nq, kh = j / kl, d = j % kl;
    chan = (int64_t)part * nk * KD + kh * KD + d;
  } else {
    const int j = i - 2 * nq, vslot = j / VD, d = j % VD;
    const int kh = vslot / rl, rr = vslot % rl;
    chan = 2 * (int64_t)nk * KD + (int64_t)(kh * R + rr) * VD + d;
  }
  uint16_t* w = ly.conv + chan * 4;
  const uint16_t a = w[1], b = w[2], c = w[3];
  w[0] = a;
  w[1] = b;
  w[2] = c;
  w[3] = (uint16_t)(fbits(p.P[i]) >> 16);
}

// ---------------------------------------------------------------------------------------------
// Host side.
static int rows_grid(int nrows) {
  const int g = (nrows + NW - 1) / NW;
  return g < 2048 ? g : 2048;
}

template <int G, int MODE>
static void launch_rows(const uint16_t* W, int nrows, const float* x, float* out, hipStream_t st) {
  hipLaunchKernelGGL((dn_rows<G, MODE>), dim3(rows_grid(nrows)), dim3(NT), 0, st, W, nrows, x, out);
}

// rows of K entries (K / 64 per lane): the supported lengths
template <int MODE>
static bool rows(int K, const uint16_t* W, int nrows, const float* x, float* out, hipStream_t st) {
  switch (K) {
    case 256: launch_rows<4, MODE>(W, nrows, x, out, st); return true;
    case 512: launch_rows<8, MODE>(W, nrows, x, out, st); return true;
    case 2560: launch_rows<40, MODE>(W, nrows, x, out, st); return true;
    case 4096: launch_rows<64, MODE>(W, nrows, x, out, st); return true;
    case 9216: launch_rows<144, MODE>(W, nrows, x, out, st); return true;
    default: return false;
  }
}
static bool units(int K, const uint16_t* Wg, const uint16_t* Wu, int n, const float* x, float* act,
                  hipStream_t st) {
  const dim3 g(rows_grid(n)), b(NT);
  switch (K) {
    case 256: hipLaunchKernelGGL(dn_units<4>, g, b, 0, st, Wg, Wu, n, x, act); return true;
    case 2560: hipLaunchKernelGGL(dn_units<40>, g, b, 0, st, Wg, Wu, n, x, act); return true;
    default: return false;
  }
}
static bool head(int K, const uint16_t* W, int n, const float* x, unsigned long long* keys,
                 hipStream_t st) {
  const dim3 g(rows_grid(n)), b(NT);
  switch (K) {
    case 256: hipLaunchKernelGGL(dn_head<4>, g, b, 0, st, W, n, x, keys); return true;
    case 2560: hipLaunchKernelGGL(dn_head<40>, g, b, 0, st, W, n, x, keys); return true;
    default: return false;
  }
}

extern "C" int lxm_dn_step(const lxm_dn_params* ph, const lxm_dn_params* pd, void* stream) {
  if (!ph || ph->hidden <= 0 || ph->hidden > 4096 || ph->kl > KD || ph->nv % ph->nk ||
      ph->nk * ph->rl > 128 || !ph->layers || !ph->layers_host)
    return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  const int H = ph->hidden, I = ph->inter, nk = ph->nk, kl = ph->kl, rl = ph->rl;
  const int nq = nk * kl, nvr = nk * rl * VD, nproj = 2 * nq + 2 * nvr + 2 * nk * rl;
  hipLaunchKernelGGL(dn_embed, dim3(1), dim3(NT), 0, st, pd);
  for (int L = 0; L < ph->n_layers; L++) {
    // the row kernels take their weights as arguments (from the host copy of the table); the
    // other kernels read the device table
    const lxm_dn_layer& ly = ph->layers_host[L];
    hipLaunchKernelGGL(dn_norm, dim3(1), dim3(NT), 0, st, pd, ly.ln_in, ph->rms_eps);
    if (!rows<0>(H, ly.proj, nproj, ph->xn, ph->P, st)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(dn_gdn, dim3(nk * rl), dim3(NT), 0, st, pd, L);
    hipLaunchKernelGGL(dn_windows, dim3((2 * nq + nvr + 255) / 256), dim3(256), 0, st, pd, L);
    if (!rows<1>(nvr, ly.out, H, ph->on, ph->h, st)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(dn_norm, dim3(1), dim3(NT), 0, st, pd, ly.ln_post, ph->rms_eps);
    if (!units(H, ly.gate, ly.up, I, ph->xn, ph->xn + H, st)) return (int)hipErrorInvalidValue;
    if (!rows<1>(I, ly.down, H, ph->xn + H, ph->h, st)) return (int)hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(dn_norm, dim3(1), dim3(NT), 0, st, pd, ph->w_final, ph->rms_eps);
  if (!head(H, ph->embed, ph->vocab, ph->xn, ph->keys, st)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(dn_next, dim3(1), dim3(64), 0, st, pd);
  return (int)hipGetLastError();
}
