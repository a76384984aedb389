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
  lds_barrier();  // (weight rows already requested stay in flight)
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

// The RMSNorm factor r = rsqrt(mean(h^2) + eps) of TF:720-737, computed by every workgroup that
// consumes the norm (the sum in the 512-lane order above); x[c] = D((h[c] * r) * (1 + w[c])).
__device__ __forceinline__ float norm_factor(const float* h, int H, float eps, float* wsum) {
  return rsqrt_(hidden_sum(h, H, wsum) / (float)H + eps);
}
__device__ __forceinline__ float norm_el(float h, float r, float w) {
  return bf16r((h * r) * (1.0f + w));
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (fbits(lo) >> 16) | (fbits(hi) & 0xffff0000u);
}

// ---------------------------------------------------------------------------------------------
// Dense rows, one wave per row (grid-stride, rows ascending per wave). G = entries per lane (the
// row's length / 64). A row is stored in 16-byte chunks lane-interleaved: chunk q (entries
// 8q..8q+7 of lane l's G) at (q * 64 + l) * 16 bytes, so each of the wave's loads reads 1 KB in
// one piece (G = 4: lane l's 8 bytes at l * 8).
template <int G>
struct WRow {
  static_assert(G % 8 == 0 || G == 4, "16-byte weight loads (or 8)");
  static constexpr int N = G == 4 ? 1 : G / 8;
  v4u w[N];
  __device__ __forceinline__ void load(const uint16_t* W, int r, int lane) {
    const uint16_t* row = W + (int64_t)r * 64 * G;
    if constexpr (G == 4) {
      const uint2 u = reinterpret_cast<const uint2*>(row)[lane];
      w[0] = v4u{u.x, u.y, 0u, 0u};
    } else {
#pragma unroll
      for (int q = 0; q < N; q++) w[q] = reinterpret_cast<const v4u*>(row)[q * 64 + lane];
    }
  }
};
// The lane's share of the input (bf16-exact values) as bf16 pairs in registers: chunk q = the
// lane's entries 8q..8q+7 (G = 4: entries 0..3 in the first two words).
template <int G>
struct XRegs {
  static_assert(G % 4 == 0, "16-byte input loads");
  uint32_t v[G / 2 < 4 ? 4 : G / 2];
  // x[lane G .. lane G + G)
  __device__ __forceinline__ void load(const float* x, int lane) {
    if constexpr (G == 4) v[2] = v[3] = 0u;
    const v4f* src = reinterpret_cast<const v4f*>(x + lane * G);
    v4f a[G / 4];
#pragma unroll
    for (int k = 0; k < G / 4; k++) a[k] = src[k];
#pragma unroll
    for (int k = 0; k < G / 4; k++) {
      v[2 * k] = pack2(a[k].x, a[k].y);
      v[2 * k + 1] = pack2(a[k].z, a[k].w);
    }
  }
  // the norm's output over the lane's entries: D((h * r) * (1 + w))
  __device__ __forceinline__ void load_norm(const float* h, const float* nw, float r, int lane) {
    if constexpr (G == 4) v[2] = v[3] = 0u;
    const v4f* hs = reinterpret_cast<const v4f*>(h + lane * G);
    const v4f* ws = reinterpret_cast<const v4f*>(nw + lane * G);
    v4f a[G / 4], b[G / 4];
#pragma unroll
    for (int k = 0; k < G / 4; k++) {
      a[k] = hs[k];
      b[k] = ws[k];
    }
#pragma unroll
    for (int k = 0; k < G / 4; k++) {
      v[2 * k] = pack2(norm_el(a[k].x, r, b[k].x), norm_el(a[k].y, r, b[k].y));
      v[2 * k + 1] = pack2(norm_el(a[k].z, r, b[k].z), norm_el(a[k].w, r, b[k].w));
    }
  }
  __device__ __forceinline__ v4u chunk(int q) const {
    return v4u{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  }
};
// The lane's sum of its G entries, in order from +0 (bf16 x bf16 products are exact in fp32:
// one fused op per term)
template <int G, class X>
__device__ __forceinline__ float lane_dot(const WRow<G>& r, const X& x) {
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < WRow<G>::N; q++) {
    const v4u xx = x.chunk(q);
#pragma unroll
    for (int k = 0; k < (G == 4 ? 2 : 4); k++) {
      const uint32_t a = xx[k], b = r.w[q][k];
      s = __builtin_fmaf(bitsf(a << 16), bitsf(b << 16), s);
      s = __builtin_fmaf(bitsf(a & 0xffff0000u), bitsf(b & 0xffff0000u), s);
    }
  }
  return s;
}
// the row's sum in the dense order (lane 0 holds it)
template <int G, class X>
__device__ __forceinline__ float row_dot(const WRow<G>& r, const X& x) {
  return wave_tree(lane_dot<G>(r, x));
}

// Rows: out[r] = D(row . x) (MODE 0) or out[r] = D(out[r] + D(row . x)) (MODE 1, the residual).
// XS 0: x from a vector; 1: x = the RMSNorm of h with weight nw (hidden H; every workgroup forms
// it). NTB threads per workgroup. Each wave requests its first row before it forms x.
template <int G, int MODE, int XS, int NTB>
__global__ __launch_bounds__(NTB) void dn_rows(const uint16_t* __restrict__ W, int nrows,
                                               const float* __restrict__ x,
                                               const float* __restrict__ nw, float eps, int H,
                                               float* out) {
  static_assert(XS != 1 || NTB == NT, "the norm's 512-lane sum");
  constexpr int NWB = NTB / 64;
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NWB + (threadIdx.x >> 6), nwv = gridDim.x * NWB;
  WRow<G> cur;
  if (wv < nrows) cur.load(W, wv, lane);
  XRegs<G> xc;
  if constexpr (XS == 1) {
    __shared__ float wsum[NW];
    xc.load_norm(x, nw, norm_factor(x, H, eps, wsum), lane);
  } else {
    xc.load(x, lane);
  }
  for (int r = wv; r < nrows; r += nwv) {
    if (r != wv) cur.load(W, r, lane);
    const float s = row_dot<G>(cur, xc);
    if (lane == 0) {
      if constexpr (MODE == 0) out[r] = bf16r(s);
      else out[r] = bf16r(out[r] + bf16r(s));
    }
  }
}

// SwiGLU over the post norm of h: unit u's gate and up rows, act[u] = D(D(silu(D(g))) * D(u))
// (TF:704-717)
template <int G>
__global__ __launch_bounds__(NT) void dn_units(const uint16_t* __restrict__ Wg,
                                               const uint16_t* __restrict__ Wu, int nunits,
                                               const float* __restrict__ h,
                                               const float* __restrict__ nw, float eps, int H,
                                               float* act) {
  __shared__ float wsum[NW];
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NW + (threadIdx.x >> 6), nwv = gridDim.x * NW;
  WRow<G> cg, cu;
  if (wv < nunits) {
    cg.load(Wg, wv, lane);
    cu.load(Wu, wv, lane);
  }
  XRegs<G> xc;
  xc.load_norm(h, nw, norm_factor(h, H, eps, wsum), lane);
  for (int u = wv; u < nunits; u += nwv) {
    if (u != wv) {
      cg.load(Wg, u, lane);
      cu.load(Wu, u, lane);
    }
    const float g = row_dot<G>(cg, xc);
    const float v = row_dot<G>(cu, xc);
    if (lane == 0) act[u] = bf16r(silu_bf16(bf16r(g)) * bf16r(v));
  }
}

// The head over the final norm of h: logits D(row . x) over the vocabulary, the first maximum
// (ties to the lower index, NaN above everything: torch.argmax) folded into *keys by 64-bit
// atomic max. Each wave takes rows in ascending order and keeps its first strict maximum (and
// its first NaN apart).
template <int G>
__global__ __launch_bounds__(NT) void dn_head(const uint16_t* __restrict__ W, int nrows,
                                              const float* __restrict__ h,
                                              const float* __restrict__ nw, float eps, int H,
                                              unsigned long long* keys) {
  __shared__ float wsum[NW];
  const int lane = threadIdx.x & 63;
  const int wv = blockIdx.x * NW + (threadIdx.x >> 6), nwv = gridDim.x * NW;
  WRow<G> cur;
  if (wv < nrows) cur.load(W, wv, lane);
  XRegs<G> xc;
  xc.load_norm(h, nw, norm_factor(h, H, eps, wsum), lane);
  float best = 0.0f;
  int bidx = -1, nanr = -1;
  for (int r = wv; r < nrows; r += nwv) {
    if (r != wv) cur.load(W, r, lane);
    const float v = bf16r(row_dot<G>(cur, xc));
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
// The delta rule of one live value head (vslot = kh x rl + r; value head kh x R + r), split by
// state columns over QC workgroups (32 columns each): the key head's query and key (conv over
// the window [x(t-3), x(t-2), x(t-1), P], silu, TF:199-216; l2norm in the model dtype, the query
// times 1/16; every workgroup of the head forms them), the workgroup's values, beta = sigmoid(b),
// g = -exp(A_log) softplus(a + dt_bias) (:497-499), the recurrent step (TF:330-380) on its
// 256 x 32 tile in registers (thread = one column of one of ATen's 16-row cascade blocks), and
// o = D(S^T q) into on (0 for a head without a live query or key: the oracle's proc 1). The
// gated norm and the query/key windows' shift belong to the out_proj kernel.
#define QC 4
#define QW (VD / QC)
static_assert(NT == 16 * QW && NT >= KD + QW, "dn_gdn: one thread per (16-row block, column)");
struct DnGdn {
  const uint16_t* conv_qk;  // (2, nk, kl, 4)
  const uint16_t* conv_v;   // (nk, rl, 128, 4)
  const float* A_log;
  const float* dt_bias;
  float* rec;
  uint16_t* conv;           // the windows (the value channels' advance here)
  const float* P;
  float* on;
  int nk, kl, rl, R;
};
__device__ __forceinline__ float conv_y(const uint16_t* cs, int64_t chan, const uint16_t* taps, float P) {
  float y = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float x = k < 3 ? bf16f(cs[chan * 4 + k + 1]) : P;
    y = __builtin_fmaf(bf16f(taps[k]), x, y);
  }
  return silu_bf16(bf16r(y));
}
__global__ __launch_bounds__(NT) void dn_gdn(DnGdn g) {
  __shared__ __align__(16) float qd[KD], kd_[KD], qn[KD], kn[KD], vb[QW], dl[QW];
  __shared__ __align__(16) float bs[16 * QW];
  __shared__ float misc[4];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nk = g.nk, kl = g.kl, rl = g.rl;
  const int vslot = blockIdx.x / QC, c0 = (blockIdx.x % QC) * QW;
  const int kh = vslot / rl, vh = kh * g.R + vslot % rl;
  const int nq = nk * kl, nvr = nk * rl * VD;
  const float* P = g.P;
  // the state tile first (its loads overlap the inputs' work below): column c0 + c of rows
  // 16 rb .. 16 rb + 15
  const int c = t % QW, rb = t / QW;
  float* S = g.rec + (size_t)vh * KD * VD + c0 + c;
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; i++) s[i] = S[(rb * 16 + i) * VD];
  // rows of P: q [0, nq), k [nq, 2nq), v [2nq, 2nq + nvr), z [.., + nvr), b [.., + nk rl), a
  if (t < KD) {
    float q = 0.0f, k = 0.0f;
    if (t < kl) {
      const int64_t cq = (int64_t)kh * KD + t, ck = (int64_t)nk * KD + kh * KD + t;
      q = conv_y(g.conv, cq, g.conv_qk + ((int64_t)kh * kl + t) * 4, P[kh * kl + t]);
      k = conv_y(g.conv, ck, g.conv_qk + ((int64_t)(nk + kh) * kl + t) * 4, P[nq + kh * kl + t]);
    }
    qd[t] = q;
    kd_[t] = k;
  } else if (t < KD + QW) {
    // the workgroup's value channels: no other workgroup reads their windows, so they advance
    // here (causal_conv1d_update's shift: [x(t-2), x(t-1), P] behind the oldest)
    const int d = c0 + t - KD;
    const int64_t ch = 2 * (int64_t)nk * KD + (int64_t)vh * VD + d;
    const float pv = P[2 * nq + vslot * VD + d];
    vb[t - KD] = conv_y(g.conv, ch, g.conv_v + ((int64_t)vslot * VD + d) * 4, pv);
    uint16_t* w = g.conv + ch * 4;
    const uint16_t w1 = w[1], w2 = w[2], w3 = w[3];
    w[0] = w1;
    w[1] = w2;
    w[2] = w3;
    w[3] = (uint16_t)(fbits(pv) >> 16);
  }
  if (t == 0) {
    const float b = P[2 * nq + 2 * nvr + vslot], a = P[2 * nq + 2 * nvr + nk * rl + vslot];
    misc[0] = bf16r(sigmoid(b));
    misc[1] = cr_exp((-cr_exp(g.A_log[vh])) * softplus(a + g.dt_bias[vh]));
  }
  __syncthreads();
  // l2norm of the query (wave 0) and key (wave 1) in the model dtype; live: any nonzero
  if (wv < 2) {
    const float* x = wv ? kd_ : qd;
    float* o = wv ? kn : qn;
    float xs[4], ss = 0.0f;
    bool nz = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xs[i] = x[lane + 64 * i];
      nz |= xs[i] != 0.0f;
      ss = ss + bf16r(xs[i] * xs[i]);
    }
    if (lane == 0) misc[2 + wv] = __ballot(nz) != 0ull ? 1.0f : 0.0f;
    ss = bf16r(sum64(ss));
    const float inv = bf16r(rsqrt_(bf16r(ss + 1e-6f)));
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
  float* o_out = g.on + vslot * VD + c0;
  if (live) {
    float kr[16], qr[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      kr[i] = kn[rb * 16 + i];
      qr[i] = qn[rb * 16 + i];
    }
    // kv = S^T k: the block's rows in order (a zero factor adds nothing), then the 16 blocks
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) a = kr[i] != 0.0f ? a + s[i] * kr[i] : a;
    bs[rb * QW + c] = a;
    __syncthreads();
    if (t < QW) {
      float kv = 0.0f;
#pragma unroll
      for (int q = 0; q < 16; q++) kv = kv + bs[q * QW + t];
      dl[t] = (vb[t] - kv) * beta;
    }
    __syncthreads();
    const float d = dl[c];
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      // (rows with a zero key factor keep their state exactly: -0 stays -0)
      s[i] = kr[i] != 0.0f ? s[i] + kr[i] * d : s[i];
      o = qr[i] != 0.0f ? o + s[i] * qr[i] : o;
    }
    bs[rb * QW + c] = o;
    __syncthreads();
    if (t < QW) {
      float q = 0.0f;
#pragma unroll
      for (int b = 0; b < 16; b++) q = q + bs[b * QW + t];
      o_out[t] = bf16r(q);
    }
  } else if (t < QW) {
    o_out[t] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 16; i++) S[(rb * 16 + i) * VD] = s[i];
}

// ---------------------------------------------------------------------------------------------
// out_proj and the residual, after the delta rule: every workgroup forms the gated norm of the
// live heads (TF:168-184: y = D(D(w * D(o * r)) * silu(z)), r = rsqrt(mean(o^2) + eps), the
// squares summed per lane over dims lane, lane + 64 and then by the pairwise tree; one wave per
// head) into LDS, then h[r] = D(h[r] + D(row . y)) for its rows. Then the workgroups advance the
// windows of the live query/key channels (every key head's live dims), which the delta rule has
// read (causal_conv1d_update's shift: [x(t-2), x(t-1), P] behind the oldest).
struct DnOut {
  const uint16_t* W;  // (hidden, nh x 128), interleaved
  int nrows, nh;
  const float* on;    // (nh x 128): o
  const float* z;     // (nh x 128): in_proj_z's rows of P
  const float* gw;    // (128)
  float geps;
  float* h;
  uint16_t* conv;
  const float* P;
  int nk, kl;
};
template <int G, int NTB>
__global__ __launch_bounds__(NTB) void dn_out(DnOut a) {
  static_assert(G * 64 <= 4096, "dn_out: at most 32 value heads");
  constexpr int NWB = NTB / 64;
  __shared__ __align__(16) float ys[G * 64];
  const int t = threadIdx.x, lane = t & 63, wvl = t >> 6;
  const int wv = blockIdx.x * NWB + wvl, nwv = gridDim.x * NWB;
  WRow<G> cur;
  if (wv < a.nrows) cur.load(a.W, wv, lane);
  // the wave's heads wvl, wvl + NWB, ...: every input requested first, then the norms
  constexpr int HPW = (4096 / VD + NWB - 1) / NWB;
  const float g0 = a.gw[lane], g1 = a.gw[lane + 64];
  float o[HPW][2], z[HPW][2];
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int hh = wvl + j * NWB;
    if (hh < a.nh) {
      o[j][0] = a.on[hh * VD + lane];
      o[j][1] = a.on[hh * VD + lane + 64];
      z[j][0] = a.z[hh * VD + lane];
      z[j][1] = a.z[hh * VD + lane + 64];
    }
  }
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int hh = wvl + j * NWB;
    if (hh < a.nh) {
      float ss = 0.0f;
      ss = ss + o[j][0] * o[j][0];
      ss = ss + o[j][1] * o[j][1];
      ss = sum64(ss);
      const float rr = rsqrt_(ss / (float)VD + a.geps);
      ys[hh * VD + lane] = bf16r(bf16r(g0 * bf16r(o[j][0] * rr)) * silu(z[j][0]));
      ys[hh * VD + lane + 64] = bf16r(bf16r(g1 * bf16r(o[j][1] * rr)) * silu(z[j][1]));
    }
  }
  lds_barrier();
  XRegs<G> xc;
  xc.load(ys, lane);
  for (int r = wv; r < a.nrows; r += nwv) {
    if (r != wv) cur.load(a.W, r, lane);
    const float s = row_dot<G>(cur, xc);
    if (lane == 0) a.h[r] = bf16r(a.h[r] + bf16r(s));
  }
  // the query/key windows, spread over the workgroups (channel i: workgroup i % grid)
  const int nq = a.nk * a.kl;
  for (int i = blockIdx.x + gridDim.x * t; i < 2 * nq; i += gridDim.x * NTB) {
    const int part = i / nq, j = i % nq, kh = j / a.kl, d = j % a.kl;
    uint16_t* w = a.conv + ((int64_t)part * a.nk * KD + kh * KD + d) * 4;
    const uint16_t w1 = w[1], w2 = w[2], w3 = w[3];
    w[0] = w1;
    w[1] = w2;
    w[2] = w3;
    w[3] = (uint16_t)(fbits(a.P[i]) >> 16);
  }
}

// ---------------------------------------------------------------------------------------------
// Host side. Launch shapes (measured on MI355X over these matrices): the hidden rows (out_proj,
// down_proj: few long rows) in 4-wave workgroups, one per CU, each wave taking rows in turn;
// the wide sets (projections, SwiGLU units, the head) in 8-wave workgroups, two per CU.
#define NTL 256
static int grid_for(int nrows, int ntb, int cap) {
  const int w = ntb / 64, g = (nrows + w - 1) / w;
  return g < cap ? g : cap;
}
#define CAP_L 256
#define CAP_W 512

// G (entries per lane) of a supported row length K
static int g_of(int K) {
  switch (K) {
    case 256: return 4;
    case 512: return 8;
    case 2560: return 40;
    case 4096: return 64;
    case 9216: return 144;
    default: return 0;
  }
}

template <int G, int MODE, int XS, int NTB>
static void launch_rows(const uint16_t* W, int nrows, const float* x, const float* nw, float eps,
                        int H, float* out, hipStream_t st) {
  hipLaunchKernelGGL((dn_rows<G, MODE, XS, NTB>), dim3(grid_for(nrows, NTB, NTB == NTL ? CAP_L : CAP_W)),
                     dim3(NTB), 0, st, W, nrows, x, nw, eps, H, out);
}
// the residual's rows: x from a vector (in LDS for the longest rows)
static bool res_rows(int K, const uint16_t* W, int nrows, const float* x, float* out,
                     hipStream_t st) {
  switch (g_of(K)) {
    case 4: launch_rows<4, 1, 0, NTL>(W, nrows, x, nullptr, 0.0f, 0, out, st); return true;
    case 8: launch_rows<8, 1, 0, NTL>(W, nrows, x, nullptr, 0.0f, 0, out, st); return true;
    case 40: launch_rows<40, 1, 0, NTL>(W, nrows, x, nullptr, 0.0f, 0, out, st); return true;
    case 64: launch_rows<64, 1, 0, NTL>(W, nrows, x, nullptr, 0.0f, 0, out, st); return true;
    case 144: launch_rows<144, 1, 0, NTL>(W, nrows, x, nullptr, 0.0f, 0, out, st); return true;
    default: return false;
  }
}
// rows over the RMSNorm of h (K = hidden)
static bool norm_rows(int K, const uint16_t* W, int nrows, const float* h, const float* nw,
                      float eps, float* out, hipStream_t st) {
  switch (g_of(K)) {
    case 4: launch_rows<4, 0, 1, NT>(W, nrows, h, nw, eps, K, out, st); return true;
    case 40: launch_rows<40, 0, 1, NT>(W, nrows, h, nw, eps, K, out, st); return true;
    default: return false;
  }
}
template <int G>
static void launch_units(const uint16_t* Wg, const uint16_t* Wu, int n, const float* h,
                         const float* nw, float eps, int K, float* act, hipStream_t st) {
  const dim3 g(grid_for(n, NT, CAP_W));
  hipLaunchKernelGGL(dn_units<G>, g, dim3(NT), 0, st, Wg, Wu, n, h, nw, eps, K, act);
}
static bool units(int K, const uint16_t* Wg, const uint16_t* Wu, int n, const float* h,
                  const float* nw, float eps, float* act, hipStream_t st) {
  switch (g_of(K)) {
    case 4: launch_units<4>(Wg, Wu, n, h, nw, eps, K, act, st); return true;
    case 40: launch_units<40>(Wg, Wu, n, h, nw, eps, K, act, st); return true;
    default: return false;
  }
}
template <int G>
static void launch_head(const uint16_t* W, int n, const float* h, const float* nw, float eps,
                        int K, unsigned long long* keys, hipStream_t st) {
  const dim3 g(grid_for(n, NT, CAP_W));
  hipLaunchKernelGGL(dn_head<G>, g, dim3(NT), 0, st, W, n, h, nw, eps, K, keys);
}
static bool head(int K, const uint16_t* W, int n, const float* h, const float* nw, float eps,
                 unsigned long long* keys, hipStream_t st) {
  switch (g_of(K)) {
    case 4: launch_head<4>(W, n, h, nw, eps, K, keys, st); return true;
    case 40: launch_head<40>(W, n, h, nw, eps, K, keys, st); return true;
    default: return false;
  }
}
static bool out_proj(int K, const DnOut& a, hipStream_t st) {
  const dim3 g(grid_for(a.nrows, NTL, CAP_L)), b(NTL);
  switch (g_of(K)) {
    case 8: hipLaunchKernelGGL((dn_out<8, NTL>), g, b, 0, st, a); return true;
    case 64: hipLaunchKernelGGL((dn_out<64, NTL>), g, b, 0, st, a); return true;
    default: return false;
  }
}

extern "C" int lxm_dn_step(const lxm_dn_params* ph, const lxm_dn_params* pd, void* stream) {
  if (!ph || ph->hidden <= 0 || ph->hidden > 4096 || ph->kl > KD || ph->nv % ph->nk ||
      ph->nk * ph->rl > 32 || !ph->layers || !ph->layers_host)
    return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  const int H = ph->hidden, I = ph->inter, nk = ph->nk, kl = ph->kl, rl = ph->rl;
  const int nq = nk * kl, nvr = nk * rl * VD, nproj = 2 * nq + 2 * nvr + 2 * nk * rl;
  const float eps = ph->rms_eps;
  float* act = ph->xn + H;
  hipLaunchKernelGGL(dn_embed, dim3(1), dim3(NT), 0, st, pd);
  for (int L = 0; L < ph->n_layers; L++) {
    // every kernel takes its pointers as arguments (from the host copy of the table)
    const lxm_dn_layer& ly = ph->layers_host[L];
    if (!norm_rows(H, ly.proj, nproj, ph->h, ly.ln_in, eps, ph->P, st)) return (int)hipErrorInvalidValue;
    const DnGdn g{ly.conv_qk, ly.conv_v, ly.A_log, ly.dt_bias, ly.rec, ly.conv, ph->P, ph->on,
                  nk, kl, rl, ph->nv / nk};
    hipLaunchKernelGGL(dn_gdn, dim3(nk * rl * QC), dim3(NT), 0, st, g);
    const DnOut o{ly.out, H, nk * rl, ph->on, ph->P + 2 * nq + nvr, ly.gnorm, ph->geps, ph->h,
                  ly.conv, ph->P, nk, kl};
    if (!out_proj(nvr, o, st)) return (int)hipErrorInvalidValue;
    if (!units(H, ly.gate, ly.up, I, ph->h, ly.ln_post, eps, act, st)) return (int)hipErrorInvalidValue;
    if (!res_rows(I, ly.down, H, act, ph->h, st)) return (int)hipErrorInvalidValue;
  }
  if (!head(H, ph->embed, ph->vocab, ph->h, ph->w_final, eps, ph->keys, st)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(dn_next, dim3(1), dim3(64), 0, st, pd);
  return (int)hipGetLastError();
}
