// Greedy decode of the dense padded text-view stack (benchmark config 4) on MI355X (gfx950).
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
//
// Two drivers share the row sums and the delta rule below: lxm_dn_step (one step as five kernels
// per layer, for a caller that captures it in a graph) and lxm_dn_run (n steps in one persistent
// launch: one workgroup per CU, the phases separated by grid barriers; the vectors that cross
// workgroups move through agent-scope loads and stores; a control wave per workgroup polls the
// barriers and stages each phase's input while seven stream waves hold the next phase's weight
// rows in flight).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lxm_chunk.h"
#include "../../include/lxm_dense.h"
#include "lxm_math.h"
#include "lxm_sync.h"

using namespace lxm;

#define NT 512
#define NW (NT / 64)
#define KD 256
#define VD 128
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// The thread index, opaque to the compiler: values computed from it stay where they are used
// instead of being hoisted out of the persistent run's step and layer loops (where they would
// hold registers across every phase).
__device__ __forceinline__ int tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
// the wave's index in the workgroup, in a scalar register
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(tid() >> 6); }

// Vector accesses: COH = the data crosses workgroups inside one launch (agent-scope, coherent
// across the XCDs); otherwise plain (a kernel boundary orders them).
template <bool COH>
__device__ __forceinline__ float ldf(const float* p) {
  if constexpr (COH) return ld_rlxf(p);
  else return *p;
}
template <bool COH>
__device__ __forceinline__ void stf(float* p, float v) {
  if constexpr (COH) st_rlxf(p, v);
  else *p = v;
}
// 16 bytes at base[idx] (base uniform over the wave)
template <bool COH>
__device__ __forceinline__ v4f ldf4(const float* base, int idx) {
  if constexpr (COH) return ld4_rlx(wave_ptr(const_cast<float*>(base)), idx);
  else return *reinterpret_cast<const v4f*>(base + idx);
}
// a channel's window (4 bf16 values, 8 bytes)
template <bool COH>
__device__ __forceinline__ uint64_t ldw(const uint16_t* w) {
  if constexpr (COH) {
    return __hip_atomic_load(gp(reinterpret_cast<const uint64_t*>(w)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  } else {
    return *reinterpret_cast<const uint64_t*>(w);
  }
}
template <bool COH>
__device__ __forceinline__ void stw(uint16_t* w, uint64_t v) {
  if constexpr (COH) {
    __hip_atomic_store(gp(reinterpret_cast<uint64_t*>(w)), v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<uint64_t*>(w) = v;
  }
}
// causal_conv1d_update's shift: [x(t-2), x(t-1), P] behind the oldest (tap k at bits 16k)
__device__ __forceinline__ uint64_t shifted(uint64_t w, float p) {
  return (w >> 16) | ((uint64_t)(fbits(p) >> 16) << 48);
}

// ---------------------------------------------------------------------------------------------
// The 512-lane hidden sum of x * x over n <= 4096 values (thread t: its values 4t..4t+3, then
// 2048+4t..2048+4t+3; waves at offsets 32..1; the 8 wave totals at offsets 4, 2, 1).
template <bool COH>
__device__ __forceinline__ float hidden_sum(const float* x, int n, float* wsum) {
  const int t = tid();
  float s = 0.0f;
#pragma unroll
  for (int half = 0; half < 2; half++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = half * 2048 + 4 * t + i;
      if (c < n) {
        const float v = ldf<COH>(x + c);
        s = acc<true>(s, v, v);
      }
    }
  s = wave_tree(s);
  if ((t & 63) == 0) wsum[t >> 6] = s;
  lds_barrier();  // (weight rows already requested stay in flight)
  float w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
  lds_barrier();  // (wsum is free again)
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
    if (tid() == 0) *p.err = 1;
    tok = 0;
  }
  const uint16_t* e = p.embed + (int64_t)tok * p.hidden;
  const int G = p.hidden / 64;
  for (int c = tid(); c < p.hidden; c += NT) {
    // entry c is lane c / G's entry c % G (interleaved in 8-entry chunks when G >= 8)
    const int l = c / G, k = c % G;
    const int at = G < 8 ? c : ((k >> 3) * 64 + l) * 8 + (k & 7);
    p.h[c] = bf16f(e[at]);
  }
  if (tid() == 0) *p.keys = 0ull;
}

// The RMSNorm factor r = rsqrt(mean(h^2) + eps) of TF:720-737, computed by every workgroup that
// consumes the norm (the sum in the 512-lane order above); x[c] = D((h[c] * r) * (1 + w[c])).
template <bool COH>
__device__ __forceinline__ float norm_factor(const float* h, int H, float eps, float* wsum) {
  return rsqrt_(hidden_sum<COH>(h, H, wsum) / (float)H + eps);
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
  // (global loads: a flat load would also count against the LDS counter, and an LDS barrier
  // would then wait for the rows in flight)
  __device__ __forceinline__ void load(const uint16_t* W, int r, int lane) {
    const uint16_t* row = W + (int64_t)r * 64 * G;
    if constexpr (G == 4) {
      typedef uint32_t v2u __attribute__((ext_vector_type(2)));
      const v2u u = gp(reinterpret_cast<const v2u*>(row))[lane];
      w[0] = v4u{u.x, u.y, 0u, 0u};
    } else {
#pragma unroll
      for (int q = 0; q < N; q++) w[q] = gp(reinterpret_cast<const v4u*>(row))[q * 64 + lane];
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
  // (in pieces of 16 values: the unpacked floats would crowd out the weights in flight)
  template <bool COH>
  __device__ __forceinline__ void load(const float* x, int lane) {
    if constexpr (G == 4) v[2] = v[3] = 0u;
    constexpr int PC = G / 4 < 4 ? G / 4 : 4;
#pragma unroll
    for (int k0 = 0; k0 < G / 4; k0 += PC) {
      v4f a[PC];
#pragma unroll
      for (int k = 0; k < PC; k++) a[k] = ldf4<COH>(x, lane * G + 4 * (k0 + k));
#pragma unroll
      for (int k = 0; k < PC; k++) {
        v[2 * (k0 + k)] = pack2(a[k].x, a[k].y);
        v[2 * (k0 + k) + 1] = pack2(a[k].z, a[k].w);
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
  }
  // the norm's output over the lane's entries: D((h * r) * (1 + w)) (in pieces, as load)
  template <bool COH>
  __device__ __forceinline__ void load_norm(const float* h, const float* nw, float r, int lane) {
    if constexpr (G == 4) v[2] = v[3] = 0u;
    const v4f* ws = reinterpret_cast<const v4f*>(nw + lane * G);
    constexpr int PC = G / 4 < 4 ? G / 4 : 4;
#pragma unroll
    for (int k0 = 0; k0 < G / 4; k0 += PC) {
      v4f a[PC], b[PC];
#pragma unroll
      for (int k = 0; k < PC; k++) {
        a[k] = ldf4<COH>(h, lane * G + 4 * (k0 + k));
        b[k] = ws[k0 + k];
      }
#pragma unroll
      for (int k = 0; k < PC; k++) {
        v[2 * (k0 + k)] = pack2(norm_el(a[k].x, r, b[k].x), norm_el(a[k].y, r, b[k].y));
        v[2 * (k0 + k) + 1] = pack2(norm_el(a[k].z, r, b[k].z), norm_el(a[k].w, r, b[k].w));
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
  }
  __device__ __forceinline__ v4u chunk(int q) const {
    return v4u{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  }
};
// The same input staged in LDS in the weights' interleaved order (chunk q of lane l at q * 64 +
// l), for the longest rows: the registers then hold the weights in flight instead.
template <int G>
struct XLds {
  static_assert(G % 8 == 0, "16-byte chunks");
  const v4u* xs;
  int lane;
  // every thread of the workgroup: x (64 G values) into xs
  template <bool COH>
  __device__ __forceinline__ static void stage(v4u* xs, const float* x) {
    for (int c8 = tid(); c8 < 8 * G; c8 += blockDim.x) {
      const int l = c8 / (G / 8), q = c8 % (G / 8);
      const v4f a = ldf4<COH>(x, 8 * c8), b = ldf4<COH>(x, 8 * c8 + 4);
      xs[q * 64 + l] = v4u{pack2(a.x, a.y), pack2(a.z, a.w), pack2(b.x, b.y), pack2(b.z, b.w)};
    }
  }
  __device__ __forceinline__ v4u chunk(int q) const { return xs[q * 64 + lane]; }
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

// A wave's rows: w0, then in round j >= 1 row j nw + (w0 + rot) % nw (rot 0: w0 + j nw), so a
// phase's rows past the first nw go to the waves rot places on (cur holds row w0, requested
// earlier). MODE 0 out[r] = D(row . x); MODE 1 out[r] = D(out[r] + D(row . x)) (the residual).
__device__ __forceinline__ int round_row(int w0, int j, int nw, int rot) {
  return j == 0 ? w0 : j * nw + (w0 + rot) % nw;
}
template <int G, int MODE, bool COH, class X>
__device__ __forceinline__ void rows_run(const uint16_t* W, int nrows, const X& xc, WRow<G>& cur,
                                         int w0, int nw, float* out, int rot = 0) {
  const int lane = tid() & 63;
  for (int j = 0;; j++) {
    const int r = round_row(w0, j, nw, rot);
    if (r >= nrows) break;
    if (j) cur.load(W, r, lane);
    const float s = row_dot<G, X>(cur, xc);
    if (lane == 0) {
      if constexpr (MODE == 0) stf<COH>(out + r, bf16r(s));
      else stf<COH>(out + r, bf16r(ldf<COH>(out + r) + bf16r(s)));
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // (the next row's loads stay after this one's sums)
  }
}
// SwiGLU units, dealt as rows_run deals rows (cg / cu hold unit w0's gate and up rows): act[u]
// = D(D(silu(D(g))) * D(u)) (TF:704-717)
template <int G, bool COH>
__device__ __forceinline__ void units_run(const uint16_t* Wg, const uint16_t* Wu, int nunits,
                                          const XRegs<G>& xc, WRow<G>& cg, WRow<G>& cu, int w0,
                                          int nw, float* act, int rot = 0) {
  const int lane = tid() & 63;
  for (int j = 0;; j++) {
    const int u = round_row(w0, j, nw, rot);
    if (u >= nunits) break;
    if (j) {
      cg.load(Wg, u, lane);
      cu.load(Wu, u, lane);
    }
    const float g = row_dot<G>(cg, xc);
    const float v = row_dot<G>(cu, xc);
    if (lane == 0) stf<COH>(act + u, bf16r(silu_bf16(bf16r(g)) * bf16r(v)));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }
}
// The head's rows r = w0, w0 + nw, ...: logits D(row . x), the wave's first maximum (ties to the
// lower index, NaN above everything: torch.argmax) folded into *keys by 64-bit atomic max. Each
// wave takes rows in ascending order and keeps its first strict maximum (and its first NaN apart).
template <int G>
__device__ __forceinline__ void head_run(const uint16_t* W, int nrows, const XRegs<G>& xc,
                                         WRow<G>& cur, int w0, int nw, unsigned long long* keys) {
  const int lane = tid() & 63;
  float best = 0.0f;
  int bidx = -1, nanr = -1;
  for (int r = w0; r < nrows; r += nw) {
    if (r != w0) cur.load(W, r, lane);
    const float v = bf16r(row_dot<G>(cur, xc));
    if (v != v) {
      if (nanr < 0) nanr = r;
    } else if (bidx < 0 || v > best) {
      best = v;
      bidx = r;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
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
  const int lane = tid() & 63;
  const int wv = blockIdx.x * NWB + (tid() >> 6), nwv = gridDim.x * NWB;
  WRow<G> cur;
  if (wv < nrows) cur.load(W, wv, lane);
  XRegs<G> xc;
  if constexpr (XS == 1) {
    __shared__ float wsum[NW];
    xc.template load_norm<false>(x, nw, norm_factor<false>(x, H, eps, wsum), lane);
  } else {
    xc.template load<false>(x, lane);
  }
  rows_run<G, MODE, false>(W, nrows, xc, cur, wv, nwv, out);
}

// SwiGLU over the post norm of h
template <int G>
__global__ __launch_bounds__(NT) void dn_units(const uint16_t* __restrict__ Wg,
                                               const uint16_t* __restrict__ Wu, int nunits,
                                               const float* __restrict__ h,
                                               const float* __restrict__ nw, float eps, int H,
                                               float* act) {
  __shared__ float wsum[NW];
  const int lane = tid() & 63;
  const int wv = blockIdx.x * NW + (tid() >> 6), nwv = gridDim.x * NW;
  WRow<G> cg, cu;
  if (wv < nunits) {
    cg.load(Wg, wv, lane);
    cu.load(Wu, wv, lane);
  }
  XRegs<G> xc;
  xc.template load_norm<false>(h, nw, norm_factor<false>(h, H, eps, wsum), lane);
  units_run<G, false>(Wg, Wu, nunits, xc, cg, cu, wv, nwv, act);
}

// The head over the final norm of h
template <int G>
__global__ __launch_bounds__(NT) void dn_head(const uint16_t* __restrict__ W, int nrows,
                                              const float* __restrict__ h,
                                              const float* __restrict__ nw, float eps, int H,
                                              unsigned long long* keys) {
  __shared__ float wsum[NW];
  const int lane = tid() & 63;
  const int wv = blockIdx.x * NW + (tid() >> 6), nwv = gridDim.x * NW;
  WRow<G> cur;
  if (wv < nrows) cur.load(W, wv, lane);
  XRegs<G> xc;
  xc.template load_norm<false>(h, nw, norm_factor<false>(h, H, eps, wsum), lane);
  head_run<G>(W, nrows, xc, cur, wv, nwv, keys);
}

// the prediction, fed back; the step advanced
__global__ void dn_next(const lxm_dn_params* __restrict__ pp) {
  const lxm_dn_params& p = *pp;
  if (tid() == 0) {
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
// gated norm and the query/key windows' shift belong to the out_proj phase.
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
struct GdnLds {
  float qd[KD], kd[KD], qn[KD], kn[KD], vb[QW], dl[QW], bs[16 * QW];
  float misc[4];
};
// (the channel's four bf16 taps as one 8-byte word, tap k in bits 16k.., requested by the caller
// with the window and the input, so that the three loads are waited for together)
__device__ __forceinline__ uint64_t taps_of(const uint16_t* taps) {
  return *gp(reinterpret_cast<const uint64_t*>(taps));
}
__device__ __forceinline__ float conv_y(uint64_t win, uint64_t taps, float P) {
  float y = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float x = k < 3 ? bf16f((uint32_t)(win >> (16 * (k + 1))) & 0xffffu) : P;
    y = __builtin_fmaf(bf16f((uint32_t)(taps >> (16 * k)) & 0xffffu), x, y);
  }
  return silu_bf16(bf16r(y));
}
// the thread's 16 state values: column c0 + t % 32 of rows 16 (t / 32) .. + 15 of value head vh
__device__ __forceinline__ float* gdn_tile(const DnGdn& g, int blk) {
  const int t = tid(), vslot = blk / QC, c0 = (blk % QC) * QW;
  const int vh = (vslot / g.rl) * g.R + vslot % g.rl;
  return g.rec + (size_t)vh * KD * VD + c0 + t % QW + (t / QW) * 16 * VD;
}
template <bool COH>
__device__ __forceinline__ void gdn_load(const DnGdn& g, int blk, float (&s)[16]) {
  const float* S = gdn_tile(g, blk);
#pragma unroll
  for (int i = 0; i < 16; i++) s[i] = ldf<COH>(S + i * VD);
}
template <bool COH>
__device__ __forceinline__ void gdn_body(const DnGdn& g, int blk, float (&s)[16], GdnLds& l) {
  const int t = tid(), lane = t & 63, wv = t >> 6;
  const int nk = g.nk, kl = g.kl, rl = g.rl;
  const int vslot = blk / QC, c0 = (blk % QC) * QW;
  const int kh = vslot / rl, vh = kh * g.R + vslot % rl;
  const int nq = nk * kl, nvr = nk * rl * VD;
  const float* P = g.P;
  const int c = t % QW, rb = t / QW;
  // rows of P: q [0, nq), k [nq, 2nq), v [2nq, 2nq + nvr), z [.., + nvr), b [.., + nk rl), a
  if (t < KD) {
    float q = 0.0f, k = 0.0f;
    if (t < kl) {
      const int64_t cq = (int64_t)kh * KD + t, ck = (int64_t)nk * KD + kh * KD + t;
      const uint64_t wq = ldw<COH>(g.conv + cq * 4), wk = ldw<COH>(g.conv + ck * 4);
      const uint64_t tq = taps_of(g.conv_qk + ((int64_t)kh * kl + t) * 4);
      const uint64_t tk = taps_of(g.conv_qk + ((int64_t)(nk + kh) * kl + t) * 4);
      const float pq = ldf<COH>(P + kh * kl + t), pk = ldf<COH>(P + nq + kh * kl + t);
      q = conv_y(wq, tq, pq);
      k = conv_y(wk, tk, pk);
    }
    l.qd[t] = q;
    l.kd[t] = k;
  } else if (t < KD + QW) {
    // the workgroup's value channels: no other workgroup reads their windows, so they advance
    // here (causal_conv1d_update's shift)
    const int d = c0 + t - KD;
    uint16_t* w = g.conv + (2 * (int64_t)nk * KD + (int64_t)vh * VD + d) * 4;
    const float pv = ldf<COH>(P + 2 * nq + vslot * VD + d);
    const uint64_t win = ldw<COH>(w);
    const uint64_t tv = taps_of(g.conv_v + ((int64_t)vslot * VD + d) * 4);
    l.vb[t - KD] = conv_y(win, tv, pv);
    stw<COH>(w, shifted(win, pv));
  }
  if (t == 0) {
    // (the four loads requested before any is used)
    const float b = ldf<COH>(P + 2 * nq + 2 * nvr + vslot);
    const float a = ldf<COH>(P + 2 * nq + 2 * nvr + nk * rl + vslot);
    const float al = *gp(g.A_log + vh), dtb = *gp(g.dt_bias + vh);
    l.misc[0] = bf16r(sigmoid(b));
    l.misc[1] = cr_exp((-cr_exp(al)) * softplus(a + dtb));
  }
  lds_barrier();
  // l2norm of the query (wave 0) and key (wave 1) in the model dtype; live: any nonzero
  if (wv < 2) {
    const float* x = wv ? l.kd : l.qd;
    float* o = wv ? l.kn : l.qn;
    float xs[4], ss = 0.0f;
    bool nz = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xs[i] = x[lane + 64 * i];
      nz |= xs[i] != 0.0f;
      ss = ss + bf16r(xs[i] * xs[i]);
    }
    if (lane == 0) l.misc[2 + wv] = __ballot(nz) != 0ull ? 1.0f : 0.0f;
    ss = bf16r(sum64(ss));
    const float inv = bf16r(rsqrt_(bf16r(ss + 1e-6f)));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v = bf16r(xs[i] * inv);
      if (!wv) v = v * 0.0625f;
      o[lane + 64 * i] = v;
    }
  }
  lds_barrier();
  const float beta = l.misc[0], e = l.misc[1];
  const bool live = l.misc[2] != 0.0f || l.misc[3] != 0.0f;
  if (e != 1.0f) {
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = s[i] * e;
  }
  float* o_out = g.on + vslot * VD + c0;
  if (live) {
    const float* kr = l.kn + rb * 16;
    const float* qr = l.qn + rb * 16;
    // kv = S^T k: the block's rows in order (a zero factor adds nothing), then the 16 blocks
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) a = kr[i] != 0.0f ? a + s[i] * kr[i] : a;
    l.bs[rb * QW + c] = a;
    lds_barrier();
    if (t < QW) {
      float kv = 0.0f;
#pragma unroll
      for (int q = 0; q < 16; q++) kv = kv + l.bs[q * QW + t];
      l.dl[t] = (l.vb[t] - kv) * beta;
    }
    lds_barrier();
    const float d = l.dl[c];
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      // (rows with a zero key factor keep their state exactly: -0 stays -0)
      s[i] = kr[i] != 0.0f ? s[i] + kr[i] * d : s[i];
      o = qr[i] != 0.0f ? o + s[i] * qr[i] : o;
    }
    l.bs[rb * QW + c] = o;
    lds_barrier();
    if (t < QW) {
      float q = 0.0f;
#pragma unroll
      for (int b = 0; b < 16; b++) q = q + l.bs[b * QW + t];
      stf<COH>(o_out + t, bf16r(q));
    }
  } else if (t < QW) {
    stf<COH>(o_out + t, 0.0f);
  }
  float* S = gdn_tile(g, blk);
#pragma unroll
  for (int i = 0; i < 16; i++) stf<COH>(S + i * VD, s[i]);
  lds_barrier();  // (the scratch is free for the next use)
}
__global__ __launch_bounds__(NT) void dn_gdn(DnGdn g) {
  __shared__ GdnLds l;
  float s[16];
  gdn_load<false>(g, blockIdx.x, s);  // the state tile first: its loads overlap the inputs' work
  gdn_body<false>(g, blockIdx.x, s, l);
}

// ---------------------------------------------------------------------------------------------
// out_proj and the residual, after the delta rule: every workgroup forms the gated norm of the
// live heads (TF:168-184: y = D(D(w * D(o * r)) * silu(z)), r = rsqrt(mean(o^2) + eps), the
// squares summed per lane over dims lane, lane + 64 and then by the pairwise tree; one wave per
// head) into LDS, then h[r] = D(h[r] + D(row . y)) for its rows. Then the workgroups advance the
// windows of the live query/key channels (every key head's live dims), which the delta rule has
// read (causal_conv1d_update's shift).
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
// the gated norm of every live head into ys (nh x 128), the NWB waves taking heads in turn (SZ:
// a.z holds silu(z) already, fp32, as the persistent run's projections store it)
template <int NWB, bool COH, bool SZ = false>
__device__ __forceinline__ void gated_norm(const DnOut& a, float* ys) {
  const int lane = tid() & 63, wvl = tid() >> 6;
  // the wave's heads wvl, wvl + NWB, ...: every input requested first, then the norms
  constexpr int HPW = (4096 / VD + NWB - 1) / NWB;
  const float g0 = a.gw[lane], g1 = a.gw[lane + 64];
  float o[HPW][2], z[HPW][2];
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int hh = wvl + j * NWB;
    if (hh < a.nh) {
      o[j][0] = ldf<COH>(a.on + hh * VD + lane);
      o[j][1] = ldf<COH>(a.on + hh * VD + lane + 64);
      z[j][0] = ldf<COH>(a.z + hh * VD + lane);
      z[j][1] = ldf<COH>(a.z + hh * VD + lane + 64);
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
      const float s0 = SZ ? z[j][0] : silu(z[j][0]), s1 = SZ ? z[j][1] : silu(z[j][1]);
      ys[hh * VD + lane] = bf16r(bf16r(g0 * bf16r(o[j][0] * rr)) * s0);
      ys[hh * VD + lane + 64] = bf16r(bf16r(g1 * bf16r(o[j][1] * rr)) * s1);
    }
  }
}
// the query/key windows, spread over the workgroups (channel i: workgroup i % nblk)
template <bool COH>
__device__ __forceinline__ void qk_windows(const DnOut& a, int blk, int nblk, int ntb) {
  const int nq = a.nk * a.kl;
  for (int i = blk + nblk * tid(); i < 2 * nq; i += nblk * ntb) {
    const int part = i / nq, j = i % nq, kh = j / a.kl, d = j % a.kl;
    uint16_t* w = a.conv + ((int64_t)part * a.nk * KD + kh * KD + d) * 4;
    stw<COH>(w, shifted(ldw<COH>(w), ldf<COH>(a.P + i)));
  }
}
template <int G, int NTB>
__global__ __launch_bounds__(NTB) void dn_out(DnOut a) {
  static_assert(G * 64 <= 4096, "dn_out: at most 32 value heads");
  constexpr int NWB = NTB / 64;
  __shared__ __align__(16) float ys[G * 64];
  const int lane = tid() & 63;
  const int wv = blockIdx.x * NWB + (tid() >> 6), nwv = gridDim.x * NWB;
  WRow<G> cur;
  if (wv < a.nrows) cur.load(a.W, wv, lane);
  gated_norm<NWB, false>(a, ys);
  lds_barrier();
  XRegs<G> xc;
  xc.template load<false>(ys, lane);
  rows_run<G, 1, false>(a.W, a.nrows, xc, cur, wv, nwv, a.h);
  qk_windows<false>(a, blockIdx.x, gridDim.x, NTB);
}

// ---------------------------------------------------------------------------------------------
// The persistent run: n steps in one launch of one workgroup per CU. Per step, per layer five
// phases (the projections over the input norm; the delta rule in nk x rl x QC workgroups; the
// gated norm, out_proj and the query/key windows; SwiGLU over the post norm; down_proj), then
// the head over the final norm. A phase ends at a grid barrier: each wave drains its stores
// (agent-scope, coherent across the XCDs) and the workgroup arrives on a monotone counter.
//
// Each workgroup's wave 0 is its control wave: it holds no weight rows. It polls the barriers
// and stages each row phase's input in LDS: h and the norm's weight (every wave then forms the
// norm from LDS in the 512-lane order), or down_proj's input and the residual. Waves 1-7 stream
// the weight rows: right after a phase's arrival each requests its rows of the next phase (the
// first D; each later one as the row before it in its slot has been summed), which then stream
// from HBM while the barrier and the input complete. A vector memory counter counts every load
// of a wave in order, so a wave with rows in flight must not load anything else it has to wait
// for: the stream waves read their inputs and residuals from LDS only, and the layer tables
// come through scalar loads. The delta rule runs on all 8 waves of its workgroups; out_proj's
// rows go to the stream waves of the other workgroups, which request them before the delta rule
// (they have landed when its gated norm, formed by all 8 waves, is ready). The projections store
// silu(z) for the gated norm's z rows; SwiGLU stores its bf16 outputs in down_proj's interleaved
// input order.
// (Measured on MI355X: a CU's vector memory requests are served in order, so the control wave's
// polls and input loads wait behind the rows its CU requested at the arrival; a phase boundary
// costs about that burst's time at the CU's share of HBM bandwidth, 4-11 us.)
//
// The step's embedding row becomes h through LDS in the control wave (workgroup 0 also writes
// it to h for the residual). The head's keys alternate between two slots by step parity (the
// other slot is cleared for the next step). Every wait gives up after 3 s with the error word set
// (code 2), and so do the other workgroups on seeing it.
// The counter has 8 copies 128 bytes apart (workgroup b adds to copy b % 8, the XCD it lands on
// when workgroups are dealt round-robin), so at most 32 workgroups' atomics meet on one line; a
// waiter polls the sum. (One shared counter measured 3.9 us per barrier of 256 workgroups on
// MI355X, eight copies 1.6 us.)
#define BAR_COPIES 8
struct Bar {
  uint32_t* ctr;
  int32_t* err;
  uint32_t target;
  int nblk;
  int* flag;        // LDS
  uint64_t* tarr;   // LDS: the arrival's time (the sub-phase profiling build), or null
  __device__ __forceinline__ void arrive() {
    drain();
    lds_barrier();
#ifdef LXM_SUBPROF
    if (tid() == 0) *tarr = wall();
#endif
    target += (uint32_t)nblk;
    if (tid() == 0) add_rlx(ctr + 32 * (blockIdx.x % BAR_COPIES), 1u);
  }
  __device__ __forceinline__ bool wait() {
    if (tid() == 0) {
      const uint64_t t0 = wall();
      int ok = 1;
      for (;;) {
        uint32_t v[BAR_COPIES], sum = 0;
#pragma unroll
        for (int g = 0; g < BAR_COPIES; g++) v[g] = ld_rlx(ctr + 32 * g);
#pragma unroll
        for (int g = 0; g < BAR_COPIES; g++) sum += v[g];
        if ((int32_t)(sum - target) >= 0) break;
        __builtin_amdgcn_s_sleep(1);
        if (__hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          ok = 0;
          break;
        }
        if (wall() - t0 > TIMEOUT_TICKS) {
          __hip_atomic_fetch_max(gp(err), 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
      }
      *flag = ok;
    }
    lds_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const bool ok = *flag != 0;
    lds_barrier();  // (flag is free again)
    return ok;
  }
};

// h (n values, written by other workgroups) into LDS: thread t copies the values of its share
// of the 512-lane order (4t..4t+3, 2048 + 4t..)
__device__ __forceinline__ void stage_h(const float* h, int n, float* hs) {
  const int t = tid();
  // (both loads are issued before either value is stored, a column past n reading column 0: a
  // load under its column test was waited on inside its branch)
  const int c0 = 4 * t, c1 = 2048 + 4 * t;
  const v4f a = ldf4<true>(h, c0 < n ? c0 : 0), b = ldf4<true>(h, c1 < n ? c1 : 0);
  if (c0 < n) *reinterpret_cast<v4f*>(hs + c0) = a;
  if (c1 < n) *reinterpret_cast<v4f*>(hs + c1) = b;
}

// A stream wave's weight rows of one phase in flight: round j's row (round_row) in slot j % D.
// The first D are requested by prefetch (right after the arrival ahead of the phase), each later
// one when the row before it in its slot has been summed. prefetch fills every slot (a slot past
// the wave's last row requests its first row again, a cache hit), so no slot's old contents stay
// live from one phase to the next.
__device__ __forceinline__ int slot_row(int w0, int s, int nw, int rot, int n) {
  const int r = round_row(w0, s, nw, rot);
  return r < n ? r : min(w0, n - 1);
}
template <int G, int D>
struct RowSet {
  WRow<G> w[D];
  __device__ __forceinline__ void prefetch(const uint16_t* W, int nrows, int w0, int nw, int rot) {
#pragma unroll
    for (int s = 0; s < D; s++) w[s].load(W, slot_row(w0, s, nw, rot, nrows), tid() & 63);
  }
};
// the number of rows round_row deals to the wave w0 (of nw) out of nrows
__device__ __forceinline__ int rows_of(int w0, int nw, int rot, int nrows) {
  return w0 < nrows ? 1 + (nrows - (w0 + rot) % nw - 1) / nw : 0;
}
// A wave's n rows in rounds of D slots: while a round is not the last, each slot's row is summed
// and the slot then requests its row D rounds on (clamped to the wave's last row: the last full
// round's surplus requests hit the cache); the last round sums the rows left, with no requests.
// emit(s, r): row r's sum (lane 0 holds it) from slot s.
template <int D, class Dot, class Load, class Emit>
__device__ __forceinline__ void pipe(int n, int w0, int nw, int rot, Dot&& dot, Load&& load,
                                     Emit&& emit) {
  int j0 = 0;
  for (; j0 + D < n; j0 += D) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      const int r = round_row(w0, j0 + s, nw, rot);
      dot(s, r);
      // (the slot's next row is requested after its sums have read it: one copy per slot)
      __builtin_amdgcn_sched_barrier(0);
      load(s, round_row(w0, min(j0 + s + D, n - 1), nw, rot));
      emit(s, r);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < D; s++) {
    if (j0 + s < n) {
      const int r = round_row(w0, j0 + s, nw, rot);
      dot(s, r);
      emit(s, r);
    }
  }
}
// the wave's rows: MODE 0 out[r] = D(row . x); MODE 1 out[r] = D(hs[r] + D(row . x)), hs the
// staged residual; MODE 2 as 0, silu of it for the rows [zlo, zhi) (the gated norm's z)
template <int G, int D, int MODE, class X>
__device__ __forceinline__ void pipe_rows(RowSet<G, D>& rs, const uint16_t* W, int nrows,
                                          const X& xc, int w0, int nw, int rot, float* out,
                                          const float* hs, int zlo = 0, int zhi = 0) {
  float v = 0.0f;
  pipe<D>(
      rows_of(w0, nw, rot, nrows), w0, nw, rot, [&](int s, int r) { v = row_dot<G>(rs.w[s], xc); },
      [&](int s, int r) { rs.w[s].load(W, r, tid() & 63); },
      [&](int s, int r) {
        if ((tid() & 63) == 0) {
          if constexpr (MODE == 1) {
            stf<true>(out + r, bf16r(hs[r] + bf16r(v)));
          } else {
            const float y = bf16r(v);
            stf<true>(out + r, MODE == 2 && r >= zlo && r < zhi ? silu(y) : y);
          }
        }
      });
}
// SwiGLU units the same way (gate and up rows of unit u in slot j % D): act[u] =
// D(D(silu(D(g))) * D(u)) (TF:704-717), stored as bf16 at act16[pos(u)]: down_proj's interleaved
// input order (GI entries per lane)
template <int G, int D>
struct UnitSet {
  WRow<G> g[D], u[D];
  __device__ __forceinline__ void prefetch(const uint16_t* Wg, const uint16_t* Wu, int n, int w0,
                                           int nw, int rot) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      const int r = slot_row(w0, s, nw, rot, n);
      g[s].load(Wg, r, tid() & 63);
      u[s].load(Wu, r, tid() & 63);
    }
  }
};
// entry c of a row whose lanes hold G entries each, in the interleaved order: its halfword
__device__ __forceinline__ int il_pos(int c, int G) {
  const int l = c / G, k = c % G;
  return ((k >> 3) * 64 + l) * 8 + (k & 7);
}
template <int G, int GI, int D>
__device__ __forceinline__ void pipe_units(UnitSet<G, D>& us, const uint16_t* Wg,
                                           const uint16_t* Wu, int n, const XRegs<G>& xc, int w0,
                                           int nw, int rot, uint16_t* act16) {
  float g = 0.0f, v = 0.0f;
  pipe<D>(
      rows_of(w0, nw, rot, n), w0, nw, rot,
      [&](int s, int r) {
        g = row_dot<G>(us.g[s], xc);
        v = row_dot<G>(us.u[s], xc);
      },
      [&](int s, int r) {
        us.g[s].load(Wg, r, tid() & 63);
        us.u[s].load(Wu, r, tid() & 63);
      },
      [&](int s, int r) {
        if ((tid() & 63) == 0) {
          const float a = bf16r(silu_bf16(bf16r(g)) * bf16r(v));
          __hip_atomic_store(gp(act16 + il_pos(r, GI)), (uint16_t)(fbits(a) >> 16),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      });
}
// The head's rows w0, w0 + nw, ... (slot j % D): logits D(row . x), the wave's first maximum
// (ties to the lower index, NaN above everything: torch.argmax) folded into *keys by 64-bit
// atomic max.
template <int G, int D>
__device__ __forceinline__ void pipe_head(RowSet<G, D>& rs, const uint16_t* W, int nrows,
                                          const XRegs<G>& xc, int w0, int nw,
                                          unsigned long long* keys) {
  float best = 0.0f, v = 0.0f;
  int bidx = -1, nanr = -1;
  pipe<D>(
      rows_of(w0, nw, 0, nrows), w0, nw, 0,
      [&](int s, int r) { v = bf16r(row_dot<G>(rs.w[s], xc)); },
      [&](int s, int r) { rs.w[s].load(W, r, tid() & 63); },
      [&](int s, int r) {
        if (v != v) {
          if (nanr < 0) nanr = r;
        } else if (bidx < 0 || v > best) {
          best = v;
          bidx = r;
        }
      });
  if ((tid() & 63) == 0) {
    unsigned long long k = bidx < 0 ? 0ull : argmax_key(best, bidx);
    if (nanr >= 0) {
      const unsigned long long kn = argmax_key(__builtin_nanf(""), nanr);
      k = kn > k ? kn : k;
    }
    if (k) atomicMax(keys, k);
  }
}

// a layer's table through scalar loads (it never changes during a run; vector or flat loads
// would wait for every weight row the wave has in flight). Field by field: a struct copy is
// lowered to flat loads.
__device__ __forceinline__ lxm_dn_layer layer_of(const lxm_dn_layer* t, int L) {
  const __attribute__((address_space(4))) lxm_dn_layer* q =
      (const __attribute__((address_space(4))) lxm_dn_layer*)t + L;
  lxm_dn_layer y;
  y.proj = q->proj;
  y.conv_qk = q->conv_qk;
  y.conv_v = q->conv_v;
  y.A_log = q->A_log;
  y.dt_bias = q->dt_bias;
  y.gnorm = q->gnorm;
  y.ln_in = q->ln_in;
  y.ln_post = q->ln_post;
  y.out = q->out;
  y.gate = q->gate;
  y.up = q->up;
  y.down = q->down;
  y.rec = q->rec;
  y.conv = q->conv;
  return y;
}

// The control wave's share of a hidden vector of n <= 4096 values in the 512-lane order: lane l,
// slot m < M holds the 4 values at 256 m + 4 l (thread t = 64 (m % 8) + l's values 4t.. for
// m < 8, its values 2048 + 4t.. for m >= 8).
template <int M>
struct HVec {
  v4f v[M];
  // from a vector other workgroups write (agent scope)
  __device__ __forceinline__ void load_coh(const float* x, int n) {
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int c = 256 * m + 4 * (tid() & 63);
      v[m] = c < n ? ldf4<true>(x, c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  // from a constant vector (a norm's weight)
  __device__ __forceinline__ void load(const float* x, int n) {
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int c = 256 * m + 4 * (tid() & 63);
      v[m] = c < n ? *gp(reinterpret_cast<const v4f*>(x + c)) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  __device__ __forceinline__ void load_lds(const float* hs, int n) {
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int c = 256 * m + 4 * (tid() & 63);
      v[m] = c < n ? *reinterpret_cast<const v4f*>(hs + c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  __device__ __forceinline__ void store_lds(float* hs, int n) const {
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int c = 256 * m + 4 * (tid() & 63);
      if (c < n) *reinterpret_cast<v4f*>(hs + c) = v[m];
    }
  }
};
// rows in flight per stream wave: the projections' and the head's (GH entries per lane),
// out_proj's, SwiGLU's units, down_proj's
#define D_P 3
#define D_O 2
#define D_U 2
#define D_D 2

// The persistent run's phase clock (the sub-phase profiling build, LXM_SUBPROF): thread 0 (the
// control wave's lane 0) stamps each phase's start (the barrier before it passed), its input
// staged (dp_x) and every wave's rows summed (the arrival, in Bar::arrive); dp_phase(k) closes
// phase k and adds its three spans to the workgroup's sums, written to p.prof at the end.
#define DP_NPH 6
struct DnProf {
  uint64_t acc[DP_NPH][3];
  uint64_t t[3];  // start, input staged, arrival
};
template <class S>
__device__ __forceinline__ void dp_x(S& sm) {
#ifdef LXM_SUBPROF
  if (tid() == 0) sm.dp.t[1] = wall();
#endif
}
template <class S>
__device__ __forceinline__ void dp_phase(S& sm, int k) {
#ifdef LXM_SUBPROF
  if (tid() == 0) {
    DnProf& d = sm.dp;
    const uint64_t w = wall();
    d.acc[k][0] += d.t[1] - d.t[0];
    d.acc[k][1] += d.t[2] - d.t[1];
    d.acc[k][2] += w - d.t[2];
    d.t[0] = d.t[1] = w;
  }
#endif
}
template <class S>
__device__ __forceinline__ uint64_t* dp_tarr(S& sm) {
#ifdef LXM_SUBPROF
  return &sm.dp.t[2];
#else
  return nullptr;
#endif
}

// the shared memory of the persistent run
template <int GH, int GV, int GI>
struct RunLds {
  float hs[4096];                 // a staged hidden vector (a norm's input, the residual)
  float ws[4096];                 // a staged norm weight
  float wsum[NW];
  float ys[GV * 64];              // the gated norm's output
  v4u xd[8 * GI];                 // down_proj's bf16 input, interleaved
  GdnLds gl;
  int flag;
#ifdef LXM_SUBPROF
  DnProf dp;
#endif
};

// The run's shared state (scalar)
struct RunCtx {
  const lxm_dn_params* pp;
  int H, I, nk, kl, rl, R, nq, nvr, nproj, ngdn, nL, nit, step0;
  float eps;
};
__device__ __forceinline__ RunCtx run_ctx(const lxm_dn_params* pp, int n_run) {
  const lxm_dn_params& p = *pp;
  RunCtx c;
  c.pp = pp;
  c.H = p.hidden;
  c.I = p.inter;
  c.nk = p.nk;
  c.kl = p.kl;
  c.rl = p.rl;
  c.R = p.nv / p.nk;
  c.nq = c.nk * c.kl;
  c.nvr = c.nk * c.rl * VD;
  c.nproj = 2 * c.nq + 2 * c.nvr + 2 * c.nk * c.rl;
  c.ngdn = c.nk * c.rl * QC;
  c.nL = p.n_layers;
  c.nit = n_run * (c.nL + 1);
  c.step0 = *p.step;
  c.eps = p.rms_eps;
  return c;
}
__device__ __forceinline__ DnGdn gdn_of(const lxm_dn_params& p, const lxm_dn_layer& ly,
                                        const RunCtx& c) {
  return DnGdn{ly.conv_qk, ly.conv_v, ly.A_log, ly.dt_bias, ly.rec, ly.conv, p.P, p.on,
               c.nk, c.kl, c.rl, c.R};
}
__device__ __forceinline__ DnOut out_of(const lxm_dn_params& p, const lxm_dn_layer& ly,
                                        const RunCtx& c) {
  return DnOut{ly.out, c.H, c.nk * c.rl, p.on, p.P + 2 * c.nq + c.nvr, ly.gnorm, p.geps, p.h,
               ly.conv, p.P, c.nk, c.kl};
}
// the delta rule phase (both roles; all 8 waves of the delta rule's workgroups)
template <int GH, int GV, int GI>
__device__ __forceinline__ bool gdn_phase(const lxm_dn_params& p, const lxm_dn_layer& ly,
                                          const RunCtx& c, Bar& bar, RunLds<GH, GV, GI>& sm) {
  const DnGdn g = gdn_of(p, ly, c);
  float s[16];
  gdn_load<true>(g, blockIdx.x, s);
  if (!bar.wait()) return false;
  dp_phase(sm, 0);
  gdn_body<true>(g, blockIdx.x, s, sm.gl);
  bar.arrive();
  if (!bar.wait()) return false;
  dp_phase(sm, 1);
  return true;
}

// The control wave's loop (wave 0)
template <int GH, int GV, int GI>
__device__ __forceinline__ void run_ctl(const lxm_dn_params* pp, int n_run,
                                        RunLds<GH, GV, GI>& sm) {
  constexpr int M = (64 * GH + 255) / 256;
  const lxm_dn_params& p = *pp;
  const RunCtx c = run_ctx(pp, n_run);
  const int b = blockIdx.x, nb = gridDim.x;
  Bar bar{p.sync, p.err, 0u, nb, &sm.flag, dp_tarr(sm)};
  uint16_t* const act16 = reinterpret_cast<uint16_t*>(p.xn + c.H);
  int tok = *p.tok;
  HVec<M> w;  // the next norm's weight (staged in LDS)
  w.load(layer_of(p.layers, 0).ln_in, c.H);
  w.store_lds(sm.ws, c.H);
#ifdef LXM_SUBPROF
  if (tid() < DP_NPH * 3) sm.dp.acc[tid() / 3][tid() % 3] = 0;
  if (tid() == 0) sm.dp.t[0] = sm.dp.t[1] = sm.dp.t[2] = wall();
#endif
  for (int it = 0; it < c.nit; it++) {
    const int si = it / (c.nL + 1), L = it % (c.nL + 1), step = c.step0 + si;
    HVec<M> h;
    if (L == 0) {
      // the input; its embedding row as h, through LDS (workgroup 0 writes h)
      if (step < p.n_forced) tok = p.forced[step];
      if (tok < 0 || tok >= p.vocab) {
        if (b == 0 && tid() == 0)
          __hip_atomic_fetch_max(gp(p.err), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        tok = 0;
      }
      const uint16_t* e = p.embed + (int64_t)tok * c.H;
      // (a round's chunks all requested before any is stored: a load stored in its own
      // iteration is waited for alone)
      constexpr int EB = 8;
      const int ne = c.H / 8;
      for (int j0 = tid() & 63; j0 < ne; j0 += 64 * EB) {
        v4u u[EB];
#pragma unroll
        for (int q = 0; q < EB; q++) {
          const int j = j0 + 64 * q;
          u[q] = *gp(reinterpret_cast<const v4u*>(e) + (j < ne ? j : j0));
        }
#pragma unroll
        for (int q = 0; q < EB; q++) {
          // stored chunk j: entries 8 (j / 64) .. of lane j % 64 (GH >= 8), or entries 8j.. (GH 4);
          // a chunk past the end is chunk j0 again, stored again (unconditional stores keep the
          // compiler from moving a load into a store's branch)
          const int j = j0 + 64 * q < ne ? j0 + 64 * q : j0;
          const int c0 = GH < 8 ? 8 * j : (j % 64) * GH + 8 * (j / 64);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            sm.hs[c0 + 2 * i] = bf16f(u[q][i] & 0xffffu);
            sm.hs[c0 + 2 * i + 1] = bf16f(u[q][i] >> 16);
          }
        }
      }
      if (b == 0) {
        h.load_lds(sm.hs, c.H);
        for (int m = 0; m < M; m++) {
          const int c0 = 256 * m + 4 * (tid() & 63);
          if (c0 < c.H)
#pragma unroll
            for (int i = 0; i < 4; i++) stf<true>(p.h + c0 + i, h.v[m][i]);
        }
      }
    } else {
      h.load_coh(p.h, c.H);
      h.store_lds(sm.hs, c.H);
    }
    unsigned long long* key = p.keys + (step & 1);
    // the first phase's input: the input norm (a layer) or the final norm (the head), formed by
    // every wave from LDS
    lds_barrier();
    (void)norm_factor<false>(sm.hs, c.H, c.eps, sm.wsum);
    dp_x(sm);
    if (L < c.nL) {
      const lxm_dn_layer ly = layer_of(p.layers, L);
      bar.arrive();
      if (b < c.ngdn) {
        if (!gdn_phase<GH, GV, GI>(p, ly, c, bar, sm)) return;
      } else {
        if (!bar.wait()) return;
        dp_phase(sm, 0);
        bar.arrive();
        if (!bar.wait()) return;
        dp_phase(sm, 1);
      }
      // out_proj's phase: the gated norm and the residual (the rows' workgroups), the windows
      const DnOut o = out_of(p, ly, c);
      if (b >= c.ngdn) {
        gated_norm<NW, true, true>(o, sm.ys);
        stage_h(p.h, c.H, sm.hs);
      }
      lds_barrier();
      dp_x(sm);
      qk_windows<true>(o, b, nb, NT);
      bar.arrive();
      w.load(ly.ln_post, c.H);
      w.store_lds(sm.ws, c.H);
      if (!bar.wait()) return;
      dp_phase(sm, 2);
      // SwiGLU's input: the post norm
      h.load_coh(p.h, c.H);
      h.store_lds(sm.hs, c.H);
      lds_barrier();
      (void)norm_factor<false>(sm.hs, c.H, c.eps, sm.wsum);
      dp_x(sm);
      bar.arrive();
      if (!bar.wait()) return;
      dp_phase(sm, 3);
      // down_proj's input and the residual: the residual's loads and each round's chunks all
      // requested before any is stored (a load stored in its own iteration is waited for alone)
      h.load_coh(p.h, c.H);
      {
        constexpr int XB = 9;
        const int nx = c.I / 8;
        for (int j0 = tid() & 63; j0 < nx; j0 += 64 * XB) {
          v4u xr[XB];
#pragma unroll
          for (int q = 0; q < XB; q++) {
            const int j = j0 + 64 * q;
            xr[q] = __builtin_bit_cast(
                v4u, ldf4<true>(reinterpret_cast<const float*>(act16), 4 * (j < nx ? j : j0)));
          }
          // (a chunk past the end is chunk j0 again, stored again: unconditional stores keep the
          // compiler from moving a load into a store's branch)
#pragma unroll
          for (int q = 0; q < XB; q++) sm.xd[j0 + 64 * q < nx ? j0 + 64 * q : j0] = xr[q];
        }
      }
      h.store_lds(sm.hs, c.H);
      lds_barrier();
      dp_x(sm);
    } else {
      lds_barrier();  // (the stream waves' head rows)
    }
    bar.arrive();
    {
      const bool head = L + 1 == c.nL;
      const int Ln = L + 1 > c.nL ? 0 : L + 1;
      w.load(head ? p.w_final : layer_of(p.layers, Ln).ln_in, c.H);
      w.store_lds(sm.ws, c.H);
    }
    if (!bar.wait()) return;
    dp_phase(sm, L < c.nL ? 4 : 5);
    if (L == c.nL) {
      tok = argmax_idx(__hip_atomic_load(gp(key), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      if (b == 0 && tid() == 0) {
        if (step < p.n_steps) p.preds[step] = tok;
        __hip_atomic_store(gp(p.keys + ((step + 1) & 1)), 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
#ifdef LXM_SUBPROF
  if (p.prof && tid() < DP_NPH * 3) p.prof[32 * b + tid()] = sm.dp.acc[tid() / 3][tid() % 3];
#endif
  if (b == 0 && tid() == 0) {
    *p.step = c.step0 + n_run;
    *p.tok = tok;
  }
}

// A stream wave's loop (waves 1-7)
template <int GH, int GV, int GI>
__device__ __forceinline__ void run_stream(const lxm_dn_params* pp, int n_run,
                                           RunLds<GH, GV, GI>& sm) {
  const lxm_dn_params& p = *pp;
  const RunCtx c = run_ctx(pp, n_run);
  const int b = blockIdx.x, nb = gridDim.x;
  Bar bar{p.sync, p.err, 0u, nb, &sm.flag, dp_tarr(sm)};
  uint16_t* const act16 = reinterpret_cast<uint16_t*>(p.xn + c.H);
  // stream wave index (waves 1-7 of every workgroup); out_proj's waves (outside the delta rule's
  // workgroups)
#define SW (b * (NW - 1) + wave_id() - 1)
#define OW ((b - c.ngdn) * (NW - 1) + wave_id() - 1)
  const int nsw = nb * (NW - 1), now = (nb - c.ngdn) * (NW - 1);
  const int zlo = 2 * c.nq + c.nvr, zhi = 2 * c.nq + 2 * c.nvr;
  RowSet<GH, D_P> rp;  // the item's first rows (a layer's projections, the head's)
  rp.prefetch(layer_of(p.layers, 0).proj, c.nproj, SW, nsw, 0);
  for (int it = 0; it < c.nit; it++) {
    const int si = it / (c.nL + 1), L = it % (c.nL + 1), step = c.step0 + si;
    unsigned long long* key = p.keys + (step & 1);
    lds_barrier();  // (the control wave's h and weight)
    const float rn = norm_factor<false>(sm.hs, c.H, c.eps, sm.wsum);
    if (L < c.nL) {
      const lxm_dn_layer ly = layer_of(p.layers, L);
      // the projections (silu of the gated norm's z rows)
      {
        XRegs<GH> xc;
        xc.template load_norm<false>(sm.hs, sm.ws, rn, tid() & 63);
        pipe_rows<GH, D_P, 2>(rp, ly.proj, c.nproj, xc, SW, nsw, 0, p.P, sm.hs, zlo, zhi);
      }
      bar.arrive();
      RowSet<GV, D_O> ro;
      if (b < c.ngdn) {
        if (!gdn_phase<GH, GV, GI>(p, ly, c, bar, sm)) return;
      } else {
        ro.prefetch(ly.out, c.H, OW, now, 0);
        if (!bar.wait()) return;
        bar.arrive();
        if (!bar.wait()) return;
      }
      // out_proj (outside the delta rule's workgroups)
      const DnOut o = out_of(p, ly, c);
      if (b >= c.ngdn) {
        gated_norm<NW, true, true>(o, sm.ys);
        stage_h(p.h, c.H, sm.hs);
      }
      lds_barrier();
      if (b >= c.ngdn) {
        XRegs<GV> xc;
        xc.template load<false>(sm.ys, tid() & 63);
        pipe_rows<GV, D_O, 1>(ro, ly.out, c.H, xc, OW, now, 0, p.h, sm.hs);
      }
      qk_windows<true>(o, b, nb, NT);
      bar.arrive();
      UnitSet<GH, D_U> us;
      us.prefetch(ly.gate, ly.up, c.I, SW, nsw, 0);
      if (!bar.wait()) return;
      // SwiGLU
      lds_barrier();  // (the control wave's h and weight)
      {
        XRegs<GH> xc;
        xc.template load_norm<false>(sm.hs, sm.ws, norm_factor<false>(sm.hs, c.H, c.eps, sm.wsum),
                                     tid() & 63);
        pipe_units<GH, GI, D_U>(us, ly.gate, ly.up, c.I, xc, SW, nsw, 0, act16);
      }
      bar.arrive();
      RowSet<GI, D_D> rdn;
      rdn.prefetch(ly.down, c.H, SW, nsw, 0);
      if (!bar.wait()) return;
      // down_proj
      lds_barrier();  // (the control wave's input and residual)
      {
        const XLds<GI> xc{sm.xd, tid() & 63};
        pipe_rows<GI, D_D, 1>(rdn, ly.down, c.H, xc, SW, nsw, 0, p.h, sm.hs);
      }
    } else {
      // the head over the final norm; the argmax key of this step's parity
      XRegs<GH> xc;
      xc.template load_norm<false>(sm.hs, sm.ws, rn, tid() & 63);
      pipe_head<GH, D_P>(rp, p.embed, p.vocab, xc, SW, nsw, key);
      lds_barrier();
    }
    bar.arrive();
    // the next item's first rows: the next layer's projections, or the head's (after the last
    // item every slot requests the head's row 0, a cache hit: a request on every path, so the
    // old rows' registers are free during the item)
    {
      const bool head = L + 1 == c.nL, last = it + 1 == c.nit;
      const int Ln = L + 1 > c.nL ? 0 : L + 1;
      rp.prefetch(head || last ? p.embed : layer_of(p.layers, Ln).proj,
                  last ? 1 : head ? p.vocab : c.nproj, SW, nsw, 0);
    }
    if (!bar.wait()) return;
  }
#undef SW
#undef OW
}

template <int GH, int GV, int GI>
__global__ __launch_bounds__(NT, 1) void dn_run(const lxm_dn_params* __restrict__ pp, int n_run) {
  static_assert(GV * 64 <= 4096, "at most 32 live value heads");
  __shared__ RunLds<GH, GV, GI> sm;
  if (wave_id() == 0) run_ctl<GH, GV, GI>(pp, n_run, sm);
  else run_stream<GH, GV, GI>(pp, n_run, sm);
}

// ---------------------------------------------------------------------------------------------
// The batched prefill (lxm_dn_prefill): T forced tokens through every layer in batches of up to
// PB tokens, without the head, leaving the states and windows that T calls of lxm_dn_step leave,
// bit for bit. Per batch and layer: every token's input norm (pb_norm); the projections
// (pb_rows: each weight row read once per batch; lane l sums its 64th of the row for every token
// in the step's order, and the 64 lane sums of every (row, token) go through the step's pairwise
// tree, spread over the lanes); every token's conv, l2norms, beta and decay (pb_prep: token t's
// window is the previous tokens' projections); the delta rule token by token (pb_gdn); the gated
// norm and the windows' advance (pb_gnorm); out_proj (pb_hrows), the post norm, SwiGLU (pb_rows)
// and down_proj (pb_hrows). The row kernels' inputs are stored in their weights' interleaved
// order.
#define PB LXM_DN_PB
#define PBT 256  // threads of the row kernels: 4 waves

// position of element c of a row of K = 64 G entries in the interleaved order
__device__ __forceinline__ int il(int c, int G) {
  if (G < 8) return c;
  const int l = c / G, k = c % G;
  return ((k >> 3) * 64 + l) * 8 + (k & 7);
}

// V values per lane, each to be summed over the wave by the pairwise tree at offsets 32..1:
// after the call lane l holds the sums of values l V / 64 .. + max(1, V / 64) - 1 (in v[0..]).
// At offset o a lane keeps half of its values (the upper half where lane & o) and adds its
// partner's partial sums of them: the same pairs as the tree's (lane l + lane l + o), since
// fp32 addition is commutative.
template <int V, int S>
__device__ __forceinline__ void tree_scatter(float (&v)[V], int lane) {
  if constexpr (S < 6) {
    constexpr int o = 32 >> S, C = V >> S;
    if constexpr (C >= 2) {
      const bool up = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < C / 2; i++) {
        const float send = up ? v[i] : v[i + C / 2];
        const float keep = up ? v[i + C / 2] : v[i];
        v[i] = keep + __shfl_xor(send, o);
      }
    } else {
      v[0] = v[0] + __shfl_xor(v[0], o);
    }
    tree_scatter<V, S + 1>(v, lane);
  }
}

// A chunk (CH = 8 or 4 bf16 values) of an interleaved bf16 row as 16 bytes
template <int CH>
__device__ __forceinline__ v4u chunk_bf(const uint16_t* row, int q, int lane) {
  if constexpr (CH == 8) {
    return reinterpret_cast<const v4u*>(row)[q * 64 + lane];
  } else {
    const uint2 u = reinterpret_cast<const uint2*>(row)[lane];
    return v4u{u.x, u.y, 0u, 0u};
  }
}
// acc += the chunk's products in entry order (bf16 x bf16 products are exact in fp32)
template <int CH>
__device__ __forceinline__ float chunk_dot(v4u w, v4u x, float acc) {
#pragma unroll
  for (int k = 0; k < CH / 2; k++) {
    acc = __builtin_fmaf(bitsf(w[k] << 16), bitsf(x[k] << 16), acc);
    acc = __builtin_fmaf(bitsf(w[k] & 0xffff0000u), bitsf(x[k] & 0xffff0000u), acc);
  }
  return acc;
}
__device__ __forceinline__ uint16_t bf16_bits(float v) { return (uint16_t)(fbits(v) >> 16); }

// Rows for a batch of n <= PB tokens: the wave's R rows (MODE 2: R / 2 SwiGLU units, gate rows
// from W and up rows from W2) over X (n x 64 G bf16, interleaved). The batch's inputs are staged
// in LDS one chunk per lane at a time, double-buffered: each thread loads its share of chunk q + 1
// into registers before chunk q's sums and stores it to LDS after them, so a chunk costs one
// barrier and its loads overlap the arithmetic. MODE 0: out[b ldo + r] = D(s) (float); 1:
// out[b ldo + r] = D(out + D(s)) (float, the residual); 2: out[b ldo + il(u, og)] =
// D(D(silu(D(g))) * D(u)) (bf16).
template <int G, int R, int MODE>
__global__ __launch_bounds__(PBT) void pb_rows(const uint16_t* __restrict__ W,
                                               const uint16_t* __restrict__ W2, int nrows,
                                               const uint16_t* __restrict__ X, int n, void* out,
                                               int ldo, int og) {
  constexpr int CH = G == 4 ? 4 : 8, NC = G / CH, K = 64 * G, V = R * PB;
  constexpr int RU = MODE == 2 ? R / 2 : R;  // distinct row indices per wave
  constexpr int SPT = PB * 64 / PBT;         // staged chunks per thread
  static_assert(MODE != 2 || (R % 2 == 0 && (V == 128 || V == 64)),
                "units: gate and up sums 32 lanes apart");
  __shared__ v4u xs[2][PB * 64];
  const int lane = tid() & 63;
  const int wv = blockIdx.x * (PBT / 64) + (tid() >> 6);
  const uint16_t* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) {
    int r = wv * RU + i % RU;
    r = r < nrows ? r : nrows - 1;  // (rows past the end load the last row, unused)
    rp[i] = (MODE == 2 && i >= RU ? W2 : W) + (int64_t)r * K;
  }
  // thread t stages (token, lane) = idx / 64, idx % 64 for idx = t + j PBT; tokens past n: zero
  auto fetch = [&](int q, v4u (&st)[SPT]) {
#pragma unroll
    for (int j = 0; j < SPT; j++) {
      const int idx = tid() + j * PBT, b = idx >> 6;
      st[j] = b < n ? chunk_bf<CH>(X + (int64_t)b * K, q, idx & 63) : v4u{0u, 0u, 0u, 0u};
    }
  };
  float acc[R][PB];
#pragma unroll
  for (int i = 0; i < R; i++)
#pragma unroll
    for (int b = 0; b < PB; b++) acc[i][b] = 0.0f;
  v4u st[SPT];
  fetch(0, st);
  for (int q = 0; q < NC; q++) {
    v4u w[R];
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = chunk_bf<CH>(rp[i], q, lane);
    v4u* buf = xs[q & 1];
#pragma unroll
    for (int j = 0; j < SPT; j++) buf[tid() + j * PBT] = st[j];
    // (every thread's share of chunk q is in; the buffer written next was last read two
    // chunks ago, before this barrier)
    lds_barrier();
    if (q + 1 < NC) fetch(q + 1, st);
#pragma unroll
    for (int b = 0; b < PB; b++) {
      const v4u xx = buf[b * 64 + lane];
#pragma unroll
      for (int i = 0; i < R; i++) acc[i][b] = chunk_dot<CH>(w[i], xx, acc[i][b]);
    }
  }
  float v[V];
#pragma unroll
  for (int i = 0; i < R; i++)
#pragma unroll
    for (int b = 0; b < PB; b++) v[i * PB + b] = acc[i][b];
  tree_scatter<V, 0>(v, lane);
  // (V < 64: 64 / V lanes hold each sum; the first of them stores it)
  constexpr int PER = V >= 64 ? V / 64 : 1;
  if (V < 64 && lane % (V < 64 ? 64 / V : 1) != 0) return;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int vi = (lane * V) / 64 + j;
    const int i = vi / PB, b = vi % PB;
    if constexpr (MODE == 2) {
      const float u = __shfl_xor(v[j], 32);  // (the up row's sum, 32 lanes on)
      const int unit = wv * RU + i;
      if (lane < 32 && unit < nrows && b < n)
        static_cast<uint16_t*>(out)[(int64_t)b * ldo + il(unit, og)] =
            bf16_bits(bf16r(silu_bf16(bf16r(v[j])) * bf16r(u)));
    } else {
      const int r = wv * RU + i;
      if (r < nrows && b < n) {
        float* o = static_cast<float*>(out) + (int64_t)b * ldo + r;
        if constexpr (MODE == 0) *o = bf16r(v[j]);
        else *o = bf16r(*o + bf16r(v[j]));
      }
    }
  }
}

// Long rows (out_proj, down_proj: few rows of many entries) for a batch of PB tokens: the
// workgroup's 4 waves share R rows, wave w taking tokens w BW .. w BW + BW - 1 (BW = PB / 4), each
// wave reading its tokens' inputs straight from X (bf16; no LDS, no barriers: the rows are too
// few to share a staged input among many waves), the next chunk's loads issued before this
// chunk's sums. Sums and MODEs as pb_rows (0 and 1).
template <int G, int R, int MODE>
__global__ __launch_bounds__(PBT) void pb_hrows(const uint16_t* __restrict__ W, int nrows,
                                                const uint16_t* __restrict__ X, int n, float* out,
                                                int ldo) {
  constexpr int CH = G == 4 ? 4 : 8, NC = G / CH, K = 64 * G, BW = PB / (PBT / 64), V = R * BW;
  static_assert(V <= 64 && 64 % V == 0, "one sum per lane group");
  const int lane = tid() & 63, wvl = tid() >> 6;
  const int r0 = blockIdx.x * R, b0 = wvl * BW;
  const uint16_t* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int r = r0 + i < nrows ? r0 + i : nrows - 1;
    rp[i] = W + (int64_t)r * K;
  }
  const uint16_t* xp[BW];
#pragma unroll
  for (int b = 0; b < BW; b++) {
    const int bb = b0 + b < n ? b0 + b : n - 1;  // (tokens past n read token n - 1, unused)
    xp[b] = X + (int64_t)bb * K;
  }
  float acc[R][BW];
#pragma unroll
  for (int i = 0; i < R; i++)
#pragma unroll
    for (int b = 0; b < BW; b++) acc[i][b] = 0.0f;
  v4u w[R], x[BW];
#pragma unroll
  for (int i = 0; i < R; i++) w[i] = chunk_bf<CH>(rp[i], 0, lane);
#pragma unroll
  for (int b = 0; b < BW; b++) x[b] = chunk_bf<CH>(xp[b], 0, lane);
  for (int q = 0; q < NC; q++) {
    v4u wn[R], xn[BW];
    const int qn = q + 1 < NC ? q + 1 : q;  // (the last chunk reloads itself, unused)
#pragma unroll
    for (int i = 0; i < R; i++) wn[i] = chunk_bf<CH>(rp[i], qn, lane);
#pragma unroll
    for (int b = 0; b < BW; b++) xn[b] = chunk_bf<CH>(xp[b], qn, lane);
#pragma unroll
    for (int b = 0; b < BW; b++)
#pragma unroll
      for (int i = 0; i < R; i++) acc[i][b] = chunk_dot<CH>(w[i], x[b], acc[i][b]);
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = wn[i];
#pragma unroll
    for (int b = 0; b < BW; b++) x[b] = xn[b];
  }
  float v[V];
#pragma unroll
  for (int i = 0; i < R; i++)
#pragma unroll
    for (int b = 0; b < BW; b++) v[i * BW + b] = acc[i][b];
  tree_scatter<V, 0>(v, lane);
  if (lane % (64 / V) != 0) return;  // (64 / V lanes hold each sum; the first stores it)
  const int vi = (lane * V) / 64, i = vi / BW, b = b0 + vi % BW, r = r0 + i;
  if (r < nrows && b < n) {
    float* o = out + (int64_t)b * ldo + r;
    if constexpr (MODE == 0) *o = bf16r(v[0]);
    else *o = bf16r(*o + bf16r(v[0]));
  }
}

// every token's embedding row into its residual
__global__ __launch_bounds__(PBT) void pb_embed(const uint16_t* __restrict__ embed,
                                                const int32_t* __restrict__ tokens, int H,
                                                int vocab, float* h, int32_t* err) {
  const int b = blockIdx.x;
  int tok = tokens[b];
  if (tok < 0 || tok >= vocab) {
    if (tid() == 0) *err = 1;
    tok = 0;
  }
  const uint16_t* e = embed + (int64_t)tok * H;
  const int G = H / 64;
  for (int c = tid(); c < H; c += PBT) h[(int64_t)b * H + c] = bf16f(e[il(c, G)]);
}

// every token's RMSNorm (the step's factor and elements) into xn (bf16), interleaved for G = gx
__global__ __launch_bounds__(NT) void pb_norm(const float* __restrict__ h,
                                              const float* __restrict__ nw, float eps, int H,
                                              int gx, uint16_t* xn) {
  __shared__ float wsum[NW];
  const int b = blockIdx.x;
  const float* hb = h + (int64_t)b * H;
  const float r = norm_factor<false>(hb, H, eps, wsum);
  for (int c = tid(); c < H; c += NT)
    xn[(int64_t)b * H + il(c, gx)] = bf16_bits(norm_el(hb[c], r, nw[c]));
}

struct PbGdn {
  const uint16_t* conv_qk;  // (2, nk, kl, 4)
  const uint16_t* conv_v;   // (nk, rl, 128, 4)
  const float* A_log;
  const float* dt_bias;
  float* rec;
  uint16_t* conv;
  const float* P;           // (n, nproj)
  float* qk;                // (n, nk, 2, 256)
  float* v;                 // (n, nvr)
  float* g;                 // (n, nk rl, 2)
  float* live;              // (n, nk, 2)
  float* o;                 // (n, nvr)
  int nk, kl, rl, R, nproj, n;
  float* gl;                // (n, nk rl): the log decays g (the chunked form's input), or null
};
// conv_y for token b of the batch: the window [x(b-3), x(b-2), x(b-1)] is the batch's earlier
// projections (row ch of P) or, before the batch, the stored window's newest values
__device__ __forceinline__ float conv_b(uint64_t win, const uint16_t* taps, const float* P,
                                        int nproj, int ch, int b) {
  float y = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int idx = b - 3 + k;
    const float x = idx >= 0 ? P[(int64_t)idx * nproj + ch]
                             : bf16f((uint32_t)(win >> (16 * (idx + 4))) & 0xffffu);
    y = __builtin_fmaf(bf16f(taps[k]), x, y);
  }
  return silu_bf16(bf16r(y));
}
// one workgroup per (token, key head): the query and key (conv, l2norm in the model dtype, the
// query times 1/16, and whether any element is nonzero), the key head's value channels, and its
// value heads' beta and exp(g), as the step's delta-rule kernel forms them
__global__ __launch_bounds__(KD) void pb_prep(PbGdn a) {
  __shared__ float qd[KD], kd[KD];
  const int b = blockIdx.x, kh = blockIdx.y, t = tid(), lane = t & 63, wv = t >> 6;
  const int nk = a.nk, kl = a.kl, rl = a.rl, nq = nk * kl, nvr = nk * rl * VD;
  float q = 0.0f, k = 0.0f;
  if (t < kl) {
    const int64_t cq = (int64_t)kh * KD + t, ck = (int64_t)nk * KD + kh * KD + t;
    q = conv_b(ldw<false>(a.conv + cq * 4), a.conv_qk + ((int64_t)kh * kl + t) * 4, a.P, a.nproj,
               kh * kl + t, b);
    k = conv_b(ldw<false>(a.conv + ck * 4), a.conv_qk + ((int64_t)(nk + kh) * kl + t) * 4, a.P,
               a.nproj, nq + kh * kl + t, b);
  }
  qd[t] = q;
  kd[t] = k;
  for (int c = t; c < rl * VD; c += KD) {
    const int vslot = kh * rl + c / VD, d = c % VD, vh = kh * a.R + c / VD;
    const uint64_t win = ldw<false>(a.conv + (2 * (int64_t)nk * KD + (int64_t)vh * VD + d) * 4);
    a.v[(int64_t)b * nvr + vslot * VD + d] =
        conv_b(win, a.conv_v + ((int64_t)vslot * VD + d) * 4, a.P, a.nproj, 2 * nq + vslot * VD + d, b);
  }
  if (t < rl) {
    const int vslot = kh * rl + t, vh = kh * a.R + t;
    const float* Pb = a.P + (int64_t)b * a.nproj;
    const float bb = Pb[2 * nq + 2 * nvr + vslot], aa = Pb[2 * nq + 2 * nvr + nk * rl + vslot];
    float* g = a.g + ((int64_t)b * nk * rl + vslot) * 2;
    g[0] = bf16r(sigmoid(bb));
    const float gg = (-cr_exp(a.A_log[vh])) * softplus(aa + a.dt_bias[vh]);
    g[1] = cr_exp(gg);
    if (a.gl) a.gl[(int64_t)b * nk * rl + vslot] = gg;
  }
  lds_barrier();
  if (wv < 2) {
    const float* x = wv ? kd : qd;
    float* o = a.qk + (((int64_t)b * nk + kh) * 2 + wv) * KD;
    float xs[4], ss = 0.0f;
    bool nz = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xs[i] = x[lane + 64 * i];
      nz |= xs[i] != 0.0f;
      ss = ss + bf16r(xs[i] * xs[i]);
    }
    const bool any = __ballot(nz) != 0ull;
    ss = bf16r(sum64(ss));
    const float inv = bf16r(rsqrt_(bf16r(ss + 1e-6f)));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v = bf16r(xs[i] * inv);
      if (!wv) v = v * 0.0625f;
      o[lane + 64 * i] = v;
    }
    if (lane == 0) a.live[((int64_t)b * nk + kh) * 2 + wv] = any ? 1.0f : 0.0f;
  }
}
// the delta rule of one live value head's 32 state columns (nk x rl x QC workgroups, as the
// step's) over the batch's tokens in order, the tile in registers throughout
struct PbLds {
  float qk[PB][2][KD];
  float vb[PB][QW], bg[PB][2], lv[PB];
  float bsk[16 * QW], bso[16 * QW], dl[QW];
};
__global__ __launch_bounds__(NT) void pb_gdn(PbGdn a) {
  __shared__ PbLds l;
  const int t = tid(), blk = blockIdx.x;
  const int nk = a.nk, rl = a.rl, nvr = nk * rl * VD, n = a.n;
  const int vslot = blk / QC, c0 = (blk % QC) * QW, kh = vslot / rl, vh = kh * a.R + vslot % rl;
  const int c = t % QW, rb = t / QW;
  float* S = a.rec + (size_t)vh * KD * VD + c0 + c + rb * 16 * VD;
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; i++) s[i] = S[i * VD];
  for (int i = t; i < n * 2 * KD; i += NT) {
    const int b = i / (2 * KD), j = i % (2 * KD);
    (&l.qk[b][0][0])[j] = a.qk[((int64_t)b * nk + kh) * 2 * KD + j];
  }
  for (int i = t; i < n * QW; i += NT) {
    const int b = i / QW, j = i % QW;
    l.vb[b][j] = a.v[(int64_t)b * nvr + vslot * VD + c0 + j];
  }
  if (t < n) {
    const float* g = a.g + ((int64_t)t * nk * rl + vslot) * 2;
    l.bg[t][0] = g[0];
    l.bg[t][1] = g[1];
    const float* lv = a.live + ((int64_t)t * nk + kh) * 2;
    l.lv[t] = lv[0] != 0.0f || lv[1] != 0.0f ? 1.0f : 0.0f;
  }
  lds_barrier();
  for (int b = 0; b < n; b++) {
    const float beta = l.bg[b][0], e = l.bg[b][1];
    if (e != 1.0f) {
#pragma unroll
      for (int i = 0; i < 16; i++) s[i] = s[i] * e;
    }
    float* o_out = a.o + (int64_t)b * nvr + vslot * VD + c0;
    if (l.lv[b] != 0.0f) {
      const float* kr = &l.qk[b][1][rb * 16];
      const float* qr = &l.qk[b][0][rb * 16];
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) acc = kr[i] != 0.0f ? acc + s[i] * kr[i] : acc;
      l.bsk[rb * QW + c] = acc;
      lds_barrier();
      if (t < QW) {
        float kv = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) kv = kv + l.bsk[q * QW + t];
        l.dl[t] = (l.vb[b][t] - kv) * beta;
      }
      lds_barrier();
      const float d = l.dl[c];
      float o = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        s[i] = kr[i] != 0.0f ? s[i] + kr[i] * d : s[i];
        o = qr[i] != 0.0f ? o + s[i] * qr[i] : o;
      }
      l.bso[rb * QW + c] = o;
      lds_barrier();
      if (t < QW) {
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) q = q + l.bso[j * QW + t];
        o_out[t] = bf16r(q);
      }
    } else if (t < QW) {
      o_out[t] = 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; i++) S[i * VD] = s[i];
}
// every live channel's window after the batch: its last 4 inputs (the step's shift, n times);
// thread i0 of ni takes channels i0, i0 + ni, ...
__device__ __forceinline__ void win_after(uint16_t* conv, const float* __restrict__ P, int nproj,
                                          int n, int nk, int kl, int rl, int R, int i0, int ni) {
  const int nq = nk * kl, nch = 2 * nq + nk * rl * VD;
  for (int i = i0; i < nch; i += ni) {
    int64_t wch;
    if (i < 2 * nq) {
      const int part = i / nq, j = i % nq, kh = j / kl, d = j % kl;
      wch = (int64_t)part * nk * KD + kh * KD + d;
    } else {
      const int j = i - 2 * nq, vslot = j / VD, d = j % VD;
      const int vh = (vslot / rl) * R + vslot % rl;
      wch = 2 * (int64_t)nk * KD + (int64_t)vh * VD + d;
    }
    uint64_t* w = reinterpret_cast<uint64_t*>(conv + wch * 4);
    const uint64_t old = *w;
    uint64_t nw = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int idx = n - 4 + j;
      const uint64_t v = idx >= 0 ? (uint64_t)(fbits(P[(int64_t)idx * nproj + i]) >> 16)
                                  : (old >> (16 * (idx + 4))) & 0xffffu;
      nw |= v << (16 * j);
    }
    *w = nw;
  }
}
// every token's gated norm of the live heads (the step's, 4 waves) into ys, interleaved for G =
// gv; then (the delta rule having read them) the windows' advance
__global__ __launch_bounds__(PBT) void pb_gnorm(const float* __restrict__ o,
                                                const float* __restrict__ P, int nproj, int zoff,
                                                const float* __restrict__ gw, float geps, int nh,
                                                int gv, uint16_t* ys, uint16_t* conv, int n, int nk,
                                                int kl, int rl, int R) {
  __shared__ float y[4096];
  const int b = blockIdx.x, nvr = nh * VD;
  const DnOut d{nullptr, 0, nh, o + (int64_t)b * nvr, P + (int64_t)b * nproj + zoff, gw, geps,
                nullptr, nullptr, nullptr, 0, 0};
  gated_norm<PBT / 64, false>(d, y);
  lds_barrier();
  for (int c = tid(); c < nvr; c += PBT) ys[(int64_t)b * nvr + il(c, gv)] = bf16_bits(y[c]);
  win_after(conv, P, nproj, n, nk, kl, rl, R, blockIdx.x * PBT + tid(), gridDim.x * PBT);
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
// the residual's rows: x from a vector
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

static bool dims_ok(const lxm_dn_params* ph) {
  return ph && ph->hidden > 0 && ph->hidden <= 4096 && ph->kl > 0 && ph->kl <= KD && ph->nk > 0 &&
         ph->nv % ph->nk == 0 && ph->rl > 0 && ph->nk * ph->rl <= 32 && ph->layers &&
         ph->layers_host;
}

extern "C" int lxm_dn_step(const lxm_dn_params* ph, const lxm_dn_params* pd, void* stream) {
  if (!dims_ok(ph)) return (int)hipErrorInvalidValue;
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

// the persistent run's instances: (hidden, live value dims, inter) / 64
template <int GH, int GV, int GI>
static int launch_run(const lxm_dn_params* pd, int n, int nblk, hipStream_t st) {
  void* args[] = {(void*)&pd, (void*)&n};
  return (int)hipLaunchCooperativeKernel((const void*)dn_run<GH, GV, GI>, dim3(nblk), dim3(NT),
                                         args, 0, st);
}

extern "C" int lxm_dn_run(const lxm_dn_params* ph, const lxm_dn_params* pd, int n, void* stream) {
  if (!dims_ok(ph) || !ph->sync || n < 1) return (int)hipErrorInvalidValue;
  int dev = 0, n_cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&n_cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return (int)e;
  // one workgroup per CU; the delta rule's tiles need nk x rl x QC of them
  if (n_cus < ph->nk * ph->rl * QC) return (int)hipErrorInvalidConfiguration;
  hipStream_t st = (hipStream_t)stream;
  const int gh = g_of(ph->hidden), gv = g_of(ph->nk * ph->rl * VD), gi = g_of(ph->inter);
  if (gh == 40 && gv == 64 && gi == 144) return launch_run<40, 64, 144>(pd, n, n_cus, st);
  if (gh == 4 && gv == 8 && gi == 8) return launch_run<4, 8, 8>(pd, n, n_cus, st);
  return (int)hipErrorInvalidValue;
}

// the batched prefill's row kernels: R rows per wave (MODE 2: R / 2 units), 4 waves per workgroup
template <int G, int R, int MODE>
static void launch_pb(const uint16_t* W, const uint16_t* W2, int nrows, const uint16_t* X, int n,
                      void* out, int ldo, int og, hipStream_t st) {
  const int per = (PBT / 64) * (MODE == 2 ? R / 2 : R);
  hipLaunchKernelGGL((pb_rows<G, R, MODE>), dim3((nrows + per - 1) / per), dim3(PBT), 0, st, W, W2,
                     nrows, X, n, out, ldo, og);
}
// the residual's long rows: 8 rows per workgroup, the batch's tokens split over its 4 waves
template <int G>
static void launch_hrows(const uint16_t* W, int nrows, const uint16_t* X, int n, float* out, int ldo,
                         hipStream_t st) {
  constexpr int R = 8;
  hipLaunchKernelGGL((pb_hrows<G, R, 1>), dim3((nrows + R - 1) / R), dim3(PBT), 0, st, W, nrows, X,
                     n, out, ldo);
}
// (G of the hidden rows, live value dims, inter) = (40, 64, 144) or (4, 8, 8)
template <int GH, int GV, int GI>
static void pb_layer(const lxm_dn_params* ph, const lxm_dn_layer& ly, const lxm_dn_pbuf* pb, int n,
                     hipStream_t st) {
  const int H = ph->hidden, I = ph->inter, nk = ph->nk, kl = ph->kl, rl = ph->rl, R = ph->nv / nk;
  const int nq = nk * kl, nvr = nk * rl * VD, nproj = 2 * nq + 2 * nvr + 2 * nk * rl;
  const float eps = ph->rms_eps;
  hipLaunchKernelGGL(pb_norm, dim3(n), dim3(NT), 0, st, pb->h, ly.ln_in, eps, H, GH, pb->xn);
  launch_pb<GH, 8, 0>(ly.proj, nullptr, nproj, pb->xn, n, pb->P, nproj, 0, st);
  const PbGdn g{ly.conv_qk, ly.conv_v, ly.A_log, ly.dt_bias, ly.rec, ly.conv, pb->P, pb->qk,
                pb->v, pb->g, pb->live, pb->o, nk, kl, rl, R, nproj, n, nullptr};
  hipLaunchKernelGGL(pb_prep, dim3(n, nk), dim3(KD), 0, st, g);
  hipLaunchKernelGGL(pb_gdn, dim3(nk * rl * QC), dim3(NT), 0, st, g);
  hipLaunchKernelGGL(pb_gnorm, dim3(n), dim3(PBT), 0, st, pb->o, pb->P, nproj, 2 * nq + nvr,
                     ly.gnorm, ph->geps, nk * rl, GV, pb->ys, ly.conv, n, nk, kl, rl, R);
  launch_hrows<GV>(ly.out, H, pb->ys, n, pb->h, H, st);
  hipLaunchKernelGGL(pb_norm, dim3(n), dim3(NT), 0, st, pb->h, ly.ln_post, eps, H, GH, pb->xn);
  // (SwiGLU: 2 units per wave, 1,152 workgroups at 3 per CU; with 4 units per wave its 576
  // workgroups took two rounds of 512, 44 us against 34)
  launch_pb<GH, 4, 2>(ly.gate, ly.up, I, pb->xn, n, pb->act, I, GI, st);
  launch_hrows<GI>(ly.down, H, pb->act, n, pb->h, H, st);
}

extern "C" int lxm_dn_prefill(const lxm_dn_params* ph, const int32_t* tokens, int T,
                              const lxm_dn_pbuf* pb, void* stream) {
  if (!dims_ok(ph) || !pb || !tokens || T < 0) return (int)hipErrorInvalidValue;
  const int gh = g_of(ph->hidden), gv = g_of(ph->nk * ph->rl * VD), gi = g_of(ph->inter);
  const bool full = gh == 40 && gv == 64 && gi == 144, small = gh == 4 && gv == 8 && gi == 8;
  if (!full && !small) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  for (int b0 = 0; b0 < T; b0 += PB) {
    const int n = T - b0 < PB ? T - b0 : PB;
    hipLaunchKernelGGL(pb_embed, dim3(n), dim3(PBT), 0, st, ph->embed, tokens + b0, ph->hidden,
                       ph->vocab, pb->h, ph->err);
    for (int L = 0; L < ph->n_layers; L++) {
      if (full) pb_layer<40, 64, 144>(ph, ph->layers_host[L], pb, n, st);
      else pb_layer<4, 8, 8>(ph, ph->layers_host[L], pb, n, st);
    }
  }
  return (int)hipGetLastError();
}

// The stock forward's prompt (the T > 1 path: Qwen3_5GatedDeltaNet.forward :517-529 calls
// torch_chunk_gated_delta_rule): super-batches of up to LXM_CHUNK tokens, each a chunk of the
// chunked delta rule (lxm_gdn_chunk, MFMA), the row kernels run on its PB-token slices. Every
// other sum keeps the step's order; the delta rule's outputs and states are the chunked form's.
template <int GH, int GV, int GI>
static hipError_t pc_layer(const lxm_dn_params* ph, const lxm_dn_layer& ly, const lxm_dn_pbuf* pb,
                           int n, hipStream_t st) {
  const int H = ph->hidden, I = ph->inter, nk = ph->nk, kl = ph->kl, rl = ph->rl, R = ph->nv / nk;
  const int nq = nk * kl, nvr = nk * rl * VD, nproj = 2 * nq + 2 * nvr + 2 * nk * rl;
  const float eps = ph->rms_eps;
  hipLaunchKernelGGL(pb_norm, dim3(n), dim3(NT), 0, st, pb->h, ly.ln_in, eps, H, GH, pb->xn);
  for (int s = 0; s < n; s += PB)
    launch_pb<GH, 8, 0>(ly.proj, nullptr, nproj, pb->xn + (int64_t)s * H, n - s < PB ? n - s : PB,
                        pb->P + (int64_t)s * nproj, nproj, 0, st);
  const PbGdn g{ly.conv_qk, ly.conv_v, ly.A_log, ly.dt_bias, ly.rec, ly.conv, pb->P, pb->qk,
                pb->v, pb->g, pb->live, pb->o, nk, kl, rl, R, nproj, n, pb->gl};
  hipLaunchKernelGGL(pb_prep, dim3(n, nk), dim3(KD), 0, st, g);
  lxm_chunk_io io;
  io.q = pb->qk;
  io.k = pb->qk + KD;
  io.v = pb->v;
  io.beta = pb->g;
  io.g = pb->gl;
  io.S = ly.rec;
  io.o = pb->o;
  io.qk_ts = (int64_t)nk * 2 * KD;
  io.qk_hs = 2 * KD;
  io.v_ts = nvr;
  io.g_ts = 2 * (int64_t)nk * rl;
  io.g_hs = 2;
  io.gl_ts = (int64_t)nk * rl;
  io.o_ts = nvr;
  io.n = n;
  io.n_slots = nk * rl;
  io.rl = rl;
  io.rfull = R;
  io.kl = kl;
  io.o_bf16 = 1;
  const int e = lxm_gdn_chunk(&io, st);
  if (e) return (hipError_t)e;
  hipLaunchKernelGGL(pb_gnorm, dim3(n), dim3(PBT), 0, st, pb->o, pb->P, nproj, 2 * nq + nvr,
                     ly.gnorm, ph->geps, nk * rl, GV, pb->ys, ly.conv, n, nk, kl, rl, R);
  for (int s = 0; s < n; s += PB)
    launch_hrows<GV>(ly.out, H, pb->ys + (int64_t)s * nvr, n - s < PB ? n - s : PB,
                     pb->h + (int64_t)s * H, H, st);
  hipLaunchKernelGGL(pb_norm, dim3(n), dim3(NT), 0, st, pb->h, ly.ln_post, eps, H, GH, pb->xn);
  for (int s = 0; s < n; s += PB)
    launch_pb<GH, 4, 2>(ly.gate, ly.up, I, pb->xn + (int64_t)s * H, n - s < PB ? n - s : PB,
                        pb->act + (int64_t)s * I, I, GI, st);
  for (int s = 0; s < n; s += PB)
    launch_hrows<GI>(ly.down, H, pb->act + (int64_t)s * I, n - s < PB ? n - s : PB,
                     pb->h + (int64_t)s * H, H, st);
  return hipGetLastError();
}

extern "C" int lxm_dn_prefill_chunked(const lxm_dn_params* ph, const int32_t* tokens, int T,
                                      const lxm_dn_pbuf* pb, void* stream) {
  if (!dims_ok(ph) || !pb || !pb->gl || !tokens || T < 0 || ph->kl > 128 || ph->kl % 16)
    return (int)hipErrorInvalidValue;
  const int gh = g_of(ph->hidden), gv = g_of(ph->nk * ph->rl * VD), gi = g_of(ph->inter);
  const bool full = gh == 40 && gv == 64 && gi == 144, small = gh == 4 && gv == 8 && gi == 8;
  if (!full && !small) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  for (int b0 = 0; b0 < T; b0 += LXM_CHUNK) {
    const int n = T - b0 < LXM_CHUNK ? T - b0 : LXM_CHUNK;
    hipLaunchKernelGGL(pb_embed, dim3(n), dim3(PBT), 0, st, ph->embed, tokens + b0, ph->hidden,
                       ph->vocab, pb->h, ph->err);
    for (int L = 0; L < ph->n_layers; L++) {
      const hipError_t e = full ? pc_layer<40, 64, 144>(ph, ph->layers_host[L], pb, n, st)
                                : pc_layer<4, 8, 8>(ph, ph->layers_host[L], pb, n, st);
      if (e != hipSuccess) return (int)e;
    }
  }
  return (int)hipGetLastError();
}
