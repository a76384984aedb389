// linuxformer's chip-layer greedy decode as one persistent kernel for MI355X (gfx950).
//
// What it computes is lx.mega's decode (lx/csrc/mega.cu:653-862): per token, the embedding row,
// every chip layer's Gated DeltaNet step and SwiGLU MLP, the final norm and the tied head's
// argmax, fed back as the next input on the GPU; conv windows and recurrent states updated in
// place. How it computes it is MI355X's own design:
//
// * The dependent chain of a token (37 layers, each: RMSNorm, the write gates' check, the MLP,
//   and rarely the delta rule) runs inside ONE workgroup (block 0, "the chain"): the residual
//   stream lives in its LDS and every layer's resident tables (norm weights, MLP rows, the
//   query/key/decay rows the gates read) are streamed into LDS one layer ahead through
//   registers. A grid barrier costs ~4 us across MI355X's 8 XCDs (measured), so the reference's
//   ~38 barriered phases per token would cost more than its whole H100 step; here a token
//   crosses the grid once.
// * The output head (459,982 rows) is spread over the other 255 workgroups ("helpers"), each
//   holding its rows' sparse entries in LDS for the whole launch. The chain publishes the
//   final normed residual (agent-scope atomic stores, then a relaxed flag), every helper
//   reduces its rows to one argmax key and folds it into a 64-bit atomicMax, then counts
//   itself done; the chain waits for the count. Keys order by (value, lower index) as
//   torch.argmax breaks ties.
// * Gates instead of speculation: the chain computes, for each layer, the query/key channels'
//   conv outputs and the decays first (a few rows), so it knows exactly whether the layer's
//   delta rule runs and whether it changes the residual. Nothing is ever redone. The conv
//   windows are not shifted channel by channel every step: the chain keeps the last four
//   tokens' GDN norm outputs per layer (a ring in HBM), recomputes the few windows an active
//   head needs from them, keeps its query/key channels' windows in LDS, and writes every
//   window once at the end of the launch.
//
// Arithmetic: the rounding contract of lxm_math.h; sums in the orders documented per site.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lxm.h"
#include "lxm_math.h"

using namespace lxm;

#define NT LXM_NT
#define NW (NT / 64)
#define MAXH LXM_MAXH
#define KD LXM_KD
#define VD LXM_VD
#define RMAX LXM_RMAX
#define TIMEOUT_TICKS 300000000ull  // 3 s of the 100 MHz wall clock

// ---------------------------------------------------------------------------------------------
// LDS layout of the chain workgroup (bytes)
#define L_HOT 0
#define L_H (L_HOT + LXM_HOT_MAX)
#define L_XM (L_H + 4 * MAXH)
#define L_ACT (L_XM + 4 * MAXH)
#define L_HIST (L_ACT + 4 * LXM_MAXU)
#define L_QKCUR (L_HIST + 4 * 3 * LXM_MAXQK)
#define L_QD (L_QKCUR + 4 * LXM_MAXQKL)
#define L_KDV (L_QD + 4 * KD)
#define L_QN (L_KDV + 4 * KD)
#define L_KN (L_QN + 4 * KD)
#define L_NZQ (L_KN + 4 * KD)
#define L_NZK (L_NZQ + 4 * KD)
#define L_VB (L_NZK + 4 * KD)
#define L_OB (L_VB + 4 * RMAX * VD)
#define L_ZB (L_OB + 4 * RMAX * VD)
#define L_EV (L_ZB + 4 * RMAX * VD)
#define L_BETA (L_EV + 4 * 256)
#define L_WSUM (L_BETA + 4 * RMAX)
#define L_FLAGS (L_WSUM + 4 * 32)
#define L_PROF (L_FLAGS + 4 * 256)
#define L_XG (L_PROF + 8 * 32)
#define L_CHAIN_END (L_XG + 4 * MAXH)
// flags (int): [0] any head active, [1] any output, [2] nq, [3] nk, [4] scratch, [8] token
// [16 + kh] per key head: bit 0 query nonzero, bit 1 key nonzero, bit 2 decay
#define F_ANY 0
#define F_OUT 1
#define F_NQ 2
#define F_NK 3
#define F_OK 4
#define F_TOK 8
#define F_KH 16

// sync words (uint32, 128-byte apart groups)
#define S_TOKFLAG 0
#define S_COUNT 32
#define S_DONE 64
#define S_ERRSEEN 96

__device__ __forceinline__ uint32_t ld_rlx(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_rlx(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_rlxf(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_rlxf(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// every earlier memory op of this wave has completed (its stores are visible at agent scope
// when they were agent-scope atomics)
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint64_t wall() { return __builtin_amdgcn_s_memrealtime(); }

// global-address-space views of generic pointers: loads and stores through them are
// global_load/global_store (flat ones would also count against lgkmcnt, i.e. LDS waits)
#define GAS __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ GAS T* gp(T* q) {
  return (GAS T*)q;
}
template <class T>
__device__ __forceinline__ const GAS T* gp(const T* q) {
  return (const GAS T*)q;
}

// a workgroup barrier ordering LDS only: global loads in flight (the next layer's tables)
// stay in flight across it
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// In-kernel phase counters (lx/csrc/mega.cu's prof buffer and MK_SUBPROF checkpoints): with
// p.prof set, thread 0 of the chain adds the shader-clock cycles of each phase into an LDS
// slot; the slots are written to p.prof at the end. Phases: 0 embedding, 1 layer staging (and
// the trace), 2 the norms (stage A), 3 the gates and the MLP units (stage B), 4 active heads
// and the MLP's redo, 5 down_proj and the next norm's sums (stage C), 6 final norm + publish,
// 7 waiting for the head's argmax; counters 16 active layer-steps, 17 tokens.
#define PROF_ON (p.prof != nullptr)
__device__ __forceinline__ uint64_t cycles() { return __builtin_readcyclecounter(); }

// spin (one thread) until *p >= target; false on timeout or another block's error
__device__ bool spin_ge(const uint32_t* p, uint32_t target, int32_t* err, int code) {
  const uint64_t t0 = wall();
  while (ld_rlx(p) < target) {
    __builtin_amdgcn_s_sleep(1);
    if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    if (wall() - t0 > TIMEOUT_TICKS) {
      __hip_atomic_fetch_max(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------------------
// packed entries
template <bool BF>
struct Ent;
template <>
struct Ent<true> {
  static constexpr int SZ = 4;
  __device__ static __forceinline__ void at(const uint8_t* base, int64_t e, int& idx, float& v) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(base)[e];
    idx = (int)(w & 0xffffu);
    v = bf16f(w >> 16);
  }
};
template <>
struct Ent<false> {
  static constexpr int SZ = 8;
  __device__ static __forceinline__ void at(const uint8_t* base, int64_t e, int& idx, float& v) {
    const uint2 w = reinterpret_cast<const uint2*>(base)[e];
    idx = (int)w.x;
    v = __uint_as_float(w.y);
  }
};

// sum over a row's entries of x[idx] * w, in entry order from +0 (terms with x == 0 skipped,
// which leaves the sum's bits unchanged: a sum from +0 never yields -0)
template <bool E4>
__device__ __forceinline__ float dot_row(const uint8_t* ent, int64_t start, int len, const float* x) {
  float s = 0.0f;
  for (int k = 0; k < len; k++) {
    int i;
    float w;
    Ent<E4>::at(ent, start + k, i, w);
    const float xv = x[i];
    if (xv != 0.0f) s = s + xv * w;
  }
  return s;
}

// the 512-lane hidden sum: lane t's partial (its elements t, t + 512, ... in order), combined
// within each wave at offsets 32..1, the 8 wave totals at offsets 4, 2, 1. All threads call;
// all get the sum.
__device__ __forceinline__ float sum512(float s, float* wsum) {
  for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_down(s, off, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  lds_barrier();
  float w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
  lds_barrier();
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}

// the 64-lane head sum over one wave: lane l's partial (elements l, l + 64, ...), offsets
// 32..1; every lane gets the sum
__device__ __forceinline__ float sum64(float s) {
  for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_down(s, off, 64);
  return __shfl(s, 0, 64);
}

// ATen's CPU order for a sum over the state's rows (torch .sum(-2)): blocks of 16 rows, each
// block in order from +0, the block sums in order from +0; rows given ascending
__device__ __forceinline__ float row_cascade(const float* S, int j, const int* rows, int n,
                                             const float* f) {
  float tot = 0.0f, bs = 0.0f;
  int blk = -1;
  for (int a = 0; a < n; a++) {
    const int r = rows[a];
    if ((r >> 4) != blk) {
      if (blk >= 0) tot = tot + bs;
      bs = 0.0f;
      blk = r >> 4;
    }
    bs = bs + S[(size_t)r * VD + j] * f[r];
  }
  if (blk >= 0) tot = tot + bs;
  return tot;
}

// ---------------------------------------------------------------------------------------------
template <bool E4>
__device__ __forceinline__ float w1_at(const uint8_t* hot, int off, int c) {
  if constexpr (E4) {
    const float w = bf16f(reinterpret_cast<const uint16_t*>(hot + off)[c]);
    return 1.0f + w;
  } else {
    return reinterpret_cast<const float*>(hot + off)[c];
  }
}

// a conv state value (model dtype) as float
template <bool BF>
__device__ __forceinline__ float conv_at(const void* cs, int64_t i) {
  if constexpr (BF) return bf16f(reinterpret_cast<const uint16_t*>(cs)[i]);
  else return reinterpret_cast<const float*>(cs)[i];
}
template <bool BF>
__device__ __forceinline__ void conv_put(void* cs, int64_t i, float v) {
  if constexpr (BF) reinterpret_cast<uint16_t*>(cs)[i] = (uint16_t)(__float_as_uint(v) >> 16);
  else reinterpret_cast<float*>(cs)[i] = v;
}

// ---------------------------------------------------------------------------------------------
// The chain workgroup. Its LDS arrays are addressed from the dynamic shared array itself, so
// every access is a ds_read/ds_write.
extern __shared__ __align__(16) uint8_t smem[];
#define LF(off) reinterpret_cast<float*>(smem + (off))
#define LI(off) reinterpret_cast<int*>(smem + (off))

// Qwen3_5RMSNorm's r = rsqrt(mean(h^2) + eps) (transformers qwen3_5 :727), mean = sum / n
__device__ __forceinline__ float norm_r(float ss, int H, float eps) {
  return rsqrt_(ss / (float)H + eps);
}
__device__ __forceinline__ float hidden_ss(int H) {
  const float* h = LF(L_H);
  float s = 0.0f;
  for (int c = threadIdx.x; c < H; c += NT) s = s + h[c] * h[c];
  return sum512(s, LF(L_WSUM));
}

// stage layer L's hot blob: global -> registers (fetch, one layer ahead) -> LDS (stage); eight
// 16-byte words per thread, kept in named registers
static_assert(LXM_HOT_MAX == 16 * NT * 8, "the prefetch holds 8 words per thread");
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
struct Pf {
  v4u w0, w1, w2, w3, w4, w5, w6, w7;
};
__device__ __forceinline__ Pf fetch(const lxm_params& p, int L, int n16) {
  const GAS v4u* src = gp(reinterpret_cast<const v4u*>(p.blob + p.layers[L].hot));
  const int t = threadIdx.x;
  // words past the blob: a duplicate of word 0, never staged
#define PF_LD(k) src[t + (k) * NT < n16 ? t + (k) * NT : 0]
  Pf r;
  r.w0 = PF_LD(0);
  r.w1 = PF_LD(1);
  r.w2 = PF_LD(2);
  r.w3 = PF_LD(3);
  r.w4 = PF_LD(4);
  r.w5 = PF_LD(5);
  r.w6 = PF_LD(6);
  r.w7 = PF_LD(7);
#undef PF_LD
  return r;
}
__device__ __forceinline__ void stage(int n16, const Pf& r) {
  v4u* dst = reinterpret_cast<v4u*>(smem + L_HOT);
  const int t = threadIdx.x;
#define PF_ST(k, w) \
  if (t + (k) * NT < n16) dst[t + (k) * NT] = r.w
  PF_ST(0, w0);
  PF_ST(1, w1);
  PF_ST(2, w2);
  PF_ST(3, w3);
  PF_ST(4, w4);
  PF_ST(5, w5);
  PF_ST(6, w6);
  PF_ST(7, w7);
#undef PF_ST
}

template <bool BF, bool E4>
__device__ void gdn_active(const lxm_params& p, int L, int step);

// One chunk of up to 4 entries of a row (entries k0 .. k0 + 3 of start .. start + n): the sum
// continues in entry order; all loads of the chunk are issued together.
template <bool E4>
__device__ __forceinline__ float chunk4(const uint8_t* ent, int start, int n, int k0,
                                        const float* x, float s) {
  int i[4];
  float w[4], xv[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    i[j] = 0;
    w[j] = 0.0f;
    if (k0 + j < n) Ent<E4>::at(ent, start + k0 + j, i[j], w[j]);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) xv[j] = x[i[j]];
#pragma unroll
  for (int j = 0; j < 4; j++)
    if (k0 + j < n && xv[j] != 0.0f) s = s + xv[j] * w[j];
  return s;
}
template <bool E4>
__device__ __forceinline__ float rest4(const uint8_t* ent, int start, int n, const float* x,
                                       float s) {
  for (int k0 = 4; k0 < n; k0 += 4) s = chunk4<E4>(ent, start, n, k0, x, s);
  return s;
}

// silu and the MLP product for one unit (Qwen3_5MLP :715): D(D(silu(D(g))) * D(u))
template <bool BF>
__device__ __forceinline__ float swiglu(float gs, float us) {
  const float g = rd<BF>(gs), up = rd<BF>(us);
  const float sg = g == 0.0f ? g : silu(g);  // silu(+-0) = +-0 / 2 = +-0
  return rd<BF>(rd<BF>(sg) * up);
}

// The MLP's gate and up rows of every unit: act[u]. Two units a thread, their first chunks
// issued together.
template <bool BF, bool E4>
__device__ __forceinline__ void mlp_units(const lxm_hot& hd, const uint8_t* hot) {
  const int t = threadIdx.x;
  const float* xm = LF(L_XM);
  float* act = LF(L_ACT);
  const uint32_t* um = reinterpret_cast<const uint32_t*>(hot + hd.unit);
  const uint8_t* gu = hot + hd.gu_ent;
  for (int u = t; u < hd.n_units; u += 2 * NT) {
    const int u2 = u + NT;
    const bool two = u2 < hd.n_units;
    const uint32_t m1 = um[u], m2 = two ? um[u2] : 0u;
    const int s1 = (int)(m1 & 0xffffu), g1 = (int)((m1 >> 16) & 255), n1 = (int)(m1 >> 24);
    const int s2 = (int)(m2 & 0xffffu), g2 = (int)((m2 >> 16) & 255), n2 = (int)(m2 >> 24);
    float ag = chunk4<E4>(gu, s1, g1, 0, xm, 0.0f);
    float au = chunk4<E4>(gu, s1 + g1, n1, 0, xm, 0.0f);
    float bg = chunk4<E4>(gu, s2, g2, 0, xm, 0.0f);
    float bu = chunk4<E4>(gu, s2 + g2, n2, 0, xm, 0.0f);
    ag = rest4<E4>(gu, s1, g1, xm, ag);
    au = rest4<E4>(gu, s1 + g1, n1, xm, au);
    bg = rest4<E4>(gu, s2, g2, xm, bg);
    bu = rest4<E4>(gu, s2 + g2, n2, xm, bu);
    act[u] = swiglu<BF>(ag, au);
    if (two) act[u2] = swiglu<BF>(bg, bu);
  }
}

// The gates: the live query/key channels' projections, conv windows (history in LDS) and silu
// (causal_conv1d_update :199-216), and the decays g = -exp(A_log) softplus(a + dt_bias) (:499).
// Flags per key head: 1 query nonzero, 2 key nonzero, 4 a decay exp(g) != 1. Items run on the
// threads from the top down (the units take them from the bottom up).
template <bool BF, bool E4>
__device__ __forceinline__ void gates(const lxm_params& p, const lxm_hot& hd, const uint8_t* hot) {
  const int tt = NT - 1 - (int)threadIdx.x;
  const float* xg = LF(L_XG);
  float* hist = LF(L_HIST);
  float* qkcur = LF(L_QKCUR);
  float* ev = LF(L_EV);
  int* flags = LI(L_FLAGS);
  const lxm_qkc* qk = reinterpret_cast<const lxm_qkc*>(hot + hd.qk);
  const uint8_t* ent = hot + hd.ent;
  for (int j = tt; j < hd.n_qk; j += NT) {
    const lxm_qkc c = qk[j];
    const float P = rd<BF>(rest4<E4>(ent, c.start, c.len, xg, chunk4<E4>(ent, c.start, c.len, 0, xg, 0.0f)));
    float* hs = hist + 3 * (hd.qk_base + j);
    float y = 0.0f;
    y = y + c.taps[0] * hs[0];
    y = y + c.taps[1] * hs[1];
    y = y + c.taps[2] * hs[2];
    y = y + c.taps[3] * P;
    hs[0] = hs[1];
    hs[1] = hs[2];
    hs[2] = P;
    const float yr = rd<BF>(y);
    const float v = yr == 0.0f ? yr : rd<BF>(silu(yr));
    qkcur[j] = v;
    if (v != 0.0f) atomicOr(&flags[F_KH + (c.slot >> 9)], (c.slot & 256) ? 2 : 1);
  }
  const lxm_dec* dc = reinterpret_cast<const lxm_dec*>(hot + hd.dec);
  for (int j = ((tt - hd.n_qk) % NT + NT) % NT; j < hd.n_dec; j += NT) {
    const lxm_dec d = dc[j];
    const float a = rd<BF>(rest4<E4>(ent, d.start, d.len, xg, chunk4<E4>(ent, d.start, d.len, 0, xg, 0.0f)));
    const float x = a + d.dt_bias;
    float e;
    if (x < -104.0f && d.A_log <= 88.0f) {
      e = 1.0f;  // exp(x) rounds to 0, so softplus is 0 and g = -exp(A_log) * 0 = -0
    } else {
      const float g = (-cr_exp(d.A_log)) * softplus(x);
      e = cr_exp(g);
    }
    ev[d.vh] = e;
    if (e != 1.0f) atomicOr(&flags[F_KH + d.vh / (p.nv / p.nk)], 4);
  }
}

// stage A's norm: r = rsqrt(mean(h^2) + eps) (transformers qwen3_5 :727, mean = sum / n); both
// norms' inputs D((h * r) * (1 + w)) (:729-734) from one h * r; the GDN norm's output also to the
// ring. Only the MLP's when gdn is false (the redo after a delta rule that wrote h).
template <bool BF, bool E4>
__device__ __forceinline__ void norms(const lxm_params& p, const lxm_hot& hd, const uint8_t* hot,
                                      int L, int step, float r, bool gdn) {
  const int H = p.hidden;
  const float* h = LF(L_H);
  float* xg = LF(L_XG);
  float* xm = LF(L_XM);
  GAS float* ring = gp(p.ring + ((size_t)(step & 3) * p.n_layers + L) * H);
  for (int c = threadIdx.x; c < H; c += NT) {
    const float hr = h[c] * r;
    xm[c] = rd<BF>(hr * w1_at<E4>(hot, hd.w1_post, c));
    if (gdn) {
      const float g = rd<BF>(hr * w1_at<E4>(hot, hd.w1_in, c));
      xg[c] = g;
      ring[c] = g;
    }
  }
}

// One layer. ss: the sum of squares of h on entry; returns it for the layer's output.
template <bool BF, bool E4>
__device__ __forceinline__ float layer(const lxm_params& p, int L, int step, float ss) {
  const int t = threadIdx.x, H = p.hidden;
  const uint8_t* hot = smem + L_HOT;
  const lxm_hot hd = *reinterpret_cast<const lxm_hot*>(hot);
  float* h = LF(L_H);
  float* act = LF(L_ACT);
  float* ev = LF(L_EV);
  int* flags = LI(L_FLAGS);
  uint64_t* pa = reinterpret_cast<uint64_t*>(smem + L_PROF);
  // ---- stage A: both norms (the GDN's input_layernorm :764 and the MLP's
  // post_attention_layernorm :789 read the same h when the GDN leaves it alone)
  const float r = norm_r(ss, H, hd.eps);
  norms<BF, E4>(p, hd, hot, L, step, r, true);
  if (t < p.nk) flags[F_KH + t] = 0;
  if (t < p.nv) ev[t] = 1.0f;
  if (t == 0) flags[F_ANY] = 0;
  lds_barrier();
  uint64_t c0 = 0;
  if (PROF_ON && t == 0) {
    c0 = cycles();
    pa[2] += c0 - pa[15];
  }
  // ---- stage B: the gates and, speculatively (the GDN leaves h alone on most steps), the MLP
  mlp_units<BF, E4>(hd, hot);
  gates<BF, E4>(p, hd, hot);
  lds_barrier();
  if (t < p.nk && flags[F_KH + t]) atomicOr(&flags[F_ANY], 1);
  lds_barrier();
  if (PROF_ON && t == 0) {
    const uint64_t c1 = cycles();
    pa[3] += c1 - c0;
    c0 = c1;
  }
  if (flags[F_ANY]) {
    gdn_active<BF, E4>(p, L, step);
    if (flags[F_OUT]) {  // h changed: the MLP again, on the new h
      ss = hidden_ss(H);
      norms<BF, E4>(p, hd, hot, L, step, norm_r(ss, H, hd.eps), false);
      lds_barrier();
      mlp_units<BF, E4>(hd, hot);
      lds_barrier();
    }
    if (PROF_ON && t == 0) {
      const uint64_t c1 = cycles();
      pa[4] += c1 - c0;
      pa[16] += 1;
      c0 = c1;
    }
  }
  // ---- stage C: down_proj by residual row (units ascending), the residual add on every row
  // (:791), and this thread's terms of the next sum of squares (rows t, t + 512, ... in order)
  float s2 = 0.0f;
  {
    const uint16_t* dp = reinterpret_cast<const uint16_t*>(hot + hd.down_ptr);
    const uint8_t* de = hot + hd.down_ent;
    int a[8], n[8];
    float d[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = t + k * NT;
      a[k] = 0;
      n[k] = 0;
      if (i < H) {
        a[k] = dp[i];
        n[k] = (int)dp[i + 1] - a[k];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; k++) d[k] = chunk4<E4>(de, a[k], n[k], 0, act, 0.0f);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = t + k * NT;
      if (i < H) {
        const float dk = rd<BF>(rest4<E4>(de, a[k], n[k], act, d[k]));
        const float hv = rd<BF>(h[i] + dk);
        h[i] = hv;
        s2 = s2 + hv * hv;
      }
    }
  }
  const float ssn = sum512(s2, LF(L_WSUM));
  if (PROF_ON && t == 0) {
    const uint64_t c1 = cycles();
    pa[5] += c1 - c0;
    pa[15] = c1;
  }
  return ssn;
}

// The delta rule for the layer's active key heads (torch_recurrent_gated_delta_rule :330-380
// with l2norm :242-245 in the model dtype; Qwen3_5RMSNormGated :175-184; out_proj), adding
// out_proj's output into h. Uniform control flow: every condition is read from LDS after a
// barrier.
template <bool BF, bool E4>
__device__ void gdn_active(const lxm_params& p, int L, int step) {
  using E = Ent<E4>;
  const int t = threadIdx.x, H = p.hidden;
  const uint8_t* hot = smem + L_HOT;
  const lxm_hot hd = *reinterpret_cast<const lxm_hot*>(hot);
  float* h = LF(L_H);
  float* xm = LF(L_XM);
  float* qkcur = LF(L_QKCUR);
  float* qd = LF(L_QD);
  float* kdv = LF(L_KDV);
  float* qn = LF(L_QN);
  float* kn = LF(L_KN);
  int* nzq = LI(L_NZQ);
  int* nzk = LI(L_NZK);
  float* vb = LF(L_VB);
  float* ob = LF(L_OB);
  float* zb = LF(L_ZB);
  float* ev = LF(L_EV);
  float* beta = LF(L_BETA);
  int* flags = LI(L_FLAGS);
  const lxm_layer ly = p.layers[L];
  const uint8_t* blob = p.blob;
  const int R = p.nv / p.nk;
  const int wv = t >> 6, lane = t & 63;
  float* S0 = p.rec[L];
  const void* cs = p.conv[L];
  const lxm_chan* chans = reinterpret_cast<const lxm_chan*>(blob + ly.chan);
  const uint8_t* qent = blob + ly.qkv_ent;
  const float* xg = LF(L_XG);  // the GDN norm's output (stage A)
  if (t == 0) flags[F_OUT] = 0;
  for (int c = t; c < H; c += NT) xm[c] = 0.0f;  // out_proj's running sums
  __syncthreads();  // and the ring's stores of this step, visible to every thread
  for (int kh = 0; kh < p.nk; kh++) {
    const int fk = flags[F_KH + kh];
    if (!fk) continue;
    // dense query and key of this head (the live channels' conv outputs, zeros elsewhere)
    for (int i = t; i < KD; i += NT) {
      qd[i] = 0.0f;
      kdv[i] = 0.0f;
    }
    __syncthreads();
    {
      const lxm_qkc* qk = reinterpret_cast<const lxm_qkc*>(hot + hd.qk);
      for (int j = t; j < hd.n_qk; j += NT) {
        const int sl = qk[j].slot;
        if ((sl >> 9) != kh) continue;
        ((sl & 256) ? kdv : qd)[sl & 255] = qkcur[j];
      }
    }
    __syncthreads();
    // l2norm in the model dtype: D(x * D(rsqrt(D(D(sum D(x*x)) + 1e-6)))); query scaled by
    // 1/sqrt(256) in fp32 (:352-353); then the nonzero rows in ascending order
    if (wv < 2) {
      const float* x = wv ? kdv : qd;
      float s = 0.0f;
      for (int i = lane; i < KD; i += 64) s = s + rd<BF>(x[i] * x[i]);
      s = rd<BF>(sum64(s));
      const float inv = rd<BF>(rsqrt_(rd<BF>(s + 1e-6f)));
      float* o = wv ? kn : qn;
      int* nz = wv ? nzk : nzq;
      int n = 0;
      for (int b = 0; b < KD; b += 64) {
        float v = rd<BF>(x[b + lane] * inv);
        if (!wv) v = v * 0.0625f;
        o[b + lane] = v;
        const unsigned long long m = __ballot(v != 0.0f);
        if (v != 0.0f) nz[n + __popcll(m & ((1ull << lane) - 1))] = b + lane;
        n += __popcll(m);
      }
      if (lane == 0) flags[wv ? F_NK : F_NQ] = n;
    }
    // beta = sigmoid(b) (:497) for this head's value heads
    if (t >= 128 && t < 128 + R) {
      const int r = t - 128, vh = kh * R + r;
      const lxm_row br = reinterpret_cast<const lxm_row*>(blob + ly.b_row)[vh];
      const float b = rd<BF>(dot_row<E4>(blob + ly.b_ent, br.start, br.len, xg));
      beta[r] = rd<BF>(sigmoid(b));
    }
    __syncthreads();
    const int nq = flags[F_NQ], nk = flags[F_NK];
    // v: this head's value channels' conv outputs; the window's earlier inputs recomputed from
    // the ring (or read from the conv state before this launch)
    if (nk > 0) {
      for (int c = t; c < R * VD; c += NT) {
        const int chan = 2 * p.nk * KD + (kh * R) * VD + c;
        const lxm_chan ch = chans[chan];
        float win[4];
        win[3] = rd<BF>(dot_row<E4>(qent, ch.start, ch.len, xg));
#pragma unroll
        for (int s = 1; s <= 3; s++) {
          win[3 - s] = 0.0f;
          if (ch.taps[3 - s] == 0.0f) continue;
          if (step - s >= 0) {
            const float* xo = p.ring + ((size_t)((step - s) & 3) * p.n_layers + L) * H;
            win[3 - s] = rd<BF>(dot_row<E4>(qent, ch.start, ch.len, xo));
          } else {
            win[3 - s] = conv_at<BF>(cs, (int64_t)chan * 4 + 4 - (s - step));
          }
        }
        float y = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (ch.taps[k] != 0.0f) y = y + ch.taps[k] * win[k];
        vb[c] = rd<BF>(silu(rd<BF>(y)));
      }
    }
    __syncthreads();
    // the recurrent step, one state column per thread: decay, kv, delta, write, output
    for (int r = t >> 7; r < R; r += NT / VD) {
      const int j = t & (VD - 1), vh = kh * R + r;
      float* S = S0 + (size_t)vh * KD * VD;
      const float e = ev[vh];
      if (e != 1.0f)
        for (int i0 = 0; i0 < KD; i0 += 64) {  // 64 loads in flight, then the stores
          float v[64];
#pragma unroll
          for (int k = 0; k < 64; k++) v[k] = S[(size_t)(i0 + k) * VD + j];
#pragma unroll
          for (int k = 0; k < 64; k++) S[(size_t)(i0 + k) * VD + j] = v[k] * e;
        }
      if (nk > 0) {
        const float kv = row_cascade(S, j, nzk, nk, kn);
        const float dl = (vb[r * VD + j] - kv) * beta[r];
        for (int a = 0; a < nk; a++) {
          const int i = nzk[a];
          S[(size_t)i * VD + j] = S[(size_t)i * VD + j] + kn[i] * dl;
        }
      }
      ob[r * VD + j] = nq > 0 ? rd<BF>(row_cascade(S, j, nzq, nq, qn)) : 0.0f;
    }
    __syncthreads();
    if (nq == 0) continue;  // no query: the head's output is exactly zero
    // z = in_proj_z, then the gated norm per value head (one wave each)
    for (int c = t; c < R * VD; c += NT) {
      const lxm_row zr = reinterpret_cast<const lxm_row*>(blob + ly.z_row)[(kh * R) * VD + c];
      zb[c] = rd<BF>(dot_row<E4>(blob + ly.z_ent, zr.start, zr.len, xg));
    }
    __syncthreads();
    {
      const float* gw = reinterpret_cast<const float*>(blob + ly.gnorm);
      for (int r = wv; r < R; r += NW) {
        float s = 0.0f;
        for (int j = lane; j < VD; j += 64) s = s + ob[r * VD + j] * ob[r * VD + j];
        s = sum64(s);
        const float rr = rsqrt_(s / (float)VD + hd.geps);
        for (int j = lane; j < VD; j += 64) {
          const float t1 = rd<BF>(ob[r * VD + j] * rr);
          const float t2 = rd<BF>(gw[j] * t1);
          zb[r * VD + j] = rd<BF>(t2 * silu(zb[r * VD + j]));
        }
      }
    }
    __syncthreads();
    // out_proj rows touched by this head: the running sums continue in ascending dim order
    {
      const int32_t* op = reinterpret_cast<const int32_t*>(blob + ly.out_ptr) + (size_t)kh * (H + 1);
      const uint8_t* oe = blob + ly.out_ent;
      for (int i = t; i < H; i += NT) {
        const int a = op[i], b = op[i + 1];
        if (a == b) continue;
        float s = xm[i];
        for (int k = a; k < b; k++) {
          int d;
          float w;
          E::at(oe, k, d, w);
          const float x = zb[d];
          if (x != 0.0f) s = s + x * w;
        }
        xm[i] = s;
      }
    }
    if (t == 0) flags[F_OUT] = 1;
    __syncthreads();
  }
  // the residual add (all rows; a row with no term adds +0)
  if (flags[F_OUT]) {
    for (int i = t; i < H; i += NT) h[i] = rd<BF>(h[i] + rd<BF>(xm[i]));
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------
template <bool BF, bool E4>
__device__ void run_chain(const lxm_params& p) {
  const int t = threadIdx.x, H = p.hidden;
  int* flags = LI(L_FLAGS);
  float* h = LF(L_H);
  float* hist = LF(L_HIST);
  // the live query/key channels' windows from the conv state (positions 1..3)
  for (int L = 0; L < p.n_layers; L++) {
    const lxm_hot* hd = reinterpret_cast<const lxm_hot*>(p.blob + p.layers[L].hot);
    const lxm_qkc* qk = reinterpret_cast<const lxm_qkc*>(p.blob + p.layers[L].hot + hd->qk);
    for (int j = t; j < hd->n_qk; j += NT)
      for (int s = 0; s < 3; s++)
        hist[3 * (hd->qk_base + j) + s] = conv_at<BF>(p.conv[L], (int64_t)qk[j].chan * 4 + 1 + s);
  }
  int* n16s = flags + 128;  // per layer (< 64): its hot blob's 16-byte words
  for (int L = t; L < p.n_layers; L += NT)
    n16s[L] = reinterpret_cast<const lxm_hot*>(p.blob + p.layers[L].hot)->size / 16;
  __syncthreads();
  Pf pf = fetch(p, 0, n16s[0]);
  uint64_t* pa = reinterpret_cast<uint64_t*>(smem + L_PROF);
  if (t < 32) pa[t] = 0;
  __syncthreads();
  int tok = p.forced[0];
  const uint32_t nh = (uint32_t)(p.n_blocks - 1);
  for (int i = 0; i < p.n_tokens; i++) {
    if (tok < 0 || tok >= p.vocab) tok = 0;  // the host checks forced tokens; preds are in range
    if (t == 0 && p.inputs) p.inputs[i] = tok;
    if (PROF_ON && t == 0) pa[15] = cycles();
    // the input's embedding row
    for (int c = t; c < H; c += NT) h[c] = 0.0f;
    lds_barrier();
    {
      const int64_t a = p.emb_ptr[tok], b = p.emb_ptr[tok + 1];
      for (int64_t e = a + t; e < b; e += NT) {
        int col;
        float w;
        Ent<E4>::at(reinterpret_cast<const uint8_t*>(p.emb_ent), e, col, w);
        h[col] = w;
      }
    }
    lds_barrier();
    float ss = hidden_ss(H);
    if (PROF_ON && t == 0) {
      const uint64_t c = cycles();
      pa[0] += c - pa[15];
      pa[15] = c;
    }
    for (int L = 0; L < p.n_layers; L++) {
      stage(n16s[L], pf);
      lds_barrier();
      const int Ln = L + 1 < p.n_layers ? L + 1 : 0;
      pf = fetch(p, Ln, n16s[Ln]);
      if (PROF_ON && t == 0) {
        const uint64_t c = cycles();
        pa[1] += c - pa[15];
        pa[15] = c;
      }
      ss = layer<BF, E4>(p, L, i, ss);
      if (p.trace) {
        float* tr = p.trace + ((size_t)i * p.n_layers + L) * H;
        for (int c = t; c < H; c += NT) tr[c] = h[c];
      }
      lds_barrier();
      if (PROF_ON && t == 0) {
        const uint64_t c = cycles();
        pa[1] += c - pa[15];
        pa[15] = c;
      }
    }
    // the final norm (lx/lx/hf.py:179-184: model.norm then the tied head), to the helpers
    {
      const float r = norm_r(ss, H, p.rms_eps);
      for (int c = t; c < H; c += NT) st_rlxf(p.hn + c, rd<BF>((h[c] * r) * p.w1_final[c]));
    }
    drain();
    __syncthreads();
    if (PROF_ON && t == 0) {
      const uint64_t c = cycles();
      pa[6] += c - pa[15];
      pa[15] = c;
    }
    if (t == 0) {
      st_rlx(p.sync + S_TOKFLAG, (uint32_t)(i + 1));
      bool ok = spin_ge(p.sync + S_COUNT, nh * (uint32_t)(i + 1), p.err, 1);
      int pred = 0;
      if (ok) {
        const unsigned long long key =
            __hip_atomic_load(p.keys + (i & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pred = argmax_idx(key);
        __hip_atomic_store(p.keys + ((i + 1) & 1), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        p.preds[i] = pred;
      }
      flags[F_OK] = ok;
      flags[F_TOK] = pred;
      if (PROF_ON) {
        const uint64_t c = cycles();
        pa[7] += c - pa[15];
        pa[15] = c;
        pa[17] += 1;
      }
    }
    __syncthreads();
    if (!flags[F_OK]) return;
    tok = i + 1 < p.n_forced ? p.forced[i + 1] : flags[F_TOK];
  }
  if (PROF_ON && t < 32) p.prof[t] = pa[t];
  // every ring write visible to the other blocks, then let them write the conv windows
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (t == 0) __hip_atomic_store(p.sync + S_DONE, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool BF, bool E4>
__device__ void run_helper(const lxm_params& p) {
  uint8_t* lds = smem;
  const int t = threadIdx.x, H = p.hidden, b = blockIdx.x;
  const int r0 = p.head_rows[b], r1 = p.head_rows[b + 1], nr = r1 - r0;
  const int64_t e0 = p.head_ptr[r0], ne = p.head_ptr[r1] - e0;
  int32_t* lptr = reinterpret_cast<int32_t*>(lds);
  uint8_t* lent = lds + (((size_t)(nr + 1) * 4 + 15) & ~(size_t)15);
  float* hn = reinterpret_cast<float*>(lds + p.head_lds);
  unsigned long long* wk = reinterpret_cast<unsigned long long*>(lds + p.head_lds + 4 * MAXH);
  int* ok = reinterpret_cast<int*>(wk + NW);
  for (int k = t; k <= nr; k += NT) lptr[k] = (int32_t)(p.head_ptr[r0 + k] - e0);
  {
    const uint32_t* src = p.head_ent + e0 * (Ent<E4>::SZ / 4);
    uint32_t* dst = reinterpret_cast<uint32_t*>(lent);
    for (int64_t k = t; k < ne * (Ent<E4>::SZ / 4); k += NT) dst[k] = src[k];
  }
  __syncthreads();
  uint64_t hw = 0, hc = 0, hc0 = 0;
  for (int i = 0; i < p.n_tokens; i++) {
    const uint64_t w0 = (PROF_ON && t == 0) ? cycles() : 0;
    if (t == 0) *ok = spin_ge(p.sync + S_TOKFLAG, (uint32_t)(i + 1), p.err, 2);
    __syncthreads();
    if (!*ok) return;
    if (PROF_ON && t == 0) {
      hc0 = cycles();
      hw += hc0 - w0;
    }
    for (int c = t; c < H; c += NT) hn[c] = ld_rlxf(p.hn + c);
    __syncthreads();
    unsigned long long best = 0;
    for (int k = t; k < nr; k += NT) {
      const float v = rd<BF>(dot_row<E4>(lent, lptr[k], lptr[k + 1] - lptr[k], hn));
      const unsigned long long key = argmax_key(v, r0 + k);
      best = key > best ? key : best;
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(best, off, 64);
      best = o > best ? o : best;
    }
    if ((t & 63) == 0) wk[t >> 6] = best;
    __syncthreads();
    if (t == 0) {
      for (int w = 1; w < NW; w++) best = wk[w] > best ? wk[w] : best;
      __hip_atomic_fetch_max(p.keys + (i & 1), best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      drain();
      __hip_atomic_fetch_add(p.sync + S_COUNT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (PROF_ON) hc += cycles() - hc0;
    }
  }
  if (PROF_ON && t == 0) {
    p.prof[32 + 2 * blockIdx.x] = hw;
    p.prof[33 + 2 * blockIdx.x] = hc;
  }
  if (t == 0) *ok = spin_ge(p.sync + S_DONE, 1u, p.err, 3);
  __syncthreads();
  if (*ok) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Every conv window once, at the end: [P(n-4), P(n-3), P(n-2), P(n-1)] per channel, P(s) the
// channel's projection of step s's GDN norm output (the ring), or the launch's initial window
// for s < 0 (causal_conv1d_update's state after n steps, :210-211).
template <bool BF, bool E4>
__device__ void write_windows(const lxm_params& p) {
  const int64_t total = (int64_t)p.n_layers * p.n_conv;
  const int64_t per = (total + p.n_blocks - 1) / p.n_blocks;
  const int64_t a = (int64_t)blockIdx.x * per, b = a + per < total ? a + per : total;
  const int n = p.n_tokens, H = p.hidden;
  for (int64_t g = a + threadIdx.x; g < b; g += NT) {
    const int L = (int)(g / p.n_conv), c = (int)(g % p.n_conv);
    const lxm_layer ly = p.layers[L];
    const lxm_chan ch = reinterpret_cast<const lxm_chan*>(p.blob + ly.chan)[c];
    void* cs = p.conv[L];
    float w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int s = n - 4 + k;
      if (s >= 0) {
        const float* xo = p.ring + ((size_t)(s & 3) * p.n_layers + L) * H;
        w[k] = rd<BF>(dot_row<E4>(p.blob + ly.qkv_ent, ch.start, ch.len, xo));
      } else {
        w[k] = conv_at<BF>(cs, (int64_t)c * 4 + 4 + s);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) conv_put<BF>(cs, (int64_t)c * 4 + k, w[k]);
  }
}

template <bool BF, bool E4>
__global__ void __launch_bounds__(NT, 1) lxm_decode(const lxm_params* __restrict__ pp) {
  const lxm_params& p = *pp;
  if (blockIdx.x == 0) run_chain<BF, E4>(p);
  else run_helper<BF, E4>(p);
  __syncthreads();
  if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
  write_windows<BF, E4>(p);
}

// ---------------------------------------------------------------------------------------------
// test kernels: the device arithmetic on arrays
__global__ void k_elem(int fn, const float* x, float* y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  float r;
  switch (fn) {
    case 0: r = cr_exp(v); break;
    case 1: r = silu(v); break;
    case 2: r = sigmoid(v); break;
    case 3: r = softplus(v); break;
    case 4: r = rsqrt_(v); break;
    case 5: r = cr_log1p(v); break;
    default: r = bf16r(v); break;
  }
  y[i] = r;
}

__global__ void __launch_bounds__(NT) k_sum(int kind, const float* x, int n, float* out) {
  __shared__ float wsum[32];
  const float* row = x + (size_t)blockIdx.x * n;
  if (kind == 0) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += NT) s = s + row[i];
    s = sum512(s, wsum);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
  } else if (threadIdx.x < 64) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 64) s = s + row[i];
    s = sum64(s);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
  }
}

// ---------------------------------------------------------------------------------------------
extern "C" {

int lxm_lds_base(void) { return L_CHAIN_END; }

int lxm_run(const lxm_params* p_host, const lxm_params* p_dev, int n_blocks, int lds_bytes,
            void* stream) {
  const lxm_params* pd = p_dev;
  void* args[] = {&pd};
  const void* fn = p_host->bf16 ? (const void*)lxm_decode<true, true>
                   : p_host->e4 ? (const void*)lxm_decode<false, true>
                                : (const void*)lxm_decode<false, false>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
  if (e != hipSuccess) return (int)e;
  e = hipLaunchCooperativeKernel(fn, dim3(n_blocks), dim3(NT), args, (unsigned)lds_bytes,
                                 (hipStream_t)stream);
  return (int)e;
}

int lxm_max_blocks(int lds_bytes) {
  int dev = 0, cus = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipFuncSetAttribute((const void*)lxm_decode<true, true>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lxm_decode<true, true>, NT, lds_bytes) !=
      hipSuccess)
    return 0;
  return n * cus;
}

int lxm_max_lds(void) {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess) return 0;
  return v;
}

int lxm_device_cus(void) {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return v;
}

int lxm_last_error(void) { return (int)hipGetLastError(); }

int lxm_t_elem(int fn, const float* x, float* y, long n, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_elem, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     fn, x, y, n);
  return (int)hipGetLastError();
}

int lxm_t_sum(int kind, const float* x, int n, int rows, float* out, void* stream) {
  if (rows <= 0) return 0;
  hipLaunchKernelGGL(k_sum, dim3((unsigned)rows), dim3(NT), 0, (hipStream_t)stream, kind, x, n, out);
  return (int)hipGetLastError();
}

}  // extern "C"
