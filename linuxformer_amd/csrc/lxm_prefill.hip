// The verified-mode forward of the chip layers on MI355X (gfx950): lx.fast's Fast.forward,
// Fast.layer, Fast.head_argmax and Fast.decode (lx/lx/fast.py:252-361, :544-550, :365-540).
//
// T known positions go through each layer together. Everything a position needs from its own
// residual (norms, the MLP, which key heads its query/key projections reach, its decays) is
// token-parallel and runs over tiles of 4 positions held column-major in LDS (one 16-byte read
// gives a column for all four), with each layer's sparse rows read from L2 and reused by every
// tile. Only the delta rule's state carries from one position to the next, and only positions
// whose query, key or decay is live for a head change that state (lx/lx/fast.py:8-19: an idle
// head keeps its state and outputs 0): those candidates are compacted in order, their inputs
// (q, k, v, z, beta, the decay) computed in parallel, and one workgroup per value head then runs
// the recurrence over them with the head's 256x128 state in registers. The gated norm and
// out_proj run per candidate again, in parallel.
//
// Semantics: every position sees exactly the stock decode step (transformers' Qwen3_5 decoder
// layer with causal_conv1d_update and torch_recurrent_gated_delta_rule, in lx/lx/hf.py's chip
// view) with the rounding contract of the decode kernel, so T positions leave the same
// residuals, predictions, conv windows and recurrent states as T forced decode steps, bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lxm_prefill.h"
#include "lxm_math.h"

using namespace lxm;

#define NT 512
#define NW (NT / 64)
#define TT LXM_PF_TT
#define KD 256
#define VD 128
#define MAXH LXM_MAXH
static_assert(TT == 4, "a residual column of a tile is one 16-byte vector");
static_assert(NT >= KD + VD, "the delta kernel loads k/q and v with one thread each");

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ const T* tab(const uint8_t* blob, int64_t off) {
  return reinterpret_cast<const T*>(blob + off);
}
// a table item (whole words) from global memory by global loads (a generic pointer's flat loads
// would also count against the LDS counter, so every wait on a table entry would also wait for
// the LDS reads in flight, and the reverse)
#define GAS __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T gld(const T* q) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  T r;
  const GAS uint32_t* src = (const GAS uint32_t*)q;
  uint32_t* dst = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); i++) dst[i] = src[i];
  return r;
}

// ---------------------------------------------------------------------------------------------
// The residual tiles in HBM, in the model dtype: column c of tile b at (b * H + c) * 4.
// (global loads and stores: generic ones would be flat and also count against the LDS counter)
template <bool BF>
__device__ __forceinline__ v4f ld_col(const void* h, int64_t b, int H, int c) {
  if constexpr (BF) {
    const v2u u = ((const __attribute__((address_space(1))) v2u*)h)[b * H + c];
    return v4f{bitsf(u.x << 16), bitsf(u.x & 0xffff0000u), bitsf(u.y << 16), bitsf(u.y & 0xffff0000u)};
  } else {
    return ((const __attribute__((address_space(1))) v4f*)h)[b * H + c];
  }
}
// (values exact in the model dtype: bf16 keeps the upper half of each float)
template <bool BF>
__device__ __forceinline__ void st_col(void* h, int64_t b, int H, int c, v4f v) {
  if constexpr (BF) {
    v2u u;
    u.x = (fbits(v.x) >> 16) | (fbits(v.y) & 0xffff0000u);
    u.y = (fbits(v.z) >> 16) | (fbits(v.w) & 0xffff0000u);
    ((__attribute__((address_space(1))) v2u*)h)[b * H + c] = u;
  } else {
    ((__attribute__((address_space(1))) v4f*)h)[b * H + c] = v;
  }
}
__device__ __forceinline__ int64_t el_idx(int H, int t, int c) {
  return ((int64_t)(t / TT) * H + c) * TT + t % TT;
}
template <bool BF>
__device__ __forceinline__ float ld_el(const void* h, int H, int t, int c) {
  if constexpr (BF) return bf16f(reinterpret_cast<const uint16_t*>(h)[el_idx(H, t, c)]);
  else return reinterpret_cast<const float*>(h)[el_idx(H, t, c)];
}
template <bool BF>
__device__ __forceinline__ void st_el(void* h, int H, int t, int c, float v) {
  if constexpr (BF) reinterpret_cast<uint16_t*>(h)[el_idx(H, t, c)] = (uint16_t)(fbits(v) >> 16);
  else reinterpret_cast<float*>(h)[el_idx(H, t, c)] = v;
}
// a conv window value (model dtype)
template <bool BF>
__device__ __forceinline__ float conv_ld(const void* cs, int64_t i) {
  if constexpr (BF) return bf16f(reinterpret_cast<const uint16_t*>(cs)[i]);
  else return reinterpret_cast<const float*>(cs)[i];
}
template <bool BF>
__device__ __forceinline__ void conv_st(void* cs, int64_t i, float v) {
  if constexpr (BF) reinterpret_cast<uint16_t*>(cs)[i] = (uint16_t)(fbits(v) >> 16);
  else reinterpret_cast<float*>(cs)[i] = v;
}

// ---------------------------------------------------------------------------------------------
// Arithmetic on the four positions of a column, one IEEE op per position.
template <bool BF>
__device__ __forceinline__ v4f acc4(v4f s, v4f x, float w) {
  return v4f{acc<BF>(s.x, x.x, w), acc<BF>(s.y, x.y, w), acc<BF>(s.z, x.z, w), acc<BF>(s.w, x.w, w)};
}
// (bf16: the four roundings as two paired conversions)
template <bool BF>
__device__ __forceinline__ v4f rd4(v4f v) {
  if constexpr (BF) {
    const f32x2 a = bf16r2(f32x2{v.x, v.y}), b = bf16r2(f32x2{v.z, v.w});
    return v4f{a.x, a.y, b.x, b.y};
  }
  return v;
}
// D((h * r) * w1) per position: the RMSNorm's output (TF:720-737)
template <bool BF>
__device__ __forceinline__ v4f norm4(v4f h, v4f r, float w1) {
  return rd4<BF>(v4f{(h.x * r.x) * w1, (h.y * r.y) * w1, (h.z * r.z) * w1, (h.w * r.w) * w1});
}
__device__ __forceinline__ float norm_r(float ss, int H, float eps) {
  return rsqrt_(ss / (float)H + eps);
}
// The four positions' factors from their sums of squares (equal in every lane): lane k
// evaluates position k & 3's, and every lane reads positions 0-3 back from lanes 0-3, so a wave
// evaluates the IEEE divide and square root sequence once instead of four times. Every lane of
// the wave must be active.
__device__ __forceinline__ v4f norm_r4(v4f ss, int H, float eps) {
  const int k = threadIdx.x & 3;
  const float s = k == 0 ? ss.x : k == 1 ? ss.y : k == 2 ? ss.z : ss.w;
  const int u = __float_as_int(norm_r(s, H, eps));
  return v4f{__int_as_float(__builtin_amdgcn_readlane(u, 0)),
             __int_as_float(__builtin_amdgcn_readlane(u, 1)),
             __int_as_float(__builtin_amdgcn_readlane(u, 2)),
             __int_as_float(__builtin_amdgcn_readlane(u, 3))};
}

// A sparse row's dot product with a column-major tile vector x in LDS (entry offsets 16 x
// column), for the four positions at once: the terms in entry order from +0, each rounded once
// (the oracle's CSR rows: ascending columns; its zero-x skips change no bits, a sum from +0 is
// never -0). Entries load four at a time (every table is followed by four padding entries);
// the terms past the row's end are not added.
// LDS tile vectors: a column of the 4 positions per slot, fp32 (16 bytes), or bf16 (8 bytes;
// HALF) where every value kept there is exact in bf16. at(): by a table offset (16 x column).
template <bool HALF>
struct TV {
  static constexpr int B = HALF ? 8 : 16;
  static __device__ __forceinline__ v4f at(const uint8_t* v, int off) {
    if constexpr (HALF) {
      const v2u u = *reinterpret_cast<const v2u*>(v + (off >> 1));
      return v4f{bitsf(u.x << 16), bitsf(u.x & 0xffff0000u), bitsf(u.y << 16), bitsf(u.y & 0xffff0000u)};
    } else {
      return *reinterpret_cast<const v4f*>(v + off);
    }
  }
  // the same for a tile vector at LDS byte address base (the kernel's dynamic LDS at address 0):
  // the address formed from the entry's offset alone (a constant base folds into the read)
  static __device__ __forceinline__ v4f at_lds(uint32_t base, int off) {
    if constexpr (HALF) {
      const v2u u = *(const __attribute__((address_space(3))) v2u*)(size_t)(base + ((uint32_t)off >> 1));
      return v4f{bitsf(u.x << 16), bitsf(u.x & 0xffff0000u), bitsf(u.y << 16), bitsf(u.y & 0xffff0000u)};
    } else {
      return *(const __attribute__((address_space(3))) v4f*)(size_t)(base + (uint32_t)off);
    }
  }
  static __device__ __forceinline__ v4f get(const uint8_t* v, int c) { return at(v, 16 * c); }
  static __device__ __forceinline__ void put(uint8_t* v, int c, v4f x) {
    if constexpr (HALF) {
      v2u u;
      u.x = (fbits(x.x) >> 16) | (fbits(x.y) & 0xffff0000u);
      u.y = (fbits(x.z) >> 16) | (fbits(x.w) & 0xffff0000u);
      *reinterpret_cast<v2u*>(v + B * c) = u;
    } else {
      *reinterpret_cast<v4f*>(v + B * c) = x;
    }
  }
};

// the tile kernel's residual tile: LDS byte address (after 512 bytes of sums and masks)
#define X_HV 512
// (PAD: the row is padded to a multiple of 4 entries at a column holding +0, weight 0, so every
// entry of its last group adds its term with no test)
template <bool BF, bool HALF = false, bool PAD = false>
__device__ __forceinline__ v4f dot4(const lxm_pf_ent* __restrict__ e, int n, const uint8_t* x) {
  v4f s = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < n; k0 += 4) {
    lxm_pf_ent en[4];
#pragma unroll
    for (int j = 0; j < 4; j++) en[j] = gld(e + k0 + j);
    v4f xv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xv[j] = TV<HALF>::at(x, en[j].off);
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (PAD || k0 + j < n) s = acc4<BF>(s, xv[j], en[j].w);
  }
  return s;
}
// The same over the RMSNorm of a tile: each gathered column x becomes D((x * r) * w1) (norm4),
// w1 the column's norm weight from the table parallel to the entries.
// (PAD: padded rows as for dot4, and x the tile kernel's residual tile at LDS address X_HV)
template <bool BF, bool HALF, bool PAD = false>
__device__ __forceinline__ v4f dot4n(const lxm_pf_ent* __restrict__ e, const float* __restrict__ en,
                                     int n, const uint8_t* x, v4f r) {
  v4f s = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < n; k0 += 4) {
    lxm_pf_ent ee[4];
    float nw[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      ee[j] = gld(e + k0 + j);
      nw[j] = gld(en + k0 + j);
    }
    v4f xv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xv[j] = PAD ? TV<HALF>::at_lds(X_HV, ee[j].off) : TV<HALF>::at(x, ee[j].off);
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (PAD || k0 + j < n) s = acc4<BF>(s, norm4<BF>(xv[j], r, nw[j]), ee[j].w);
  }
  return s;
}
// The head's rows over a tile at LDS address 0: an entry's column offset is its LDS address (no
// base added per entry).
typedef const __attribute__((address_space(3))) v4f* lds_v4f;
template <bool BF>
__device__ __forceinline__ v4f sum4z(v4f s, const lxm_pf_ent (&en)[4]) {
  v4f xv[4];
#pragma unroll
  for (int j = 0; j < 4; j++) xv[j] = *(lds_v4f)(size_t)(uint32_t)en[j].off;
#pragma unroll
  for (int j = 0; j < 4; j++) s = acc4<BF>(s, xv[j], en[j].w);
  return s;
}
// a head row: its first four entries (at 4 r: no row pointer to wait for), and where the rest
// of a longer row sits (start, count: a multiple of 4; 0 for a row of at most four)
struct HRow {
  uint32_t e0;
  int n;
  lxm_pf_ent g[4];
};
// (LONG false: no row of the table has more than four entries, and head_more is not read)
template <bool LONG>
__device__ __forceinline__ void hrow_req(const int32_t* hmore, const lxm_pf_ent* hent, int r,
                                         HRow& h) {
  typedef int32_t v2i __attribute__((ext_vector_type(2)));
  h.e0 = 0;
  h.n = 0;
  if constexpr (LONG) {
    const v2i m = gld(reinterpret_cast<const v2i*>(hmore) + r);
    h.e0 = (uint32_t)m.x;
    h.n = m.y;
  }
#pragma unroll
  for (int j = 0; j < 4; j++) h.g[j] = gld(hent + 4 * (uint32_t)r + j);
}
// the row's sums for the tile's four positions, entries in ascending order from +0
template <bool BF>
__device__ __forceinline__ v4f hrow_sum(const lxm_pf_ent* hent, const HRow& h) {
  v4f s = sum4z<BF>(v4f{0.0f, 0.0f, 0.0f, 0.0f}, h.g);
  for (int k0 = 0; k0 < h.n; k0 += 4) {
    lxm_pf_ent en[4];
#pragma unroll
    for (int j = 0; j < 4; j++) en[j] = gld(hent + h.e0 + k0 + j);
    s = sum4z<BF>(s, en);
  }
  return s;
}
// the same for one float per entry at x + off (a flat vector, or one position's lane of a tile)
template <bool BF>
__device__ __forceinline__ float dot1(const lxm_pf_ent* __restrict__ e, int n, const uint8_t* x) {
  float s = 0.0f;
  for (int k0 = 0; k0 < n; k0 += 4) {
    lxm_pf_ent en[4];
#pragma unroll
    for (int j = 0; j < 4; j++) en[j] = gld(e + k0 + j);
    float xv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xv[j] = *reinterpret_cast<const float*>(x + en[j].off);
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (k0 + j < n) s = acc<BF>(s, xv[j], en[j].w);
  }
  return s;
}

// The 512-lane hidden sum of x * x for the four positions of a tile (the decode's order: thread
// t adds its columns 4t..4t+3, then 2048+4t..2048+4t+3; waves at offsets 32..1; the 8 wave
// totals at offsets 4, 2, 1; columns >= H are +0 and add nothing). With plus0, each column also
// becomes x + 0 (the residual add of a row with no term: -0 becomes +0). Every thread gets the
// sums. wsum: 8 vectors of LDS, not reused before the next barrier.
template <bool BF, bool HALF>
__device__ __forceinline__ v4f hsum(uint8_t* HV, int H, v4f* wsum, bool plus0) {
  const int t = threadIdx.x;
  v4f s = {0.0f, 0.0f, 0.0f, 0.0f};
  // (every column read before any is summed: a column past H reads the tile's zero column H,
  // whose +0 squares leave the sum, which starts at +0 and adds squares, unchanged)
  v4f xs[8];
#pragma unroll
  for (int half = 0; half < 2; half++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = half * 2048 + 4 * t + i;
      xs[4 * half + i] = TV<HALF>::get(HV, c < H ? c : H);
    }
#pragma unroll
  for (int half = 0; half < 2; half++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = half * 2048 + 4 * t + i;
      v4f x = xs[4 * half + i];
      if (plus0) {
        x = v4f{x.x + 0.0f, x.y + 0.0f, x.z + 0.0f, x.w + 0.0f};
        if (c < H) TV<HALF>::put(HV, c, x);
      }
      s = v4f{acc<BF>(s.x, x.x, x.x), acc<BF>(s.y, x.y, x.y), acc<BF>(s.z, x.z, x.z),
              acc<BF>(s.w, x.w, x.w)};
    }
  s = v4f{wave_tree(s.x), wave_tree(s.y), wave_tree(s.z), wave_tree(s.w)};
  if ((t & 63) == 0) wsum[t >> 6] = s;
  __syncthreads();
  v4f w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}

// ---------------------------------------------------------------------------------------------
// The tile kernel: one workgroup per tile of 4 positions. Lm >= 0: layer Lm's MLP
// (post_attention_layernorm, SwiGLU, down_proj, residual add; TF:704-717, :781-793) on the
// residual as the previous steps left it, stored back. Then Ln >= 0: layer Ln's input norm
// factor r1 per position, and which of the layer's key slots have a nonzero query/key projection
// at each position, and whether a decay can act (bit 31); or Ln == -2: the final norm into hn.
// The norms' outputs are formed as the entries gather (each entry carries its column's norm
// weight), so LDS holds 512 bytes of sums and masks, the residual (hidden columns) and the MLP
// units' outputs, as tile vectors in the model dtype (bf16, hidden 3,572, 1,024 units: 37 KB),
// each followed by a column of zeros that the rows' padding entries read (rows padded to
// multiples of 4 entries, summed with no per-entry test). At most 64 VGPRs (eight waves per
// SIMD): four workgroups per CU, as many as that LDS allows (69 VGPRs held three); each unit's
// output goes to LDS as soon as it is formed, so no unit's result is held in registers.
// A residual tile from HBM (model dtype) into LDS tile vectors (bf16 if HALF): every thread's
// columns (t, t + 512, ...) loaded at once.
template <bool BF, bool HALF>
__device__ __forceinline__ void load_tile(const void* h, int64_t b, int H, uint8_t* HV) {
  const int t = threadIdx.x;
  // (every load is issued, a column past H reading column H - 1 of the same tile, before any
  // value is looked at: a load under the column's test was waited on inside its branch)
  v4f x[MAXH / NT];
#pragma unroll
  for (int k = 0; k < MAXH / NT; k++) {
    const int c = t + k * NT;
    x[k] = ld_col<BF>(h, b, H, c < H ? c : H - 1);
  }
#pragma unroll
  for (int k = 0; k < MAXH / NT; k++)
    if (t + k * NT < H) TV<HALF>::put(HV, t + k * NT, x[k]);
}
template <bool BF>
__host__ __device__ constexpr int x_xm(int H) { return X_HV + ((TV<BF>::B * (H + 1) + 15) & ~15); }
template <bool BF>
__global__ __launch_bounds__(NT, 8) void pf_tile(const lxm_pf_params* __restrict__ pp, int Lm, int Ln) {
  extern __shared__ __align__(16) uint8_t sm[];
  using V = TV<BF>;
  const lxm_pf_params& p = *pp;
  const int t = threadIdx.x, H = p.hidden;
  const int64_t b = blockIdx.x;
  uint32_t* smask = reinterpret_cast<uint32_t*>(sm);
  v4f* wsA = reinterpret_cast<v4f*>(sm + 64);
  v4f* wsB = reinterpret_cast<v4f*>(sm + 192);
  uint8_t* HV = sm + X_HV;
  uint8_t* XM = sm + x_xm<BF>(H);
  // the residual tile is read at LDS address X_HV + offset (dot4n): the LDS must start at 0
  if ((uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)sm != 0u) {
    if (t == 0) *p.err = 2;
    return;
  }
  if (t < TT) smask[t] = 0;
  if (t == 0) V::put(HV, H, v4f{0.0f, 0.0f, 0.0f, 0.0f});  // the padding entries' zero column
  load_tile<BF, BF>(p.h, b, H, HV);
  __syncthreads();
  if (Lm >= 0) {
    const lxm_pf_layer& ly = p.layers[Lm];
    const lxm_pf_ent* ent = tab<lxm_pf_ent>(p.blob, ly.ent);
    const float* entn = tab<float>(p.blob, ly.entn);
    const v4f ss = hsum<BF, BF>(HV, H, wsA, false);
    const v4f r = norm_r4(ss, H, ly.eps);
    // units over the post norm (formed as the entries gather): act = D(D(silu(D(gate . x))) *
    // D(up . x))
    const lxm_pf_unit* un = tab<lxm_pf_unit>(p.blob, ly.units);
    for (int u = t; u < ly.n_units; u += NT) {
      const lxm_pf_unit q = gld(un + u);
      const v4f g = rd4<BF>(dot4n<BF, BF, true>(ent + q.gs, entn + q.gs, q.gn, HV, r));
      const v4f v = rd4<BF>(dot4n<BF, BF, true>(ent + q.us, entn + q.us, q.un, HV, r));
      V::put(XM, u, v4f{rd<BF>(silu_rd<BF>(g.x) * v.x), rd<BF>(silu_rd<BF>(g.y) * v.y),
                        rd<BF>(silu_rd<BF>(g.z) * v.z), rd<BF>(silu_rd<BF>(g.w) * v.w)});
    }
    if (t == 0) V::put(XM, ly.n_units, v4f{0.0f, 0.0f, 0.0f, 0.0f});  // the down rows' zero column
    __syncthreads();
    // down_proj rows over the units (entries 16 x unit position), added to the residual
    const lxm_pf_drow* dr = tab<lxm_pf_drow>(p.blob, ly.drows);
    // (a row of one entry: its padding entries read the zero column with weight 0 and add +0 to
    // a sum that is never -0, so the sum is its one term; the rows come longest first, so a
    // wave's rows take one path or the other except at one boundary)
    for (int i = t; i < ly.n_drows; i += NT) {
      const lxm_pf_drow d = gld(dr + i);
      v4f s;
      if (d.len == 1) {
        const lxm_pf_ent e = gld(ent + d.start);
        s = rd4<BF>(acc4<BF>(v4f{0.0f, 0.0f, 0.0f, 0.0f}, V::at(XM, e.off), e.w));
      } else {
        s = rd4<BF>(dot4<BF, BF, true>(ent + d.start, d.len, XM));
      }
      V::put(HV, d.row, rd4<BF>(V::get(HV, d.row) + s));
    }
    __syncthreads();
  }
  if (Ln >= 0) {
    const lxm_pf_layer& ly = p.layers[Ln];
    const lxm_pf_ent* ent = tab<lxm_pf_ent>(p.blob, ly.ent);
    const float* entn = tab<float>(p.blob, ly.entn);
    const v4f ss = hsum<BF, BF>(HV, H, wsB, Lm >= 0);
    const v4f r = norm_r4(ss, H, ly.eps);
    if (t < TT && b * TT + t < p.T) p.r1[b * TT + t] = t == 0 ? r.x : t == 1 ? r.y : t == 2 ? r.z : r.w;
    // query/key projections of the live key heads' channels over the input norm (formed as the
    // entries gather): which slots are nonzero
    const lxm_pf_qk* qk = tab<lxm_pf_qk>(p.blob, ly.qk);
    for (int i = t; i < ly.n_qk; i += NT) {
      const lxm_pf_qk q = gld(qk + i);
      const v4f P = rd4<BF>(dot4n<BF, BF, true>(ent + q.start, entn + q.start, q.len, HV, r));
      const uint32_t bit = 1u << q.kslot;
      if (P.x != 0.0f) atomicOr(smask + 0, bit);
      if (P.y != 0.0f) atomicOr(smask + 1, bit);
      if (P.z != 0.0f) atomicOr(smask + 2, bit);
      if (P.w != 0.0f) atomicOr(smask + 3, bit);
    }
    // decays: g = -exp(A_log) * softplus(a + dt_bias) (:499); a step decays when exp(g) != 1
    const lxm_pf_dec* dc = tab<lxm_pf_dec>(p.blob, ly.dec);
    for (int i = t; i < ly.n_dec; i += NT) {
      const lxm_pf_dec d = gld(dc + i);
      const v4f a = d.len ? rd4<BF>(dot4n<BF, BF, true>(ent + d.start, entn + d.start, d.len, HV, r))
                          : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      const float na = -cr_exp(d.A_log);
#pragma unroll
      for (int k = 0; k < TT; k++) {
        // (x < -104: exp(x) rounds to 0, so softplus(x) is 0 and, na being finite, exp(na * 0)
        // is 1 without evaluating it)
        const float x = a[k] + d.dt_bias;
        if (x < -104.0f && na > -__builtin_inff()) continue;
        if (cr_exp(na * softplus(x)) != 1.0f) atomicOr(smask + k, 0x80000000u);
      }
    }
    __syncthreads();
    if (t < TT && b * TT + t < p.T) p.mask[b * TT + t] = smask[t];
  } else if (Ln == -2) {
    const v4f ss = hsum<BF, BF>(HV, H, wsB, Lm >= 0);
    const v4f r = norm_r4(ss, H, p.rms_eps);
    float w[MAXH / NT];
#pragma unroll
    for (int k = 0; k < MAXH / NT; k++) w[k] = t + k * NT < H ? p.w1_final[t + k * NT] : 0.0f;
#pragma unroll
    for (int k = 0; k < MAXH / NT; k++)
      if (t + k * NT < H) st_col<BF>(p.hn, b, H, t + k * NT, norm4<BF>(V::get(HV, t + k * NT), r, w[k]));
  } else if (Lm >= 0) {
    for (int c = t; c < H; c += NT) V::put(HV, c, V::get(HV, c) + v4f{0.0f, 0.0f, 0.0f, 0.0f});
  }
  if (Lm >= 0)
    for (int c = t; c < H; c += NT) st_col<BF>(p.h, b, H, c, V::get(HV, c));
}

// ---------------------------------------------------------------------------------------------
// The candidates of layer L, in position order: positions whose query/key channels of some live
// key head can be nonzero (a nonzero projection within the earliest tap's reach, or a window
// from before the call), or that decay. One workgroup of 1,024 threads; each thread takes 32
// consecutive positions per round.
#define C_NT 1024
#define C_PER 32
__global__ __launch_bounds__(C_NT) void pf_compact(const lxm_pf_params* __restrict__ pp, int L) {
  __shared__ int wtot[C_NT / 64];
  __shared__ int base_s;
  const lxm_pf_params& p = *pp;
  const lxm_pf_layer& ly = p.layers[L];
  const int t = threadIdx.x, T = p.T, reach = ly.reach;
  const uint32_t allk = ly.n_ks >= 32 ? 0xffffffffu : ((1u << ly.n_ks) - 1u);
  const bool vec = (reinterpret_cast<uintptr_t>(p.mask) & 15u) == 0;
  if (t == 0) base_s = 0;
  __syncthreads();
  for (int r0 = 0; r0 < T; r0 += C_NT * C_PER) {
    const int t0 = r0 + t * C_PER;
    uint32_t m[C_PER + 3];
    // m[3 + i]: the mask of position t0 + i, by eight 16-byte loads where the thread's 32 lie
    // inside T and the array is 16-byte aligned (a lane's run is one 128-byte line); m[0..2]: the
    // three before t0, from the lane below (its last three), lane 0 reading its own
    if (vec && t0 + C_PER <= T) {
      const uint4* src = reinterpret_cast<const uint4*>(p.mask + t0);
#pragma unroll
      for (int j = 0; j < C_PER / 4; j++) {
        const uint4 v = gld(src + j);
        m[3 + 4 * j] = v.x;
        m[4 + 4 * j] = v.y;
        m[5 + 4 * j] = v.z;
        m[6 + 4 * j] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < C_PER; i++) m[3 + i] = t0 + i < T ? p.mask[t0 + i] : 0u;
    }
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const uint32_t below = __shfl_up(m[C_PER + i], 1);
      const int tp = t0 - 3 + i;
      m[i] = (t & 63) ? below : (tp >= 0 && tp < T) ? p.mask[tp] : 0u;
    }
    int n = 0;
    uint32_t cm[C_PER];
#pragma unroll
    for (int i = 0; i < C_PER; i++) {
      const int tp = t0 + i;
      uint32_t kb = m[i + 3] & 0xffffu;
      if (reach >= 1) kb |= m[i + 2] & 0xffffu;
      if (reach >= 2) kb |= m[i + 1] & 0xffffu;
      if (reach >= 3) kb |= m[i] & 0xffffu;
      if (tp < reach) kb |= allk;
      kb |= m[i + 3] & 0x80000000u;
      cm[i] = tp < T ? kb : 0u;
      n += cm[i] != 0u;
    }
    // exclusive scan of n over the workgroup
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if ((t & 63) >= off) incl += y;
    }
    if ((t & 63) == 63) wtot[t >> 6] = incl;
    __syncthreads();
    int wbase = 0, all = 0;
    for (int w = 0; w < C_NT / 64; w++) {
      if (w < (t >> 6)) wbase += wtot[w];
      all += wtot[w];
    }
    int o = base_s + wbase + incl - n;
#pragma unroll
    for (int i = 0; i < C_PER; i++)
      if (cm[i] != 0u) {
        p.cand[o] = t0 + i;
        p.cmask[o] = cm[i];
        o++;
      }
    __syncthreads();
    if (t == 0) base_s += all;
    __syncthreads();
  }
  if (t == 0) p.count[L] = base_s;
}

// ---------------------------------------------------------------------------------------------
// Candidate records. Offsets inside one (see lxm_pf_layer): header {tok, live slots}, qn, kn, v,
// z, beta, e, proc.
struct RecOff {
  int q, k, v, z, b, e, pr;
  __device__ RecOff(int nks, int nvs) {
    q = 16;
    k = q + 1024 * nks;
    v = k + 1024 * nks;
    z = v + 512 * nvs;
    b = z + 512 * nvs;
    e = b + 4 * nvs;
    pr = e + 4 * nvs;
  }
};

// The conv output of a channel at position tok: the window [x(tok-3) .. x(tok)] from the
// projections P (lane s: position tok - s) or, before the call's first position, the window the
// cache held (TF:199-216: silu(D(sum of taps * window)), rounded to the model dtype).
template <bool BF>
__device__ __forceinline__ float conv_y(const v4f P, const float* taps, int tok, const void* cs,
                                        int64_t chan) {
  float y = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if (taps[k] == 0.0f) continue;
    const int s = 3 - k;
    const float x = tok - s >= 0 ? P[s] : conv_ld<BF>(cs, chan * 4 + 4 + (tok - s));
    y = acc<BF>(y, taps[k], x);
  }
  return silu_rd<BF>(rd<BF>(y));
}

// One workgroup per candidate (grid-stride): the input norm's output at positions tok..tok-3
// (lanes 0..3 of a tile-shaped vector in LDS), the query/key conv outputs of its key slots,
// which slots are live, their l2norms; for the live slots' value heads the value channels' conv
// outputs, the in_proj_z rows and beta; every slot's decay factor exp(g). LDS: the normed input
// (64 KB), q/k per key slot (32 KB), the live word.
#define A_QK (16 * MAXH)
#define A_MISC (A_QK + 4 * LXM_PF_MAXKS * 2 * KD)
template <bool BF>
__global__ __launch_bounds__(NT) void pf_act(const lxm_pf_params* __restrict__ pp, int L) {
  extern __shared__ __align__(16) uint8_t sm[];
  const lxm_pf_params& p = *pp;
  const lxm_pf_layer& ly = p.layers[L];
  const int t = threadIdx.x, H = p.hidden, lane = t & 63, wv = t >> 6;
  v4f* XN = reinterpret_cast<v4f*>(sm);
  float* QK = reinterpret_cast<float*>(sm + A_QK);
  uint32_t* live_s = reinterpret_cast<uint32_t*>(sm + A_MISC);
  const lxm_pf_ent* ent = tab<lxm_pf_ent>(p.blob, ly.ent);
  const float* w1 = tab<float>(p.blob, ly.w1_in);
  const void* cs = p.conv[L];
  const RecOff ro(ly.n_ks, ly.n_vs);
  const int count = p.count[L];
  for (int j = blockIdx.x; j < count; j += gridDim.x) {
    const int tok = p.cand[j];
    const uint32_t cm = p.cmask[j];
    uint8_t* rec = p.recs + (int64_t)j * ly.rec_bytes;
    float rr[4];
#pragma unroll
    for (int s = 0; s < 4; s++) rr[s] = tok - s >= 0 ? p.r1[tok - s] : 0.0f;
    // positions tok - s, s = 0..3: lane l0 - s of tile tok / 4 for s <= l0, else lane l0 - s + 4 of
    // the tile before (tok / 4 and l0 the same for the whole workgroup), read as columns
    const int64_t b0 = tok >> 2;
    const int l0 = tok & 3;
    for (int c = t; c < H; c += NT) {
      const v4f c0 = ld_col<BF>(p.h, b0, H, c);
      const v4f c1 = l0 < 3 && b0 > 0 ? ld_col<BF>(p.h, b0 - 1, H, c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      const float w = w1[c];
      v4f x;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const float h = s <= l0 ? c0[l0 - s] : c1[l0 - s + 4];
        x[s] = tok - s >= 0 ? rd<BF>((h * rr[s]) * w) : 0.0f;
      }
      XN[c] = x;
    }
    for (int i = t; i < ly.n_ks * 2 * KD; i += NT) QK[i] = 0.0f;
    if (t == 0) *live_s = 0u;
    __syncthreads();
    // the query/key conv outputs of the slots to evaluate
    const lxm_pf_qk* qk = tab<lxm_pf_qk>(p.blob, ly.qk);
    for (int i = t; i < ly.n_qk; i += NT) {
      const lxm_pf_qk q = gld(qk + i);
      if (!((cm >> q.kslot) & 1u)) continue;
      const v4f P = rd4<BF>(dot4<BF>(ent + q.start, q.len, sm));
      QK[q.kslot * 2 * KD + q.pos] = conv_y<BF>(P, q.taps, tok, cs, q.chan);
    }
    __syncthreads();
    // live slots (a nonzero query or key) and the l2norms (TF:242-245, :352-353): one wave per
    // (slot, query | key); D(x * D(rsqrt(D(D(sum64 D(x*x)) + 1e-6)))), the query times 1/16
    for (int task = wv; task < 2 * ly.n_ks; task += NW) {
      const int slot = task >> 1, isk = task & 1;
      if (!((cm >> slot) & 1u)) continue;
      const float* x = QK + slot * 2 * KD + isk * KD;
      float xs[4], s = 0.0f;
      bool nz = false;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        xs[i] = x[lane + 64 * i];
        nz |= xs[i] != 0.0f;
        s = s + rd<BF>(xs[i] * xs[i]);
      }
      if (__ballot(nz) != 0ull && lane == 0) atomicOr(live_s, 1u << slot);
      s = rd<BF>(sum64(s));
      const float inv = rd<BF>(rsqrt_(rd<BF>(s + 1e-6f)));
      float* o = reinterpret_cast<float*>(rec + (isk ? ro.k : ro.q)) + slot * KD;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float v = rd<BF>(xs[i] * inv);
        if (!isk) v = v * 0.0625f;
        o[lane + 64 * i] = v;
      }
    }
    __syncthreads();
    const uint32_t live = *live_s;
    const lxm_pf_vs* vs = tab<lxm_pf_vs>(p.blob, ly.vs);
    const lxm_pf_vc* vc = tab<lxm_pf_vc>(p.blob, ly.vc);
    const lxm_row* zr = tab<lxm_row>(p.blob, ly.zrow);
    float* rv = reinterpret_cast<float*>(rec + ro.v);
    float* rz = reinterpret_cast<float*>(rec + ro.z);
    for (int i = t; i < ly.n_vs * VD; i += NT) {
      const lxm_pf_vs sv = vs[i >> 7];
      if (sv.kslot < 0 || !((live >> sv.kslot) & 1u)) continue;
      const lxm_pf_vc c = vc[i];
      const v4f P = rd4<BF>(dot4<BF>(ent + c.start, c.len, sm));
      const int64_t chan = 2 * (int64_t)p.nk * KD + (int64_t)sv.vh * VD + (i & 127);
      rv[i] = conv_y<BF>(P, c.taps, tok, cs, chan);
      const lxm_row z = zr[i];
      rz[i] = rd<BF>(dot1<BF>(ent + z.start, z.len, sm));
    }
    const lxm_row* br = tab<lxm_row>(p.blob, ly.brow);
    const lxm_pf_dec* dc = tab<lxm_pf_dec>(p.blob, ly.dec);
    for (int i = t; i < ly.n_vs; i += NT) {
      const lxm_pf_vs sv = vs[i];
      float e = 1.0f;
      if (sv.dslot >= 0) {
        const lxm_pf_dec d = dc[sv.dslot];
        const float a = d.len ? rd<BF>(dot1<BF>(ent + d.start, d.len, sm)) : 0.0f;
        const float na = -cr_exp(d.A_log), x = a + d.dt_bias;
        // (x < -104: softplus(x) is 0, and exp(na * 0) is 1 for a finite na)
        if (!(x < -104.0f && na > -__builtin_inff())) e = cr_exp(na * softplus(x));
      }
      reinterpret_cast<float*>(rec + ro.e)[i] = e;
      if (sv.kslot >= 0 && ((live >> sv.kslot) & 1u)) {
        const lxm_row bb = br[i];
        reinterpret_cast<float*>(rec + ro.b)[i] = rd<BF>(sigmoid(rd<BF>(dot1<BF>(ent + bb.start, bb.len, sm))));
      }
    }
    if (t == 0) {
      reinterpret_cast<int32_t*>(rec)[0] = tok;
      reinterpret_cast<uint32_t*>(rec)[1] = live;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// The conv windows the call leaves (causal_conv1d_update's state after the last position: each
// channel's last 4 projections, TF:199-216), for every channel of layer L. Runs while p->h holds
// the layer's input and after pf_act has read the windows the call started from.
template <bool BF>
__global__ __launch_bounds__(256) void pf_tail(const lxm_pf_params* __restrict__ pp, int L) {
  const lxm_pf_params& p = *pp;
  const lxm_pf_layer& ly = p.layers[L];
  const int c = blockIdx.x * 256 + threadIdx.x, H = p.hidden, T = p.T;
  if (c >= p.n_conv) return;
  const lxm_pf_ent* ent = tab<lxm_pf_ent>(p.blob, ly.ent);
  const float* w1 = tab<float>(p.blob, ly.w1_in);
  const lxm_row row = tab<lxm_row>(p.blob, ly.cc)[c];
  void* cs = p.conv[L];
  // one pass over the channel's entries forms the four window sums (each in entry order); the
  // positions T-4..T-1 are lanes of the last tile and the one before it, read as columns
  const int64_t b0 = (T - 1) >> 2;
  const int l0 = (T - 1) & 3;
  float r[4], s[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    r[j] = T - 4 + j >= 0 ? p.r1[T - 4 + j] : 0.0f;
    s[j] = 0.0f;
  }
  for (int k = 0; k < row.len; k++) {
    const lxm_pf_ent e = ent[row.start + k];
    const int col = e.off >> 4;
    const float w = w1[col];
    const v4f c0 = ld_col<BF>(p.h, b0, H, col);
    const v4f c1 = l0 < 3 && b0 > 0 ? ld_col<BF>(p.h, b0 - 1, H, col) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = 3 - j;  // position T-1-d
      const float h = d <= l0 ? c0[l0 - d] : c1[l0 - d + 4];
      if (T - 4 + j >= 0) s[j] = acc<BF>(s[j], rd<BF>((h * r[j]) * w), e.w);
    }
  }
  float win[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    win[j] = T - 4 + j >= 0 ? rd<BF>(s[j]) : conv_ld<BF>(cs, (int64_t)c * 4 + j + T);
#pragma unroll
  for (int j = 0; j < 4; j++) conv_st<BF>(cs, (int64_t)c * 4 + j, win[j]);
}

// ---------------------------------------------------------------------------------------------
// The recurrence of one value-head slot over the layer's candidates, in position order
// (torch_recurrent_gated_delta_rule, TF:330-380, one token at a time): S <- S * exp(g) when
// exp(g) != 1; with a live query or key kv = S^T k, delta = (v - kv) beta, S += k delta^T,
// o = D(S^T q) into the record (over v, which this step has read). One wave per DCW = 4 of the
// slot's 128 state columns (DWS = 32 one-wave workgroups a slot): lane 16 c + b holds column
// c0 + c of rows 16b..16b+15 in registers, one of ATen's 16-row cascade blocks (torch .sum(-2)
// on the CPU: each block from +0 in row order, the block sums from +0 in block order). Both of a
// step's sums over the 16 blocks stay in the wave: each lane's block sum goes to the wave's row
// of LDS and every lane of the column reads the column's 16 back and adds them in block order
// (a wave's LDS accesses run in order, so no barrier). No sum crosses columns, so each column's
// sums are those of the whole tile.
#define DCW 4
#define DWS (VD / DCW)
#define KQ_Q (20 * KD / 16)  // the q half of a wave's k and q staging
// A candidate's inputs as one lane holds them (loaded three candidates ahead): the header word,
// the slot's decay factor, its column's v, beta, and an eighth of the slot's k and q (lanes
// 0-31 k, 32-63 q, 8 values each), which the step stages in the wave's LDS for every lane.
struct DeltaIn {
  uint32_t live;
  float e, v, beta;
  v4f kq[2];
};
__device__ __forceinline__ DeltaIn delta_in(const uint8_t* rec, const RecOff& ro, int vslot,
                                            int kslot, int col, int b) {
  // (global loads: a generic pointer's flat loads would also count against the LDS counter, and
  // every LDS wait of a step would then wait for the candidates in flight)
  const GAS uint8_t* g = (const GAS uint8_t*)rec;
  DeltaIn d;
  d.live = ((const GAS uint32_t*)g)[1];
  d.e = ((const GAS float*)(g + ro.e))[vslot];
  d.v = d.beta = 0.0f;
  d.kq[0] = d.kq[1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  if (kslot >= 0) {
    // (the record's k and q rows start at 16-byte multiples: 16 + 1024 x slot)
    const int lane = threadIdx.x;
    const GAS v4f* kq = (const GAS v4f*)(g + (lane < 32 ? ro.k : ro.q) + 4 * KD * kslot) +
                        2 * (lane & 31);
    d.kq[0] = kq[0];
    d.kq[1] = kq[1];
    d.v = ((const GAS float*)(g + ro.v))[vslot * VD + col];
    d.beta = ((const GAS float*)(g + ro.b))[vslot];
  }
  return d;
}
// the 16 block sums of this lane's column, from +0 in block order (every lane of the column
// gets the same sum)
__device__ __forceinline__ float col_sum16(float* red, int c, int b, float x) {
  red[16 * c + b] = x;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const v4f* r = reinterpret_cast<const v4f*>(red + 16 * c);
  const v4f w0 = r[0], w1 = r[1], w2 = r[2], w3 = r[3];
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  float q = 0.0f;
  q = q + w0.x; q = q + w0.y; q = q + w0.z; q = q + w0.w;
  q = q + w1.x; q = q + w1.y; q = q + w1.z; q = q + w1.w;
  q = q + w2.x; q = q + w2.y; q = q + w2.z; q = q + w2.w;
  q = q + w3.x; q = q + w3.y; q = q + w3.z; q = q + w3.w;
  return q;
}

// One candidate's step for one lane (see pf_delta). (Skipping the row offsets where no lane of
// the wave has a nonzero factor, by a wave-uniform branch per row, measured slower: the branches
// cost more than the rows they save.)
template <bool BF>
__device__ __forceinline__ void delta_step(const DeltaIn& cur, float (&s)[16], float* red,
                                           float* kqs, int c, int b, int kslot, uint8_t* rec,
                                           const RecOff& ro, int vslot, int col, bool first,
                                           bool& wrote) {
  const bool live = kslot >= 0 && ((cur.live >> kslot) & 1u);
  const float e = cur.e;
  int proc = 0;
  if (live || e != 1.0f) {
    wrote = true;
    if (e != 1.0f) {
#pragma unroll
      for (int i = 0; i < 16; i++) s[i] = s[i] * e;
    }
    proc = 1;
    if (live) {
      proc = 2;
      // k and q through the wave's LDS: value v of k at 20 (v / 16) + v % 16, of q at KQ_Q plus
      // the same (rows of 16 values 80 bytes apart, so the 16 rows a pass of 16 lanes reads lie
      // on distinct bank groups; 64 bytes apart they shared four)
      {
        const int v0 = 8 * (threadIdx.x & 31);
        v4f* dst = reinterpret_cast<v4f*>(kqs + (threadIdx.x < 32 ? 0 : KQ_Q) + 20 * (v0 >> 4) +
                                          (v0 & 15));
        dst[0] = cur.kq[0];
        dst[1] = cur.kq[1];
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const v4f* kq4 = reinterpret_cast<const v4f*>(kqs + 20 * b);
      float kr[16], qr[16];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const v4f kv4 = kq4[j], qv4 = kq4[KQ_Q / 4 + j];
        kr[4 * j] = kv4.x; kr[4 * j + 1] = kv4.y; kr[4 * j + 2] = kv4.z; kr[4 * j + 3] = kv4.w;
        qr[4 * j] = qv4.x; qr[4 * j + 1] = qv4.y; qr[4 * j + 2] = qv4.z; qr[4 * j + 3] = qv4.w;
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // the block's sum; a zero factor adds nothing (the oracle skips it; a sum from +0 is
      // never -0)
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) a = kr[i] != 0.0f ? a + s[i] * kr[i] : a;
      const float kv = col_sum16(red, c, b, a);
      const float d = (cur.v - kv) * cur.beta;
      float o = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        // (the update keeps rows with a zero key factor exactly as they are: -0 stays -0)
        s[i] = kr[i] != 0.0f ? s[i] + kr[i] * d : s[i];
        o = qr[i] != 0.0f ? o + s[i] * qr[i] : o;
      }
      const float q = col_sum16(red, c, b, o);
      // o goes into the record over v (read three candidates ago); the gated norm is pf_out's
      if (b == 0) ((GAS float*)((GAS uint8_t*)rec + ro.v))[vslot * VD + col] = rd<BF>(q);
    }
  }
  if (first) ((GAS int32_t*)((GAS uint8_t*)rec + ro.pr))[vslot] = proc;
}

template <bool BF>
__global__ __launch_bounds__(64) void pf_delta(const lxm_pf_params* __restrict__ pp, int L) {
  __shared__ __align__(16) float red[DCW * 16];
  __shared__ __align__(16) float kqs[2 * KQ_Q];  // a live step's k and q (rows of 20)
  const lxm_pf_params& p = *pp;
  const lxm_pf_layer& ly = p.layers[L];
  const int lane = threadIdx.x, c = lane >> 4, b = lane & 15;
  // a slot's DWS workgroups on one XCD (workgroups are dealt to the 8 XCDs in turn): the slot's
  // records are then fetched into one L2, and its columns' outputs merge in it
  const int xcd = blockIdx.x & 7, jx = blockIdx.x >> 3;
  const int vslot = xcd + 8 * (jx / DWS), c0 = (jx % DWS) * DCW;
  if (vslot >= ly.n_vs) return;
  // everything the loop needs in registers: its stores to the records could alias p and ly
  const lxm_pf_vs sv = tab<lxm_pf_vs>(p.blob, ly.vs)[vslot];
  const RecOff ro(ly.n_ks, ly.n_vs);
  const int count = p.count[L];
  const int64_t rec_b = ly.rec_bytes;
  uint8_t* const recs = p.recs;
  const int col = c0 + c, ks = sv.kslot;
  const bool first = lane == 0 && c0 == 0;
  float* S = p.rec[L] + (size_t)sv.vh * KD * VD + col;
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; i++) s[i] = S[(16 * b + i) * VD];
  bool wrote = false;
  // the inputs of the next three candidates in flight, in three fixed buffers (the loop taken
  // three candidates a round, so none is copied)
  DeltaIn n0 = {}, n1 = {}, n2 = {};
  if (count > 0) n0 = delta_in(recs, ro, vslot, ks, col, b);
  if (count > 1) n1 = delta_in(recs + rec_b, ro, vslot, ks, col, b);
  if (count > 2) n2 = delta_in(recs + 2 * rec_b, ro, vslot, ks, col, b);
  for (int j = 0; j < count; j += 3) {
    uint8_t* rec = recs + (int64_t)j * rec_b;
    {
      const DeltaIn cur = n0;
      if (j + 3 < count) n0 = delta_in(rec + 3 * rec_b, ro, vslot, ks, col, b);
      delta_step<BF>(cur, s, red, kqs, c, b, ks, rec, ro, vslot, col, first, wrote);
    }
    if (j + 1 < count) {
      const DeltaIn cur = n1;
      if (j + 4 < count) n1 = delta_in(rec + 4 * rec_b, ro, vslot, ks, col, b);
      delta_step<BF>(cur, s, red, kqs, c, b, ks, rec + rec_b, ro, vslot, col, first, wrote);
    }
    if (j + 2 < count) {
      const DeltaIn cur = n2;
      if (j + 5 < count) n2 = delta_in(rec + 5 * rec_b, ro, vslot, ks, col, b);
      delta_step<BF>(cur, s, red, kqs, c, b, ks, rec + 2 * rec_b, ro, vslot, col, first, wrote);
    }
  }
  if (wrote) {
#pragma unroll
    for (int i = 0; i < 16; i++) S[(16 * b + i) * VD] = s[i];
  }
}

// ---------------------------------------------------------------------------------------------
// The gated norm of each head that ran (TF:168-184): y = D(D(w * D(o * r)) * silu(z)), r =
// rsqrt(mean(o^2) + eps) with the squares summed per lane (dims lane, lane + 64) and then by the
// pairwise tree, one wave per head. Then out_proj and the residual add at the candidate
// (TF:541-543, :777-779): per residual row the terms over every value dim in ascending order,
// rounded once (lx/lx/fast.py:349-361), then h = D(h + that). Heads that did not run add nothing
// (their output is exactly 0 and the oracle skips zero inputs). One workgroup per candidate.
template <bool BF>
__global__ __launch_bounds__(NT) void pf_out(const lxm_pf_params* __restrict__ pp, int L) {
  extern __shared__ __align__(16) uint8_t sm[];
  __shared__ int any_s;
  const lxm_pf_params& p = *pp;
  const lxm_pf_layer& ly = p.layers[L];
  const int t = threadIdx.x, H = p.hidden, lane = t & 63, wv = t >> 6;
  float* ON = reinterpret_cast<float*>(sm);
  const RecOff ro(ly.n_ks, ly.n_vs);
  const lxm_pf_drow* orows = tab<lxm_pf_drow>(p.blob, ly.orows);
  const lxm_pf_ent* ent = tab<lxm_pf_ent>(p.blob, ly.ent);
  const float* gwp = tab<float>(p.blob, ly.gnorm);
  const float gw0 = gwp[lane], gw1 = gwp[lane + 64], geps = ly.geps;
  const int count = p.count[L], n_vs = ly.n_vs;
  for (int j = blockIdx.x; j < count; j += gridDim.x) {
    const uint8_t* rec = p.recs + (int64_t)j * ly.rec_bytes;
    const int tok = reinterpret_cast<const int32_t*>(rec)[0];
    const int32_t* pr = reinterpret_cast<const int32_t*>(rec + ro.pr);
    const float* o = reinterpret_cast<const float*>(rec + ro.v);
    const float* z = reinterpret_cast<const float*>(rec + ro.z);
    if (t == 0) any_s = 0;
    __syncthreads();
    for (int v = wv; v < n_vs; v += NT / 64) {
      float y0 = 0.0f, y1 = 0.0f;
      if (pr[v] == 2) {
        const float o0 = o[v * VD + lane], o1 = o[v * VD + lane + 64];
        const float z0 = z[v * VD + lane], z1 = z[v * VD + lane + 64];
        float ss = 0.0f;
        ss = ss + o0 * o0;
        ss = ss + o1 * o1;
        ss = sum64(ss);
        const float rr = rsqrt_(ss / (float)VD + geps);
        y0 = rd<BF>(rd<BF>(gw0 * rd<BF>(o0 * rr)) * silu(z0));
        y1 = rd<BF>(rd<BF>(gw1 * rd<BF>(o1 * rr)) * silu(z1));
        if (lane == 0) any_s = 1;
      }
      ON[v * VD + lane] = y0;
      ON[v * VD + lane + 64] = y1;
    }
    __syncthreads();
    if (any_s) {
      for (int i = t; i < ly.n_orows; i += NT) {
        const lxm_pf_drow r = orows[i];
        const float y = rd<BF>(dot1<BF>(ent + r.start, r.len, sm));
        st_el<BF>(p.h, H, tok, r.row, rd<BF>(ld_el<BF>(p.h, H, tok, r.row) + y));
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// The head (lx/lx/hf.py:179-184): logits D(hn . row) over the tied embedding rows, the first
// maximum per position. Workgroup (tile, slice): slice = the XCD the workgroup lands on, so each
// XCD's L2 keeps one eighth of the head. A thread takes rows in ascending order and keeps the
// first strict maximum; NaN logits (which compare false) are tracked apart and, where one
// occurred, the thread finds its first NaN row. The thread keys (value, lower index, NaN above
// everything: torch.argmax) fold into p->keys by 64-bit atomic max.
__device__ __forceinline__ unsigned long long kmax(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}
__device__ __forceinline__ unsigned long long wave_kmax(unsigned long long k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) k = kmax(k, __shfl_xor(k, off));
  return k;
}
// The head's scan over rows r0..r1 of a slice for the tile at LDS address 0 (pf_head)
template <bool BF, bool LONG>
__device__ __forceinline__ void head_scan(const lxm_pf_params& p, int64_t b, int r0, int r1) {
  const int t = threadIdx.x;
  const int32_t* hmore = p.head_more;
  const lxm_pf_ent* hent = p.head_ent;
  // each position's first strict maximum over the thread's rows: from -inf, so a row is taken
  // when it is above every earlier one; a thread whose rows are all -inf keeps its first row
  // (with a NaN row the NaN pass below decides, as NaN outranks every number)
  float best[TT];
  int bidx[TT];
  bool nan_any = false;
#pragma unroll
  for (int k = 0; k < TT; k++) {
    best[k] = -__builtin_inff();
    bidx[k] = r0 + t;
  }
  for (int r = r0 + t; r < r1; r += 4 * NT) {
    // four rows a step (r, r + NT, r + 2 NT, r + 3 NT, each coalesced across the wave), their
    // entries requested together; rows taken in ascending order (the first strict maximum); a
    // row past the slice is r again, which adds nothing (not above itself)
    int rr[4];
    HRow h[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      rr[i] = r + i * NT < r1 ? r + i * NT : r;
      hrow_req<LONG>(hmore, hent, rr[i], h[i]);
    }
    v4f sv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sv[i] = rd4<BF>(hrow_sum<BF>(hent, h[i]));
#pragma unroll
    for (int k = 0; k < TT; k++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v = sv[i][k];
        nan_any |= v != v;
        if (v > best[k]) {
          best[k] = v;
          bidx[k] = rr[i];
        }
      }
    }
  }
  unsigned long long key[TT];
#pragma unroll
  for (int k = 0; k < TT; k++) key[k] = r0 + t < r1 ? argmax_key(best[k], bidx[k]) : 0ull;
  if (nan_any) {  // rare: the first NaN row of each position, which outranks every number
    for (int r = r0 + t; r < r1; r += NT) {
      HRow h;
      hrow_req<LONG>(hmore, hent, r, h);
      const v4f s = rd4<BF>(hrow_sum<BF>(hent, h));
#pragma unroll
      for (int k = 0; k < TT; k++)
        if (s[k] != s[k]) key[k] = kmax(key[k], argmax_key(s[k], r));
    }
  }
#pragma unroll
  for (int k = 0; k < TT; k++) {
    const unsigned long long w = wave_kmax(key[k]);
    if ((t & 63) == 0 && b * TT + k < p.T && w != 0ull) atomicMax(p.keys + b * TT + k, w);
  }
}

template <bool BF>
__global__ __launch_bounds__(NT) void pf_head(const lxm_pf_params* __restrict__ pp) {
  extern __shared__ __align__(16) uint8_t sm[];
  const lxm_pf_params& p = *pp;
  const int t = threadIdx.x, H = p.hidden;
  const int slice = blockIdx.x % LXM_PF_SLICES;
  const int64_t b = blockIdx.x / LXM_PF_SLICES;
  // the tile's columns are read at LDS address 16 x column (sum4z): the tile must start at 0
  if ((uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)sm != 0u) {
    if (t == 0) *p.err = 2;
    return;
  }
  load_tile<BF, false>(p.hn, b, H, sm);
  if (t == 0) reinterpret_cast<v4f*>(sm)[H] = v4f{0.0f, 0.0f, 0.0f, 0.0f};  // the padding's column
  __syncthreads();
  const int r0 = p.head_slice[slice], r1 = p.head_slice[slice + 1];
  if (p.head_long) head_scan<BF, true>(p, b, r0, r1);
  else head_scan<BF, false>(p, b, r0, r1);
}

__global__ void pf_fill_keys(const lxm_pf_params* __restrict__ pp) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < pp->T) pp->keys[i] = 0ull;
}
__global__ void pf_preds(const lxm_pf_params* __restrict__ pp) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < pp->T) pp->preds[i] = argmax_idx(pp->keys[i]);
}

// ---------------------------------------------------------------------------------------------
// The embedding rows of the positions' tokens into the residual tiles (one workgroup per tile).
template <bool BF>
__global__ __launch_bounds__(NT) void pf_embed(const lxm_pf_params* __restrict__ pp) {
  extern __shared__ __align__(16) uint8_t sm[];
  const lxm_pf_params& p = *pp;
  const int t = threadIdx.x, H = p.hidden;
  const int64_t b = blockIdx.x;
  float* HV = reinterpret_cast<float*>(sm);
  for (int i = t; i < H * TT; i += NT) HV[i] = 0.0f;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < TT; k++) {
    const int64_t pos = b * TT + k;
    if (pos >= p.T) continue;
    const int tok = p.tokens[pos];
    if (tok < 0 || tok >= p.vocab) {
      if (t == 0) *p.err = 1;
      continue;
    }
    const int64_t e0 = p.emb_ptr[tok], e1 = p.emb_ptr[tok + 1];
    for (int64_t e = e0 + t; e < e1; e += NT) {
      const lxm_pf_ent en = p.emb_ent[e];
      HV[en.off * TT + k] = en.w;
    }
  }
  __syncthreads();
  for (int c = t; c < H; c += NT) st_col<BF>(p.h, b, H, c, reinterpret_cast<const v4f*>(HV)[c]);
}

// row-major (T, H) <-> tiles, one element per thread
template <bool BF>
__global__ void pf_tiles_k(const void* x, void* y, int T, int H, int dir) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)T * H) return;
  const int t = (int)(i / H), c = (int)(i % H);
  const int64_t j = el_idx(H, t, c);
  const int64_t from = dir == 0 ? i : j, to = dir == 0 ? j : i;
  if constexpr (BF) reinterpret_cast<uint16_t*>(y)[to] = reinterpret_cast<const uint16_t*>(x)[from];
  else reinterpret_cast<float*>(y)[to] = reinterpret_cast<const float*>(x)[from];
}

// ---------------------------------------------------------------------------------------------
// Host side.
template <bool BF>
static int tile_lds(int H, int n_units_max) {
  return x_xm<BF>(H) + TV<BF>::B * (n_units_max + 1);
}
#define ACT_LDS (A_MISC + 16)
#define ACT_GRID 1024
#define OUT_GRID 1024

// Dynamic LDS above 64 KB needs the kernel's attribute raised first (to the bytes it launches with).
static hipError_t lds_attr(const void* k, int bytes) {
  return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <bool BF>
static hipError_t run_layers(const lxm_pf_params* ph, const lxm_pf_params* pd, int l0, int l1,
                             hipStream_t st) {
  const int ntiles = ph->ntiles;
  int umax = 0;
  for (int L = l0; L < l1; L++) umax = ph->layers_host[L].n_units > umax ? ph->layers_host[L].n_units : umax;
  const int xl = tile_lds<BF>(ph->hidden, umax);
  hipError_t e = lds_attr((const void*)pf_tile<BF>, xl);
  if (e == hipSuccess) e = lds_attr((const void*)pf_act<BF>, ACT_LDS);
  if (e == hipSuccess) e = lds_attr((const void*)pf_out<BF>, 4 * VD * LXM_PF_MAXVS + 16);
  if (e != hipSuccess) return e;
  for (int L = l0; L < l1; L++) {
    const lxm_pf_layer& ly = ph->layers_host[L];
    hipLaunchKernelGGL(pf_tile<BF>, dim3(ntiles), dim3(NT), xl, st, pd, L == l0 ? -1 : L - 1, L);
    hipLaunchKernelGGL(pf_compact, dim3(1), dim3(C_NT), 0, st, pd, L);
    hipLaunchKernelGGL(pf_act<BF>, dim3(ACT_GRID), dim3(NT), ACT_LDS, st, pd, L);
    hipLaunchKernelGGL(pf_tail<BF>, dim3((ph->n_conv + 255) / 256), dim3(256), 0, st, pd, L);
    // (DWS one-wave workgroups per value-head slot, DCW state columns each, a slot's on one XCD)
    if (ly.n_vs > 0)
      hipLaunchKernelGGL(pf_delta<BF>, dim3(8 * DWS * ((ly.n_vs + 7) / 8)), dim3(64), 0, st, pd, L);
    if (ly.n_vs > 0)
      hipLaunchKernelGGL(pf_out<BF>, dim3(OUT_GRID), dim3(NT), 4 * VD * ly.n_vs + 16, st, pd, L);
  }
  hipLaunchKernelGGL(pf_tile<BF>, dim3(ntiles), dim3(NT), xl, st, pd, l1 - 1, -1);
  return hipGetLastError();
}

template <bool BF>
static hipError_t run_head(const lxm_pf_params* ph, const lxm_pf_params* pd, hipStream_t st) {
  const int ntiles = ph->ntiles, T = ph->T;
  hipError_t e = lds_attr((const void*)pf_tile<BF>, tile_lds<BF>(ph->hidden, 0));
  if (e == hipSuccess) e = lds_attr((const void*)pf_head<BF>, 16 * ph->hidden + 64);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(pf_fill_keys, dim3((T + 255) / 256), dim3(256), 0, st, pd);
  hipLaunchKernelGGL(pf_tile<BF>, dim3(ntiles), dim3(NT), tile_lds<BF>(ph->hidden, 0), st, pd, -1, -2);
  hipLaunchKernelGGL(pf_head<BF>, dim3(ntiles * LXM_PF_SLICES), dim3(NT), 16 * ph->hidden + 64, st, pd);
  hipLaunchKernelGGL(pf_preds, dim3((T + 255) / 256), dim3(256), 0, st, pd);
  return hipGetLastError();
}

static bool ok_params(const lxm_pf_params* ph) {
  return ph && ph->hidden > 0 && ph->hidden <= MAXH && ph->T > 0 &&
         ph->ntiles == (ph->T + TT - 1) / TT && ph->layers_host;
}

extern "C" {

int lxm_pf_layers(const lxm_pf_params* ph, const lxm_pf_params* pd, int l0, int l1, void* stream) {
  if (!ok_params(ph) || l0 < 0 || l1 > ph->n_layers || l0 >= l1) return (int)hipErrorInvalidValue;
  for (int L = l0; L < l1; L++) {
    const lxm_pf_layer& ly = ph->layers_host[L];
    if (ly.n_units > LXM_PF_UPT * NT || ly.n_ks > LXM_PF_MAXKS || ly.n_vs > LXM_PF_MAXVS ||
        ly.rec_bytes > ph->max_rec)
      return (int)hipErrorInvalidValue;
  }
  hipStream_t st = (hipStream_t)stream;
  return (int)(ph->bf16 ? run_layers<true>(ph, pd, l0, l1, st) : run_layers<false>(ph, pd, l0, l1, st));
}

int lxm_pf_head(const lxm_pf_params* ph, const lxm_pf_params* pd, void* stream) {
  if (!ok_params(ph)) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  return (int)(ph->bf16 ? run_head<true>(ph, pd, st) : run_head<false>(ph, pd, st));
}

int lxm_pf_embed(const lxm_pf_params* ph, const lxm_pf_params* pd, void* stream) {
  if (!ok_params(ph)) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  const int lds = 16 * ph->hidden;
  hipError_t e = lds_attr(ph->bf16 ? (const void*)pf_embed<true> : (const void*)pf_embed<false>, lds);
  if (e != hipSuccess) return (int)e;
  if (ph->bf16) hipLaunchKernelGGL(pf_embed<true>, dim3(ph->ntiles), dim3(NT), lds, st, pd);
  else hipLaunchKernelGGL(pf_embed<false>, dim3(ph->ntiles), dim3(NT), lds, st, pd);
  return (int)hipGetLastError();
}

int lxm_pf_tiles(const lxm_pf_params* ph, const void* x, void* y, int dir, void* stream) {
  if (!ok_params(ph) || (dir != 0 && dir != 1)) return (int)hipErrorInvalidValue;
  const int64_t n = (int64_t)ph->T * ph->hidden;
  hipStream_t st = (hipStream_t)stream;
  const dim3 g((unsigned)((n + 255) / 256));
  if (ph->bf16) hipLaunchKernelGGL(pf_tiles_k<true>, g, dim3(256), 0, st, x, y, ph->T, ph->hidden, dir);
  else hipLaunchKernelGGL(pf_tiles_k<false>, g, dim3(256), 0, st, x, y, ph->T, ph->hidden, dir);
  return (int)hipGetLastError();
}

int lxm_pf_lds(int bf16, int hidden, int n_units) {
  return bf16 ? tile_lds<true>(hidden, n_units) : tile_lds<false>(hidden, n_units);
}

}  // extern "C"
