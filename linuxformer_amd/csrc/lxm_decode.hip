// linuxformer's chip-layer greedy decode as one persistent kernel for MI355X (gfx950).
//
// What it computes is lx.mega's decode (lx/csrc/mega.cu:653-862): per token, the embedding row,
// every chip layer's Gated DeltaNet step and SwiGLU MLP, the final norm and the tied head's
// argmax, fed back as the next input on the GPU; conv windows and recurrent states updated in
// place. How it computes it is MI355X's own design:
//
// * The dependent chain of a token (37 layers, each: RMSNorm, the write gates, the MLP) runs
//   inside ONE workgroup (block 0, "the chain"): the residual stream lives in its LDS and every
//   layer's resident tables (norm weights, MLP rows, the query/key/decay rows the gates read)
//   are streamed into LDS one layer ahead through registers. A grid-wide round trip costs
//   ~4 us across MI355X's 8 XCDs (measured), so the reference's ~38 barriered phases per token
//   would cost more than its whole H100 step; here a token crosses the grid once, plus once
//   per layer whose write gates open.
// * The other workgroups ("helpers") serve events the chain posts in one 32-bit word:
//   - HEAD (once per token): each helper holds a slice of the output head (459,982 rows) in
//     LDS for the whole launch, reduces its rows to one argmax key and folds it into a 64-bit
//     atomicMax. Keys order by (value, lower index) as torch.argmax breaks ties.
//   - GDN (a layer whose gates opened): helper 1 + vh owns value head vh's recurrent state (of
//     every layer: one owner, so the state never needs cross-XCD coherence) and runs its delta
//     rule, gated norm and output; then every helper computes a slice of out_proj's rows from
//     all heads' outputs. The chain adds the rows to the residual.
//   Cross-block data moves through agent-scope atomic loads and stores (sc1 on gfx950) and
//   per-writer stamps (each workgroup stores the number of the event it has finished on a line of
//   its own; the waiting workgroup reads all the lines at once), so nothing is reset.
// * Gates instead of speculation: the chain computes, for each layer, the query/key channels'
//   conv outputs and the decays first (a few rows), so it knows exactly whether the layer's
//   delta rule runs and whether it can change the residual; the MLP is computed alongside and
//   redone only when it did. The conv windows are not shifted channel by channel every step:
//   the chain keeps the last four tokens' GDN norm outputs per layer (a ring in HBM), the
//   helpers rebuild the few windows an active head needs from it, the chain keeps its
//   query/key channels' windows in LDS, and every window is written once at the launch's end.
//
// Arithmetic: the rounding contract of lxm_math.h; sums in the orders documented per site.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/lxm.h"
#include "lxm_math.h"
#include "lxm_sync.h"

using namespace lxm;

#define NT LXM_NT
#define NW (NT / 64)
#define MAXH LXM_MAXH
#define KD LXM_KD
#define VD LXM_VD
#define RMAX LXM_RMAX
static_assert(MAXH == 8 * NT, "eight residual rows per thread cover any hidden size");

// ---------------------------------------------------------------------------------------------
// LDS layout of the chain workgroup (bytes). The vectors rows gather from (act, xm, h) sit
// below 64 KB, so a gather's base folds into the ds_read's 16-bit offset.
#define L_ACT 0                       // float[MAXU]: the MLP units' outputs
#define L_XM (L_ACT + 4 * LXM_MAXU)   // float[MAXH]: the MLP norm's output
#define L_H (L_XM + 4 * MAXH)         // float[MAXH]: the residual (the gates gather from it)
#define L_DSUM (L_H + 4 * MAXH)       // float[MAXH]: down_proj's row sums
#define L_DUMMY (L_DSUM + 4 * MAXH)   // float[NT]: where a lane with no row in a pass writes
static_assert(L_DUMMY - L_DSUM + 4 * NT <= 65536, "down write offsets in 16 bits");
#define L_HIST (L_DUMMY + 4 * NT)     // the live q/k channels' conv history, 3 per channel
#define L_QKCUR (L_HIST + 4 * 3 * LXM_MAXQK)
#define L_EV (L_QKCUR + 4 * LXM_MAXQKL)
#define L_WSUM (L_EV + 4 * 256)       // float[3][8]: wave totals of the hidden sums
#define L_FLAGS (L_WSUM + 4 * 32)
#define L_PROF (L_FLAGS + 4 * 256)
#define L_LT (L_PROF + 8 * 32)        // the layer table (LtEnt[64])
#define L_PARAMS (L_LT + 32 * 64)     // the chain's copy of the parameter block
#define L_GATES (L_PARAMS + 512)      // the gate section, resident for the launch
#define L_SUBP (L_GATES + LXM_GATE_MAX + 64)  // (gate gathers read up to 4 entries past a row)
#ifdef LXM_SUBPROF
#define L_CHAIN_END (L_SUBP + 8 * (16 * SP_NS + 16))
#else
#define L_CHAIN_END L_SUBP
#endif
static_assert(L_H + 4 * MAXH <= 65536, "gathered vectors below 64 KB");
// flags (int): [0] any head active, [1] any query live (the residual may change), [4] ok,
// [8] token, [16 + kh] per key head: bit 0 query nonzero, bit 1 key nonzero, bit 2 a decay
#define F_ANY 0
#define F_OUT 1
#define F_OK 4
#define F_TOK 8
#define F_KH 16
#define F_KEYW 192  // 8 uint64: the head keys' wave maxima (key heads: nk <= F_KEYW - F_KH)
static_assert((L_FLAGS + 4 * F_KEYW) % 8 == 0 && F_KEYW + 16 <= 256, "the key words in the flags");

// LDS layout of a helper workgroup, before its head tables (p.head_lds bytes, from HX_END)
#define HX_X 0                        // hidden: the head's normed input
#define HX_QD (HX_X + 4 * MAXH)       // dense query / key of the task's key head, raw
#define HX_KD (HX_QD + 4 * KD)
#define HX_QN (HX_KD + 4 * KD)        // the same after l2norm (query scaled by 1/16)
#define HX_KN (HX_QN + 4 * KD)
#define HX_V (HX_KN + 4 * KD)         // value channels' conv outputs
#define HX_Z (HX_V + 4 * VD)          // in_proj_z rows
#define HX_DL (HX_Z + 4 * VD)         // delta = (v - kv) beta
#define HX_GW (HX_DL + 4 * VD)        // the gated norm's weight
#define HX_BS (HX_GW + 4 * VD)        // per row block (16 rows) partial sums, [16][VD]
#define HX_MISC (HX_BS + 4 * 16 * VD) // ints: [0] nq, [1] nk, [2] beta bits, [4] event, [5] ok
#define HX_OP (HX_MISC + 256)         // out_proj: the helper's row pointers (LXM_OUT_ROWS + 1)
#define HX_OE (HX_OP + 4 * (LXM_OUT_ROWS + 4))  // its entries (LXM_OUT_MAX, 8 bytes at most)
#define HX_OY (HX_OE + 8 * LXM_OUT_MAX)  // the head outputs each entry reads
#define HX_LT (HX_OY + 4 * LXM_OUT_MAX + 64)  // (reads run up to 3 slots past the end)
#define HX_PARAMS (HX_LT + 64 * (int)sizeof(lxm_layer))  // the layer table, resident for the launch
#define HX_END (HX_PARAMS + 512)      // the helper's copy of the parameter block

// sync words (uint32 indices into p.sync). The event word has one copy per group of helpers
// (group = block index mod 8, the XCD a block lands on when blocks are dealt round-robin), each
// on its own 128-byte line, so at most 32 workgroups poll one line. Completion travels as
// stamps: every writer owns its own 128-byte line and stores the number of the event it has
// finished (plain agent-scope stores, no atomics: counters that many workgroups add to
// serialise at the coherence point), and the waiting workgroup reads all the lines at once, one
// per thread, in one round trip per poll.
#define NGRP 8
#define S_EV 0       // + 32 g: seq << 8 | layer << 2 | out << 1 | kind (0 head, 1 gdn)
#define S_DONE 768
#define S_OWN 1024   // + 32 vh: the number of GDN events whose output value head vh has stored
#define S_XO (S_OWN + 32 * LXM_SCRATCH_MAXNV)  // + 32 j: the seq whose out_proj rows helper j stored
#define S_KEY (S_XO + 32 * LXM_OUT_HELPERS)    // + 32 b (a uint64): helper b's head key, stamped
#define S_END (S_KEY + 32 * LXM_MAXBLOCKS)
static_assert(S_END == LXM_NSYNC, "LXM_NSYNC matches the layout");
#define SEQ_MASK 0xffffffu   // an event's seq as its word carries it
#define KEY_STAMP 0x1fffu    // the head key's stamp bits (the seq's low 13 bits)
#define EV_GDN 1u
#define EV_OUT 2u

extern __shared__ __align__(16) uint8_t smem[];

// In-kernel phase counters (lx/csrc/mega.cu's prof buffer and MK_SUBPROF checkpoints): with
// p.prof set, thread 0 of the chain adds the shader-clock cycles of each phase into an LDS
// slot; the slots are written to p.prof at the end. Phases: 0 embedding, 1 the residual add
// and the next norm's sums (stage C2, and the trace), 2 the norms (stage A), 3 the gates and
// the MLP units (stage B), 4 a GDN event and the MLP's redo, 5 down_proj's rows (stage C1),
// 6 final norm + publish,
// 7 waiting for the head's argmax; counters 16 GDN events, 17 tokens. Helper b adds at
// 32 + 4b: 0 waiting for events, 1 head rows, 2 its value head's delta rule, 3 out_proj rows
// (with the wait for every head's output).
#define PROF_ON (p.prof != nullptr)
__device__ __forceinline__ uint64_t cycles() { return __builtin_readcyclecounter(); }

// Sub-phase profile (built with -DLXM_SUBPROF, lx.mega's MK_SUBPROF): per wave of the chain and
// per stage s (0 stage A, 1 stage B, 2 stage C1, 3 stage C2), the cycles the wave works before
// the stage's closing barrier (busy) and the cycles it then waits in the barrier (wait). The
// counters follow the helpers' in p.prof: [32 + 4 n_blocks + 16 s + w] busy, [.. + 8 + w] wait.
// GDN events, the embedding and the head are outside every stage (their time is skipped).
// The same build also timestamps every GDN event on the 100 MHz wall clock (comparable across
// workgroups): after the subprof slots, [0] the chain's sum of post times, [1] the sum of the
// times it saw every helper done, [2] the number of events; then per helper b at 4 + 4 b: the
// sums of the times it saw the event, had its value head's output stored (owners), saw every
// head's output (out_proj helpers) and had its out_proj rows stored; then per helper b at
// 4 + 4 n_blocks + 8 b: its value head's step, the sums of the times from its start to its
// checkpoints (0 query/key in, 1 values/z/beta in, 2 state tile computed, 3 state stored, 4
// output stored), the number of steps, the sum of whole steps that decayed, their number.
#define SP_NS 4
#define SP_EV (16 * SP_NS)
#ifdef LXM_SUBPROF
__device__ __forceinline__ uint64_t* sp_base() { return reinterpret_cast<uint64_t*>(smem + L_SUBP); }
__device__ __forceinline__ void sp_arrive(int s) {
  if ((threadIdx.x & 63) == 0) {
    uint64_t* sp = sp_base();
    const int w = threadIdx.x >> 6;
    const uint64_t now = cycles();
    sp[16 * s + w] += now - sp[16 * SP_NS + w];
    sp[16 * SP_NS + 8 + w] = now;
  }
}
__device__ __forceinline__ void sp_depart(int s) {
  if ((threadIdx.x & 63) == 0) {
    uint64_t* sp = sp_base();
    const int w = threadIdx.x >> 6;
    const uint64_t now = cycles();
    sp[16 * s + 8 + w] += now - sp[16 * SP_NS + 8 + w];
    sp[16 * SP_NS + w] = now;
  }
}
__device__ __forceinline__ void sp_skip() {
  if ((threadIdx.x & 63) == 0) sp_base()[16 * SP_NS + (threadIdx.x >> 6)] = cycles();
}
#else
__device__ __forceinline__ void sp_arrive(int) {}
__device__ __forceinline__ void sp_depart(int) {}
__device__ __forceinline__ void sp_skip() {}
#endif

// spin (one thread) until the word differs from last; 0 on timeout or another block's error
// (the word and the error word are requested together: one round trip a poll)
__device__ bool spin_ne(const uint32_t* p, uint32_t last, uint32_t* out, int32_t* err, int code) {
  const uint64_t t0 = wall();
  for (;;) {
    const uint32_t v = ld_rlx(p);
    const int32_t e = __hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v != last) {
      *out = v;
      return true;
    }
    if (e) return false;
    if (wall() - t0 > TIMEOUT_TICKS) {
      __hip_atomic_fetch_max(gp(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The workgroup waits until every thread t < n sees the word base[32 t] equal to want. Each wave
// holding a word spins on its own (one request of its words and of the error word a poll, its
// own time limit), with no barrier between polls; the workgroup meets once, at the end. All
// threads call; all return the same: false on an error or a timeout.
__device__ bool wait_stamps(const uint32_t* base, int n, uint32_t want, int32_t* err, int code) {
  const int t = threadIdx.x;
  int bad = 0;
  if (t - (t & 63) < n) {
    const uint64_t t0 = wall();
    for (;;) {
      const uint32_t v = ld_rlx(base + 32 * (t < n ? t : 0));
      const int32_t e = __hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (e != 0) {
        bad = 1;
        break;
      }
      if (__all(t >= n || v == want)) break;
      if (wall() - t0 > TIMEOUT_TICKS) {
        __hip_atomic_fetch_max(gp(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return __syncthreads_or(bad) == 0;
}

// Stamped words (8 bytes: a 32-bit value low, the GDN event's sequence number high), written
// and read whole at agent scope: a reader that sees the event's number in a word sees its value,
// with no separate completion flag.
__device__ __forceinline__ uint64_t ld64_rlx(const unsigned long long* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64_rlx(unsigned long long* p, uint32_t stamp, float v) {
  __hip_atomic_store(gp(p), ((unsigned long long)stamp << 32) | fbits(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// Every thread's words base[idx[i]] (idx[i] < 0: none): waits until all the workgroup's words
// carry the stamp want; v[i] their values (0 for none). Each wave spins on its own words as
// wait_stamps does. False on an error or a timeout (code).
template <int N>
__device__ bool wait_words(const unsigned long long* base, const int (&idx)[N], uint32_t want,
                           int32_t* err, int code, float (&v)[N]) {
  const uint64_t t0 = wall();
  int bad = 0;
  for (;;) {
    // (every word is requested, a thread without one reading word 0, and the error word beside
    // them, before any is looked at)
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = ld64_rlx(base + (idx[i] >= 0 ? idx[i] : 0));
    const int32_t e = __hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool mine = true;
#pragma unroll
    for (int i = 0; i < N; i++) {
      v[i] = idx[i] >= 0 ? __uint_as_float((uint32_t)w[i]) : 0.0f;
      mine = mine & ((idx[i] < 0) | ((uint32_t)(w[i] >> 32) == want));
    }
    if (e != 0) {
      bad = 1;
      break;
    }
    if (__all(mine)) break;
    if (wall() - t0 > TIMEOUT_TICKS) {
      __hip_atomic_fetch_max(gp(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bad = 1;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return __syncthreads_or(bad) == 0;
}

// The same for the head's keys: helper b = 1 .. n stores at S_KEY + 32 b a uint64 whose low 13
// bits are the HEAD event's stamp; the workgroup waits for every stamp, then takes the largest
// key (every valid key carries the same stamp, so the maximum is the maximum of the keys
// themselves). Returns false on an error or a timeout; *best: the maximum.
__device__ bool wait_keys(const uint32_t* sync, int n, uint32_t stamp, int32_t* err, int code,
                          unsigned long long* wk, unsigned long long* best) {
  const int t = threadIdx.x;
  const bool has = t >= 1 && t <= n;
  unsigned long long k = 0;
  int bad = 0;
  if (t - (t & 63) <= n) {  // the waves holding a key spin on their own, as wait_stamps's do
    const uint64_t t0 = wall();
    for (;;) {
      const unsigned long long k0 = __hip_atomic_load(
          gp(reinterpret_cast<const unsigned long long*>(sync + S_KEY + 32 * (has ? t : 1))),
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int32_t e = __hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      k = has ? k0 : 0ull;
      if (e != 0) {
        bad = 1;
        break;
      }
      if (__all(!has || (uint32_t)(k & KEY_STAMP) == stamp)) break;
      if (wall() - t0 > TIMEOUT_TICKS) {
        __hip_atomic_fetch_max(gp(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (__syncthreads_or(bad)) return false;
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(k, off, 64);
    k = o > k ? o : k;
  }
  if ((t & 63) == 0) wk[t >> 6] = k;
  __syncthreads();
  unsigned long long m = wk[0];
  for (int w = 1; w < NT / 64; w++) m = wk[w] > m ? wk[w] : m;
  *best = m;
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------------------------------------
// packed entries (LDS or global)
template <bool E4>
struct Ent;
template <>
struct Ent<true> {
  static constexpr int SZ = 4;
  __device__ static __forceinline__ void at(const uint8_t* base, int64_t e, int& idx, float& v) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(base)[e];
    idx = (int)(w & 0xffffu);
    v = bf16f(w >> 16);
  }
  __device__ static __forceinline__ void gat(const uint8_t* base, int64_t e, int& idx, float& v) {
    const uint32_t w = gp(reinterpret_cast<const uint32_t*>(base))[e];
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
  __device__ static __forceinline__ void gat(const uint8_t* base, int64_t e, int& idx, float& v) {
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    const v2u w = gp(reinterpret_cast<const v2u*>(base))[e];
    idx = (int)w.x;
    v = __uint_as_float(w.y);
  }
};

// the float at byte offset off of vector x
__device__ __forceinline__ float at_b(const float* x, int off) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(x) + off);
}
#define OFF_MASK (4 * MAXH - 4)

// Dot products of a sparse row with x (a hidden-sized or unit-sized vector), in entry order
// from +0. Entries store the column as a byte offset into x. A chunk issues the loads of N entries at once, unconditionally (every table is
// followed by at least N entries' worth of bytes, so they stay inside the LDS region or the
// blob), keeps the index inside the vector's MAXH slots (index & (MAXH - 1)) and gives the
// slots past the row's end weight 0, so the code has no branches. Every x the slots can reach
// is finite (LDS starts zeroed; the ring starts zeroed), so a weight-0 term, like a term with
// x == 0, adds +-0 to a sum that started from +0 and is never -0: the sum's bits are those of
// the row's own terms, in order (the oracle skips x == 0 terms; same bits). Where: 0 x in LDS,
// 1 entries in global memory and x in LDS.
template <bool BF, bool E4, int N, int WHERE>
__device__ __forceinline__ float chunk(const uint8_t* ent, int64_t start, int n, int k0,
                                       const float* x, float s) {
  int i[N];
  float w[N], xv[N];
#pragma unroll
  for (int j = 0; j < N; j++) {
    if constexpr (WHERE == 0) Ent<E4>::at(ent, start + k0 + j, i[j], w[j]);
    else Ent<E4>::gat(ent, start + k0 + j, i[j], w[j]);
  }
#pragma unroll
  for (int j = 0; j < N; j++) {
    i[j] &= OFF_MASK;
    w[j] = k0 + j < n ? w[j] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < N; j++) xv[j] = at_b(x, i[j]);
#pragma unroll
  for (int j = 0; j < N; j++) s = acc<BF>(s, xv[j], w[j]);
  return s;
}
template <bool BF, bool E4, int N, int WHERE>
__device__ __forceinline__ float rest(const uint8_t* ent, int64_t start, int n, const float* x,
                                      float s) {
  for (int k0 = N; k0 < n; k0 += N) s = chunk<BF, E4, N, WHERE>(ent, start, n, k0, x, s);
  return s;
}
template <bool BF, bool E4, int N, int WHERE>
__device__ __forceinline__ float dot(const uint8_t* ent, int64_t start, int n, const float* x) {
  return rest<BF, E4, N, WHERE>(ent, start, n, x, chunk<BF, E4, N, WHERE>(ent, start, n, 0, x, 0.0f));
}

// the 512-lane hidden sum: lane t's partial (its elements 4t..4t+3, then 2048+4t..2048+4t+3,
// in order), combined within each wave at offsets 32..1, the 8 wave totals at offsets 4, 2, 1.
// All threads call; all get the sum. In two halves, so a caller can put LDS writes between
// the halves' barriers (the second orders them).
__device__ __forceinline__ void sum512_begin(float s, float* wsum, int sp = -1) {
  s = wave_tree(s);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  if (sp >= 0) sp_arrive(sp);
  lds_barrier();
  if (sp >= 0) sp_depart(sp);
}
__device__ __forceinline__ float sum512_end(const float* wsum, int sp = -1) {
  float w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
  if (sp >= 0) sp_arrive(sp);
  lds_barrier();
  if (sp >= 0) sp_depart(sp);
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}
__device__ __forceinline__ float sum512(float s, float* wsum) {
  sum512_begin(s, wsum);
  return sum512_end(wsum);
}


// ---------------------------------------------------------------------------------------------
// a conv state value (model dtype) as float
template <bool BF>
__device__ __forceinline__ float conv_at(const void* cs, int64_t i) {
  if constexpr (BF) return bf16f(gp(reinterpret_cast<const uint16_t*>(cs))[i]);
  else return gp(reinterpret_cast<const float*>(cs))[i];
}
template <bool BF>
__device__ __forceinline__ void conv_put(void* cs, int64_t i, float v) {
  if constexpr (BF) gp(reinterpret_cast<uint16_t*>(cs))[i] = (uint16_t)(__float_as_uint(v) >> 16);
  else gp(reinterpret_cast<float*>(cs))[i] = v;
}

// The ring of the last four steps' layer inputs (the residual before the GDN's norm): slot
// (step & 3), layer L, MAXH floats each (bf16 models: MAXH bf16 values, the residual being
// bf16-exact there), and each entry's norm factor r (rring). The GDN norm's output of a step is
// D((h * r) * (1 + w_in)) from them.
__device__ __forceinline__ float* ring_at(const lxm_params& p, int step, int L) {
  return p.ring + ((size_t)(step & 3) * p.n_layers + L) * MAXH;
}
__device__ __forceinline__ float* rr_at(const lxm_params& p, int step, int L) {
  return p.rring + (size_t)(step & 3) * p.n_layers + L;
}
// 16 bytes to global memory at agent scope (a buffer store with the sc1 policy: written through
// to the coherence point, like the relaxed atomic stores)
__device__ __forceinline__ void st4_rlx(float* base, int idx, v4f v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(wave_ptr(base), 0, 0x7fffffff, 0x00020000);
  typedef uint32_t v4u_ __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_, v), r, idx * 4, 0, 16);
}
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
// 8 bytes to global memory at agent scope (idx in 32-bit words)
__device__ __forceinline__ void st2_rlx(float* base, int idx, v2u v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(wave_ptr(base), 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b64(v, r, idx * 4, 0, 16);
}
// four bf16-exact floats as their bf16 bits, two per word (low half first)
__device__ __forceinline__ v2u pack_bf16(const v4f& v) {
  return v2u{(__float_as_uint(v.x) >> 16) | (__float_as_uint(v.y) & 0xffff0000u),
             (__float_as_uint(v.z) >> 16) | (__float_as_uint(v.w) & 0xffff0000u)};
}
// one norm weight 1 + w of column c from a layer's w1 table (LDS or global)
template <bool E4, bool GLOBAL>
__device__ __forceinline__ float w1_one(const uint8_t* tab, int c) {
  if constexpr (E4) {
    const uint16_t b = GLOBAL ? gp(reinterpret_cast<const uint16_t*>(tab))[c]
                              : reinterpret_cast<const uint16_t*>(tab)[c];
    return 1.0f + bf16f(b);
  } else {
    return GLOBAL ? gp(reinterpret_cast<const float*>(tab))[c] : reinterpret_cast<const float*>(tab)[c];
  }
}
// The ring word holding the value at byte offset off of a ring row that is the same for every
// lane of the wave (its base is taken from the first active lane), by an agent-scope buffer load
// (sc1 policy), and the value from that word. The loads of a group of entries are all issued
// before any value is taken from its word.
template <bool BF>
__device__ __forceinline__ uint32_t ring_word(const float* hs, int off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(wave_ptr(const_cast<float*>(hs)), 0, 0x7fffffff, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, BF ? (off >> 3) * 4 : off, 0, 16);
}
template <bool BF>
__device__ __forceinline__ float ring_of(uint32_t w, int off) {
  if constexpr (BF) return __uint_as_float((off & 4) ? (w & 0xffff0000u) : (w << 16));
  else return __uint_as_float(w);
}
// the ring value at byte offset off of a ring row of this lane's own (agent-scope load)
template <bool BF>
__device__ __forceinline__ float ring_val(const float* hs, int off) {
  if constexpr (BF) {
    const uint32_t w = ld_rlx(reinterpret_cast<const uint32_t*>(hs) + (off >> 3));
    return __uint_as_float((off & 4) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return ld_rlxf(reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(hs) + off));
  }
}
// A row's dot product (entries in global memory, chunk's rules) with the GDN norm's output of
// a step, formed per entry from the ring: x[c] = D((h[c] * r) * (1 + w_in[c])), h by agent-
// scope loads. Only the columns the row names are read. UNI: the ring row hs is the same for
// every lane of the wave (a group's loads are then issued together); otherwise each lane reads
// its own.
template <bool BF, bool E4, bool UNI>
__device__ __forceinline__ float rdot(const uint8_t* ent, int64_t start, int n, const float* hs,
                                      float r, const uint8_t* w1in) {
  float s = 0.0f;
  for (int k0 = 0; k0 < n; k0 += 4) {
    int i[4];
    float w[4], hv[4], wi[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      Ent<E4>::gat(ent, start + k0 + j, i[j], w[j]);
      i[j] &= OFF_MASK;
    }
    if constexpr (UNI) {
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        u[j] = ring_word<BF>(hs, i[j]);
        wi[j] = w1_one<E4, true>(w1in, i[j] >> 2);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) hv[j] = ring_of<BF>(u[j], i[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        hv[j] = ring_val<BF>(hs, i[j]);
        wi[j] = w1_one<E4, true>(w1in, i[j] >> 2);
      }
    }
    // (a slot past the row may name a column past the weights: its term is dropped, not
    // weighted by 0)
#pragma unroll
    for (int j = 0; j < 4; j++) s = k0 + j < n ? acc<BF>(s, rd<BF>((hv[j] * r) * wi[j]), w[j]) : s;
  }
  return s;
}
// rdot over up to four steps' inputs at once, for a conv channel's window: window k (on[k], the
// same across the thread's calls) reads ring hs[k] with norm factor r[k], each row the same for
// every lane of the wave. Each sum keeps rdot's order; the entries and norm weights are read
// once, and all four windows' ring words of a group of entries are requested together.
template <bool BF, bool E4>
__device__ __forceinline__ void rdot4(const uint8_t* ent, int64_t start, int n,
                                      const float* const (&hs)[4], const float (&r)[4],
                                      const bool (&on)[4], const uint8_t* w1in, float (&out)[4]) {
#pragma unroll
  for (int k = 0; k < 4; k++) out[k] = 0.0f;
  for (int k0 = 0; k0 < n; k0 += 4) {
    int i[4];
    float w[4], wi[4], hv[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      Ent<E4>::gat(ent, start + k0 + j, i[j], w[j]);
      i[j] &= OFF_MASK;
      wi[j] = w1_one<E4, true>(w1in, i[j] >> 2);
    }
    // (an earlier window's words only where it is on; no word is looked at before all are
    // requested, so one wait covers the group)
    uint32_t u[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) u[k][j] = 0u;
#pragma unroll
    for (int k = 0; k < 3; k++)
      if (on[k]) {
#pragma unroll
        for (int j = 0; j < 4; j++) u[k][j] = ring_word<BF>(hs[k], i[j]);
      }
#pragma unroll
    for (int j = 0; j < 4; j++) u[3][j] = ring_word<BF>(hs[3], i[j]);
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) hv[k][j] = on[k] ? ring_of<BF>(u[k][j], i[j]) : 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (on[k] && k0 + j < n) out[k] = acc<BF>(out[k], rd<BF>((hv[k][j] * r[k]) * wi[j]), w[j]);
  }
}

// ---------------------------------------------------------------------------------------------
// The chain workgroup. Its LDS arrays are addressed from the dynamic shared array itself, so
// every access is a ds_read/ds_write.
#define LF(off) reinterpret_cast<float*>(smem + (off))
#define LI(off) reinterpret_cast<int*>(smem + (off))

// Qwen3_5RMSNorm's r = rsqrt(mean(h^2) + eps) (transformers qwen3_5 :727), mean = sum / n
__device__ __forceinline__ float norm_r(float ss, int H, float eps) {
  return rsqrt_(ss / (float)H + eps);
}
// The residual rows of thread t: 4t..4t+3 and 2048+4t..2048+4t+3, held in the thread's registers
// (ha, hb) and mirrored in LDS for the gates. Rows >= H hold +0, and +0 terms leave each lane's
// sum unchanged.
// (acc: s + x * x rounded once as the oracle's s + D32(x * x); for bf16 models x * x is exact)
template <bool BF>
__device__ __forceinline__ float sq_terms(const v4f& a, const v4f& b) {
  float s = 0.0f;
  s = acc<BF>(s, a.x, a.x);
  s = acc<BF>(s, a.y, a.y);
  s = acc<BF>(s, a.z, a.z);
  s = acc<BF>(s, a.w, a.w);
  s = acc<BF>(s, b.x, b.x);
  s = acc<BF>(s, b.y, b.y);
  s = acc<BF>(s, b.z, b.z);
  s = acc<BF>(s, b.w, b.w);
  return s;
}
// the sum of squares of the residual, whole (two barriers; wave totals in buffer 2)
template <bool BF>
__device__ __forceinline__ float hidden_ss(const v4f& ha, const v4f& hb) {
  return sum512(sq_terms<BF>(ha, hb), LF(L_WSUM) + 16);
}
// the second half of the sum of squares begun in stage C2 (buffer par; the buffers alternate
// by layer, so no barrier is needed after the reads)
__device__ __forceinline__ float sum512_take(const float* wsum) {
  float w[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) w[i] = wsum[i];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}

// The layer table in LDS: each layer's per-thread table and the offset of its gate tables in
// the resident gate section
struct LtEnt {
  const uint8_t* ptt;
  int32_t goff, pad;
  uint8_t words[8];  // per wave: the words of RU (low nibble) and RB (high nibble) it loads
  int32_t pad2[2];
};
// the words wave w of this thread loads of a layer's RU and RB regions
__device__ __forceinline__ uint32_t wave_words(const LtEnt* le) {
  return __builtin_amdgcn_readfirstlane((uint32_t)le->words[threadIdx.x >> 6]);
}
// The parameters the chain reads at every layer, read once into registers (a read of the
// parameter block, in LDS, would cost an LDS round trip per use)
struct ChainK {
  int H, nl, nk, nv, R;
  float* ring;
  float* rring;
  bool prof;
};
__device__ __forceinline__ float* ring_k(const ChainK& k, int step, int L) {
  return k.ring + ((size_t)(step & 3) * k.nl + L) * MAXH;
}
__device__ __forceinline__ float* rr_k(const ChainK& k, int step, int L) {
  return k.rring + (size_t)(step & 3) * k.nl + L;
}
// bf16 rounding of two values by one conversion (v_cvt_pk_bf16_f32), widened back to f32
typedef float v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2f rd2(v2f v) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
  return v2f{__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u)};
}
template <bool BF>
__device__ __forceinline__ v4f rd4(v4f v) {
  if constexpr (BF) {
    const v2f a = rd2(v2f{v.x, v.y}), b = rd2(v2f{v.z, v.w});
    return v4f{a.x, a.y, b.x, b.y};
  }
  return v;
}

// The per-thread table's slot layout (linuxformer_amd/chain.py packs it). ESZ slots per entry:
// e4 one (byte offset | bf16 << 16), else two (byte offset, float bits). Three regions, in 16-byte
// words, each prefetched into its own registers right after its last use in a layer, in the
// order the next layer uses them: RA = w1 + meta A (stages A and B), RU = the unit passes (stage
// B), RB = meta B + the down passes (stage C1).
// meta A: +0 the P0 unit's act index (bits 0-11, valid bit 15) and the P1 unit's (16-27, valid
// bit 31); +1 the lane's long unit (0-15, 0xffff = none); +2 (equal across the wave) G0 (0-3),
// G1 (4-7), shared columns in P0 (8) and P1 (9), any long unit (10).
// meta B: +0..+2 where each down pass's sum goes, 16 bits each: the byte offset from dsum of its
// row (4 row), or of the lane's dummy slot (L_DUMMY - L_DSUM + 4 lane) when it has none; +3 the
// lane's long row (0-15, 0xffff = none), the wave's down passes present (16-23) and any long
// row (24).
// A shared-column unit pass's up slots hold the weight alone (its offset bits 0), so the weight
// needs no mask.
template <bool E4>
struct PT;
template <>
struct PT<true> {
  static constexpr int ESZ = 1, W1 = 0, MA = 4, U0 = 8, U1 = 14, MB = 40, D = 44, WORDS = 15;
  static constexpr int G0MAX = 3, G1MAX = 13, ND = 6;
  // (the passes every wave uses first: a wave loads the words up to its last pass)
  __host__ __device__ static constexpr int dlen(int q) {
    return q == 2 ? 2 : q == 4 ? 4 : q == 5 ? 6 : 1;
  }
  __host__ __device__ static constexpr int doff(int q) {
    return q == 0 ? 0 : q == 1 ? 1 : q == 2 ? 2 : q == 3 ? 4 : q == 4 ? 5 : 9;
  }
};
template <>
struct PT<false> {
  static constexpr int ESZ = 2, W1 = 0, MA = 8, U0 = 12, U1 = 20, MB = 36, D = 40, WORDS = 13;
  static constexpr int G0MAX = 2, G1MAX = 4, ND = 4;
  __host__ __device__ static constexpr int dlen(int q) { return q < 2 ? 1 : 2; }
  __host__ __device__ static constexpr int doff(int q) { return q < 2 ? q : q == 2 ? 2 : 4; }
};
static_assert(PT<false>::WORDS <= LXM_PT_WORDS && PT<true>::WORDS <= LXM_PT_WORDS, "words");

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
// words A .. A + N - 1 of this thread's part of a per-thread table
template <int A, int N>
struct Words {
  v4u w[N];
  __device__ __forceinline__ uint32_t slot(int s) const { return w[(s >> 2) - A][s & 3]; }
  // every word live up to here: the register allocator may not reuse a loaded word's unused
  // slots before its consumer, which would make the next layer wait for the load in flight
  __device__ __forceinline__ void keep() const {
#pragma unroll
    for (int k = 0; k < N; k++) asm volatile("" ::"v"(w[k]));
  }
};
// (the first n of them: a wave loads only the words its passes use, n equal across the wave;
// the others stay unused)
template <int A, int N>
__device__ __forceinline__ Words<A, N> fetch_words(const uint8_t* ptt, int n = N) {
  const GAS v4u* src = gp(reinterpret_cast<const v4u*>(ptt)) + threadIdx.x;
  Words<A, N> r;
#pragma unroll
  for (int k = 0; k < N; k++) {
    if (k < n) r.w[k] = src[(A + k) * NT];
    else r.w[k] = v4u{0, 0, 0, 0};
  }
  return r;
}
template <bool E4>
struct Regions {
  using F = PT<E4>;
  static constexpr int RAA = 0, RAN = F::U0 / 4, RUA = F::U0 / 4, RUN = F::MB / 4 - F::U0 / 4,
                       RBA = F::MB / 4, RBN = F::WORDS - F::MB / 4;
  static_assert(F::MA % 4 == 0 && F::U0 % 4 == 0 && F::MB % 4 == 0 && F::D == F::MB + 4, "words");
  using RA = Words<RAA, RAN>;
  using RU = Words<RUA, RUN>;
  using RB = Words<RBA, RBN>;
};
// entry s of a region: its byte offset and weight
template <bool E4, class W>
__device__ __forceinline__ void ent_of(const W& r, int s, int& off, float& w) {
  if constexpr (E4) {
    const uint32_t e = r.slot(s);
    off = (int)(e & 0xffffu);
    w = __uint_as_float(e & 0xffff0000u);
  } else {
    off = (int)r.slot(s);
    w = __uint_as_float(r.slot(s + 1));
  }
}
#define ACT_MASK (4 * LXM_MAXU - 4)

// the MLP norm's weights 1 + w of the thread's rows: e4 the raw weights' bf16 bits (1 + w formed
// in fp32, as (1.0 + weight.float()) does), else 1 + w as fp32
template <bool E4>
__device__ __forceinline__ void w1_of(const typename Regions<E4>::RA& r1, v4f& wa, v4f& wb) {
  if constexpr (E4) {
    const v4u s = r1.w[0];
    wa = v4f{1.0f + __uint_as_float(s.x << 16), 1.0f + __uint_as_float(s.x & 0xffff0000u),
             1.0f + __uint_as_float(s.y << 16), 1.0f + __uint_as_float(s.y & 0xffff0000u)};
    wb = v4f{1.0f + __uint_as_float(s.z << 16), 1.0f + __uint_as_float(s.z & 0xffff0000u),
             1.0f + __uint_as_float(s.w << 16), 1.0f + __uint_as_float(s.w & 0xffff0000u)};
  } else {
    wa = __builtin_bit_cast(v4f, r1.w[0]);
    wb = __builtin_bit_cast(v4f, r1.w[1]);
  }
}

// silu and the MLP product for one unit (Qwen3_5MLP :715): D(D(silu(D(g))) * D(u))
template <bool BF>
__device__ __forceinline__ float swiglu(float gs, float us) {
  const float g = rd<BF>(gs), up = rd<BF>(us);
  const float sg = g == 0.0f ? g : silu_rd<BF>(g);  // silu(+-0) = +-0 / 2 = +-0
  return rd<BF>(rd<BF>(sg) * up);
}

template <bool BF>
__device__ __forceinline__ v4f norm4(const v4f& h, float r, const v4f& w) {
  return rd4<BF>(v4f{(h.x * r) * w.x, (h.y * r) * w.y, (h.z * r) * w.z, (h.w * r) * w.w});
}

// Stage A: the MLP norm's input D((h * r) * (1 + w)) (transformers qwen3_5 :729-734) of the
// thread's rows into xm, down_proj's row sums cleared, and with ring the layer input h and its
// norm factor r to the ring (the GDN norm's output, the same expression with its own weights,
// is formed where it is read). Rows past H compute from +0; nothing reads them.
template <bool BF, bool E4>
__device__ __forceinline__ void stage_a(const ChainK& k, const typename Regions<E4>::RA& r1,
                                        const v4f& ha, const v4f& hb, float r, int L, int step,
                                        bool ring, bool fly) {
  const int t = threadIdx.x;
  if (!fly) {  // (a FLY layer's unit passes form these themselves)
    v4f wa, wb;
    w1_of<E4>(r1, wa, wb);
    v4f* xm4 = reinterpret_cast<v4f*>(smem + L_XM);
    xm4[t] = norm4<BF>(ha, r, wa);
    xm4[NT + t] = norm4<BF>(hb, r, wb);
  }
  v4f* d4 = reinterpret_cast<v4f*>(smem + L_DSUM);
  d4[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  d4[NT + t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  if (ring) {
    float* rg = ring_k(k, step, L);
    if constexpr (BF) {  // four bf16 values in 8 bytes
      st2_rlx(rg, 2 * t, pack_bf16(ha));
      st2_rlx(rg, 1024 + 2 * t, pack_bf16(hb));
    } else {
      st4_rlx(rg, 4 * t, ha);
      st4_rlx(rg, 2048 + 4 * t, hb);
    }
    if (t == 0) st_rlxf(rr_k(k, step, L), r);
  }
}

// A unit pass: each lane's unit (gate row and up row, entries interleaved from slot base) over
// xm, padded to the wave's G entries, then act[u] = swiglu. Straight-line code for each G (equal
// across the wave, dispatched at run time): every gather of both passes first, then the sums
// (each row in entry order from +0; a padding entry adds +0), so the gathers' latencies overlap.
// (the gathered values travel as vector values, which stay in registers)
template <int GM>
struct PV {
  typedef float T __attribute__((ext_vector_type(GM <= 4 ? 4 : 16)));
  T x, y;
};
// FLY: the layer's passes all share columns and gather the residual h itself; pass_sum forms the
// MLP norm's output D((h * r) * (1 + w)) of each column, w from the up slot's low half (the rows
// of a FLY layer are never written to xm). Otherwise the passes gather xm.
template <bool E4, int G, bool SH, int GM, bool FLY, class RU>
__device__ __forceinline__ PV<GM> pass_gather(const RU& ru, int base) {
  constexpr int ESZ = PT<E4>::ESZ;
  const float* xm = FLY ? LF(L_H) : LF(L_XM);
  PV<GM> v;
#pragma unroll
  for (int j = 0; j < G; j++) {
    int o;
    float w;
    ent_of<E4>(ru, base + 2 * ESZ * j, o, w);
    v.x[j] = at_b(xm, o & OFF_MASK);
    if constexpr (!SH) {
      ent_of<E4>(ru, base + 2 * ESZ * j + ESZ, o, w);
      v.y[j] = at_b(xm, o & OFF_MASK);
    }
  }
  return v;
}
template <bool BF, bool E4, int G, bool SH, int GM, bool FLY, class RU>
__device__ __forceinline__ v2f pass_sum(const RU& ru, int base, const PV<GM>& v, float r) {
  constexpr int ESZ = PT<E4>::ESZ;
  float g = 0.0f, u = 0.0f;
#pragma unroll
  for (int j = 0; j < G; j++) {
    int o;
    float wg, wu;
    ent_of<E4>(ru, base + 2 * ESZ * j, o, wg);
    if constexpr (FLY) {
      const uint32_t us = ru.slot(base + 2 * j + 1);
      wu = __uint_as_float(us & 0xffff0000u);
      const float x = rd<BF>((v.x[j] * r) * (1.0f + __uint_as_float(us << 16)));
      g = acc<BF>(g, x, wg);
      u = acc<BF>(u, x, wu);
    } else {
      if constexpr (E4 && SH) wu = __uint_as_float(ru.slot(base + 2 * j + 1));
      else ent_of<E4>(ru, base + 2 * ESZ * j + ESZ, o, wu);
      g = acc<BF>(g, v.x[j], wg);
      u = acc<BF>(u, SH ? v.x[j] : v.y[j], wu);
    }
  }
  return v2f{g, u};
}
template <bool E4, int N, int GM, bool FLY, class RU>
__device__ __forceinline__ PV<GM> gather_g(const RU& ru, int base, int G, bool sh) {
  if constexpr (N >= 1) {
    if (G == N) {
      if constexpr (FLY) return pass_gather<E4, N, true, GM, true>(ru, base);
      else return sh ? pass_gather<E4, N, true, GM, false>(ru, base) : pass_gather<E4, N, false, GM, false>(ru, base);
    }
    return gather_g<E4, N - 1, GM, FLY>(ru, base, G, sh);
  } else {
    PV<GM> v;
    return v;
  }
}
template <bool BF, bool E4, int N, int GM, bool FLY, class RU>
__device__ __forceinline__ v2f sum_g(const RU& ru, int base, int G, bool sh, const PV<GM>& v, float r) {
  if constexpr (N >= 1) {
    if (G == N) {
      if constexpr (FLY) return pass_sum<BF, E4, N, true, GM, true>(ru, base, v, r);
      else return sh ? pass_sum<BF, E4, N, true, GM, false>(ru, base, v, r) : pass_sum<BF, E4, N, false, GM, false>(ru, base, v, r);
    }
    return sum_g<BF, E4, N - 1, GM, FLY>(ru, base, G, sh, v, r);
  } else {
    return v2f{0.0f, 0.0f};
  }
}

// whether a layer's unit passes form the MLP norm's output themselves (its wave-uniform word)
template <bool E4>
__device__ __forceinline__ bool fly_of(const typename Regions<E4>::RA& r1) {
  if constexpr (E4) return (__builtin_amdgcn_readfirstlane(r1.slot(PT<E4>::MA + 2)) & 2048u) != 0;
  else return false;
}

// Stage B's units: passes P0 and P1 of the thread, then its long unit (entries in LDS). r: the
// norm factor (FLY layers form each gathered column's norm output).
template <bool BF, bool E4, bool FLY>
__device__ __forceinline__ void units(const uint8_t* gt, const typename Regions<E4>::RA& r1,
                                      const typename Regions<E4>::RU& ru, float r) {
  using F = PT<E4>;
  const uint32_t m0 = r1.slot(F::MA + 0);
  const uint32_t m2 = __builtin_amdgcn_readfirstlane(r1.slot(F::MA + 2));
  const int G0 = (int)(m2 & 15u), G1 = (int)((m2 >> 4) & 15u);
  const bool sh0 = (m2 & 256u) != 0, sh1 = (m2 & 512u) != 0;
  float* act = LF(L_ACT);
  const PV<F::G0MAX> v0 = gather_g<E4, F::G0MAX, F::G0MAX, FLY>(ru, F::U0, G0, sh0);
  const PV<F::G1MAX> v1 = gather_g<E4, F::G1MAX, F::G1MAX, FLY>(ru, F::U1, G1, sh1);
  const v2f s0 = sum_g<BF, E4, F::G0MAX, F::G0MAX, FLY>(ru, F::U0, G0, sh0, v0, r);
  const v2f s1 = sum_g<BF, E4, F::G1MAX, F::G1MAX, FLY>(ru, F::U1, G1, sh1, v1, r);
  const float a0 = swiglu<BF>(s0.x, s0.y), a1 = swiglu<BF>(s1.x, s1.y);
  if (m0 & 0x8000u) act[m0 & 0xfffu] = a0;
  if (m0 & 0x80000000u) act[(m0 >> 16) & 0xfffu] = a1;
  ru.keep();
  r1.keep();
  if (m2 & 1024u) {
    const uint32_t li = r1.slot(F::MA + 1) & 0xffffu;
    if (li != 0xffffu) {  // a long unit: its rows from the layer's resident long tables
      const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
      const lxm_longu lu = reinterpret_cast<const lxm_longu*>(gt + hd.long_u)[li];
      const float* xm = LF(L_XM);
      const float g = dot<BF, E4, 4, 0>(gt + hd.long_ent, lu.gs, lu.gn, xm);
      const float u = dot<BF, E4, 4, 0>(gt + hd.long_ent, lu.us, lu.un, xm);
      act[lu.act] = swiglu<BF>(g, u);
    }
  }
}

// Stage C1: down_proj's rows, each lane one row per pass (entries in the model's unit order, from
// +0), the sum to dsum[row]; then the lane's long row
template <bool BF, bool E4>
__device__ __forceinline__ void down_rows(const uint8_t* gt, const typename Regions<E4>::RB& rdw) {
  using F = PT<E4>;
  constexpr int ESZ = F::ESZ;
  const int t = threadIdx.x;
  const uint32_t mb3 = rdw.slot(F::MB + 3);
  const uint32_t m2 = __builtin_amdgcn_readfirstlane(mb3);
  const uint32_t mask = (m2 >> 16) & 255u;
  const float* act = LF(L_ACT);
  float x[F::ND][8];
#pragma unroll
  for (int q = 0; q < F::ND; q++) {
    if (mask & (1u << q)) {
#pragma unroll
      for (int j = 0; j < F::dlen(q); j++) {
        int o;
        float w;
        ent_of<E4>(rdw, F::D + ESZ * (F::doff(q) + j), o, w);
        x[q][j] = at_b(act, o & ACT_MASK);
      }
    }
  }
  // every pass's sum first, then the writes (an LDS write between the sums would make each
  // later sum wait for it: LDS reads and writes share one counter)
  float sum[F::ND];
#pragma unroll
  for (int q = 0; q < F::ND; q++) {
    sum[q] = 0.0f;
    if (mask & (1u << q)) {
#pragma unroll
      for (int j = 0; j < F::dlen(q); j++) {
        int o;
        float w;
        ent_of<E4>(rdw, F::D + ESZ * (F::doff(q) + j), o, w);
        sum[q] = acc<BF>(sum[q], x[q][j], w);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < F::ND; q++) {
    if (mask & (1u << q)) {
      const uint32_t wo = (rdw.slot(F::MB + q / 2) >> (16 * (q & 1))) & 0xffffu;
      *reinterpret_cast<float*>(smem + L_DSUM + wo) = sum[q];
    }
  }
  rdw.keep();
  if (m2 & (1u << 24)) {
    const uint32_t li = mb3 & 0xffffu;
    if (li != 0xffffu) {  // a long row: its entries from the layer's resident long tables
      const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
      const lxm_longr lr = reinterpret_cast<const lxm_longr*>(gt + hd.long_r)[li];
      LF(L_DSUM)[lr.row] = dot<BF, E4, 4, 0>(gt + hd.long_ent, lr.start, lr.len, act);
    }
  }
}

// The gates: the live query/key channels' projections, conv windows (history in LDS) and silu
// (causal_conv1d_update :199-216), and the decays g = -exp(A_log) softplus(a + dt_bias) (:499).
// Flags per key head: 1 query nonzero, 2 key nonzero, 4 a decay exp(g) != 1; F_ANY and F_OUT
// directly.
// a gate row's dot product with the GDN norm's output D((h * r) * (1 + w_in)), formed per entry
// (w1e: the norm weight at each entry's column); slots past the row add nothing
template <bool BF, bool E4>
__device__ __forceinline__ float ndot(const uint8_t* ent, int start, int n, float r,
                                      const uint8_t* w1e) {
  const float* h = LF(L_H);
  float s = 0.0f;
  for (int k0 = 0; k0 < n; k0 += 4) {
    int i[4];
    float w[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      Ent<E4>::at(ent, start + k0 + j, i[j], w[j]);
      i[j] &= OFF_MASK;
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      xv[j] = rd<BF>((at_b(h, i[j]) * r) * w1_one<E4, false>(w1e, start + k0 + j));
#pragma unroll
    for (int j = 0; j < 4; j++) s = k0 + j < n ? acc<BF>(s, xv[j], w[j]) : s;
  }
  return s;
}

// One gate item per lane: query/key channel j on thread NT - 1 - j (the top wave(s)), decay j on
// the wave(s) below them (the packer keeps ceil(n_qk / 64) * 64 + n_dec <= NT). Its loads (item,
// history, the row's entries and the residual at their columns) need no norm factor, so they are
// issued at the start of stage A (gate_load) and overlap its work; stage B forms the norm output
// per entry and the rest (gate_compute). Rows of more than four entries take ndot in stage B.
struct GateLd {
  v4f hv, w, we;  // the residual, weight and norm weight 1 + w_in of each entry
  v4f tp;         // query/key: the conv taps; decay: dt_bias, -exp(A_log)
  float h0, h1, h2;          // query/key: the conv history
  int kind, j, len, start, info;  // kind 0 none, 1 query/key, 2 decay; info: slot, or vh
};
template <bool BF, bool E4>
__device__ __forceinline__ GateLd gate_load(const uint8_t* gt) {
  const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
  const int tt = NT - 1 - (int)threadIdx.x;
  const int nq = hd.n_qk, tq = ((nq + 63) >> 6) << 6;
  GateLd g;
  g.kind = 0;
  g.len = 0;
  if (tt < nq) {
    const lxm_qkc c = reinterpret_cast<const lxm_qkc*>(gt + hd.qk)[tt];
    const float* hs = LF(L_HIST) + 3 * (hd.qk_base + tt);
    g.kind = 1;
    g.j = tt;
    g.len = c.len;
    g.start = c.start;
    g.info = c.slot;
    g.tp = v4f{c.taps[0], c.taps[1], c.taps[2], c.taps[3]};
    g.h0 = hs[0];
    g.h1 = hs[1];
    g.h2 = hs[2];
  } else if (tt >= tq && tt - tq < hd.n_dec) {
    const lxm_dec d = reinterpret_cast<const lxm_dec*>(gt + hd.dec)[tt - tq];
    g.kind = 2;
    g.j = tt - tq;
    g.len = d.len;
    g.start = d.start;
    g.info = d.vh;
    g.tp = v4f{d.dt_bias, d.A_log, 0.0f, 0.0f};
  }
  if (g.kind != 0 && g.len <= 4) {
    const uint8_t* ent = gt + hd.ent;
    const uint8_t* w1e = gt + hd.ent_w1;
    const float* h = LF(L_H);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      int i;
      float w;
      Ent<E4>::at(ent, g.start + e, i, w);
      g.w[e] = w;
      g.we[e] = w1_one<E4, false>(w1e, g.start + e);
      g.hv[e] = at_b(h, i & OFF_MASK);
    }
  }
  return g;
}
// the row's dot product with the GDN norm's output D((h * r) * (1 + w_in)), in entry order from
// +0: from the loaded entries, or by ndot for a longer row
template <bool BF, bool E4>
__device__ __forceinline__ float gate_dot(const uint8_t* gt, const GateLd& g, float r) {
  if (g.len <= 4) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) s = e < g.len ? acc<BF>(s, rd<BF>((g.hv[e] * r) * g.we[e]), g.w[e]) : s;
    return s;
  }
  const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
  return ndot<BF, E4>(gt + hd.ent, g.start, g.len, r, gt + hd.ent_w1);
}
template <bool BF, bool E4>
__device__ __forceinline__ void gate_compute(const ChainK& k, const uint8_t* gt, const GateLd& g,
                                             float r) {
  int* flags = LI(L_FLAGS);
  if (g.kind == 1) {
    const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
    const float P = rd<BF>(gate_dot<BF, E4>(gt, g, r));
    float y = 0.0f;
    y = y + g.tp[0] * g.h0;
    y = y + g.tp[1] * g.h1;
    y = y + g.tp[2] * g.h2;
    y = y + g.tp[3] * P;
    float* hs = LF(L_HIST) + 3 * (hd.qk_base + g.j);
    hs[0] = g.h1;
    hs[1] = g.h2;
    hs[2] = P;
    const float yr = rd<BF>(y);
    const float v = yr == 0.0f ? yr : rd<BF>(silu_rd<BF>(yr));
    LF(L_QKCUR)[g.j] = v;
    if (v != 0.0f) {
      const bool isk = (g.info & 256) != 0;
      atomicOr(&flags[F_KH + (g.info >> 9)], isk ? 2 : 1);
      atomicOr(&flags[F_ANY], 1);
      if (!isk) atomicOr(&flags[F_OUT], 1);
    }
  } else if (g.kind == 2) {
    const float a = rd<BF>(gate_dot<BF, E4>(gt, g, r));
    const float x = a + g.tp[0];
    float e;
    if (x < -104.0f && g.tp[1] > -__builtin_inff()) {
      e = 1.0f;  // exp(x) rounds to 0, so softplus is 0 and g = -exp(A_log) * 0 = -0
    } else {
      const float gg = g.tp[1] * softplus(x);
      e = cr_exp(gg);
    }
    LF(L_EV)[g.info] = e;
    if (e != 1.0f) {
      atomicOr(&flags[F_KH + g.info / k.R], 4);
      atomicOr(&flags[F_ANY], 1);
    }
  }
}


// A GDN event for layer L (the chain's side): publish the value heads' tasks (bit 0 the key
// head's query or key is live, bit 2 the head decays), their decays and the layer's live
// query/key channel values; post the event; wait until the helpers have done it: with a live
// query, until every out_proj helper has stored its rows (each had waited for every value
// head's output), which the chain then adds to the residual (already rounded); without, until
// every value head has stored its state. Returns false on an error.
template <bool BF, bool E4>
__device__ bool gdn_event(const lxm_params& p, int L, const uint8_t* gt, uint32_t& seq,
                          v4f& ha, v4f& hb) {
  const int t = threadIdx.x;
  const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
  int* flags = LI(L_FLAGS);
  const float* ev = LF(L_EV);
  const bool out = flags[F_OUT] != 0;
  if (t < p.nv) {
    const int f = flags[F_KH + t / (p.nv / p.nk)];
    const float e = ev[t];
    st_rlx(p.mb_task + t, ((f & 3) ? 1u : 0u) | (e != 1.0f ? 4u : 0u));
    st_rlxf(p.mb_e + t, e);
  }
  for (int j = t; j < hd.n_qk; j += NT) st_rlxf(p.mb_qk + j, LF(L_QKCUR)[j]);
  drain();  // these and stage A's ring stores, visible at agent scope
  __syncthreads();
  seq++;
  if (t < NGRP)
    st_rlx(p.sync + S_EV + 32 * t, (seq << 8) | ((uint32_t)L << 2) | (out ? EV_OUT : 0u) | EV_GDN);
#ifdef LXM_SUBPROF
  const uint64_t tpost = wall();
#endif
  const int no = p.n_blocks - 1 < LXM_OUT_HELPERS ? p.n_blocks - 1 : LXM_OUT_HELPERS;
  const bool ok = wait_stamps(p.sync + (out ? S_XO : S_OWN), out ? no : p.nv, seq & SEQ_MASK,
                             p.err, 4);
#ifdef LXM_SUBPROF
  if (t == 0 && p.prof) {
    uint64_t* evs = reinterpret_cast<uint64_t*>(p.prof) + 32 + 4 * p.n_blocks + SP_EV;
    evs[0] += tpost;
    evs[1] += wall();
    evs[2] += 1;
  }
#endif
  if (!ok) return false;
  if (out) {  // (rows past H: xo holds +0 there, and so does h)
    const v4f xa = ld4_rlx(p.xo, 4 * t), xb = ld4_rlx(p.xo, 2048 + 4 * t);
    ha = v4f{rd<BF>(ha.x + xa.x), rd<BF>(ha.y + xa.y), rd<BF>(ha.z + xa.z), rd<BF>(ha.w + xa.w)};
    hb = v4f{rd<BF>(hb.x + xb.x), rd<BF>(hb.y + xb.y), rd<BF>(hb.z + xb.z), rd<BF>(hb.w + xb.w)};
    v4f* h4 = reinterpret_cast<v4f*>(smem + L_H);
    h4[t] = ha;
    h4[NT + t] = hb;
  }
  __syncthreads();
  return true;
}

// The gate flags and decay factors a layer's stage B writes, cleared beforehand (in the previous
// layer's stage C2, and before the first token): live key heads, each value head's exp(g), and
// whether any gate opened / any query was live.
__device__ __forceinline__ void clear_gate_flags(const ChainK& k) {
  const int t = threadIdx.x;
  int* flags = LI(L_FLAGS);
  if (t < k.nk) flags[F_KH + t] = 0;
  if (t < k.nv) LF(L_EV)[t] = 1.0f;
  if (t < 2) flags[F_ANY + t] = 0;
}

// One layer. ss: the sum of squares of h on entry. Ends inside the sum of squares of its output
// (sum512_begin into wave-total buffer par): the caller takes it. False on an error.
template <bool BF, bool E4>
__device__ __forceinline__ bool layer(const lxm_params& p, const ChainK& k, int L, int step,
                                      float ss, int par,
                                      v4f& ha, v4f& hb, typename Regions<E4>::RA& r1,
                                      typename Regions<E4>::RU& ru, typename Regions<E4>::RB& rdw,
                                      const LtEnt* lnext, uint32_t& seq) {
  using RG = Regions<E4>;
  const int t = threadIdx.x, H = k.H;
  const LtEnt le = reinterpret_cast<const LtEnt*>(smem + L_LT)[L];
  const uint8_t* gt = smem + L_GATES + le.goff;
  const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
  float* ev = LF(L_EV);
  int* flags = LI(L_FLAGS);
  uint64_t* pa = reinterpret_cast<uint64_t*>(smem + L_PROF);
  // ---- stage A: both norms' factor (the GDN's input_layernorm :764 and the MLP's
  // post_attention_layernorm :789 read the same h when the GDN leaves it alone)
  const GateLd gl = gate_load<BF, E4>(gt);
  const float r = norm_r(ss, H, hd.eps);
  const bool fly = fly_of<E4>(r1);
  stage_a<BF, E4>(k, r1, ha, hb, r, L, step, true, fly);
  if (!fly) {  // (a FLY layer writes no norm output: nothing for stage B to wait for)
    sp_arrive(0);
    lds_barrier();
    sp_depart(0);
  }
  uint64_t c0 = 0;
  if (k.prof && t == 0) {
    c0 = cycles();
    pa[2] += c0 - pa[15];
  }
  // ---- stage B: the gates and, speculatively (the GDN leaves h alone on most steps), the MLP
  // (the gate flags were cleared in the previous layer's stage C2)
  if (fly) units<BF, E4, true>(gt, r1, ru, r);
  else units<BF, E4, false>(gt, r1, ru, r);
  gate_compute<BF, E4>(k, gt, gl, r);
  sp_arrive(1);
  lds_barrier();
  sp_depart(1);
  if (k.prof && t == 0) {
    const uint64_t c1 = cycles();
    pa[3] += c1 - c0;
    c0 = c1;
  }
  if (flags[F_ANY]) {
    if (!gdn_event<BF, E4>(p, L, gt, seq, ha, hb)) return false;
    if (flags[F_OUT]) {  // h may have changed: the MLP again, on the new h
      if (k.prof && t == 0) pa[18] += 1;  // (the MLP redos)
      ss = hidden_ss<BF>(ha, hb);
      const float r2 = norm_r(ss, H, hd.eps);
      stage_a<BF, E4>(k, r1, ha, hb, r2, L, step, false, fly);
      lds_barrier();
      if (fly) units<BF, E4, true>(gt, r1, ru, r2);
      else units<BF, E4, false>(gt, r1, ru, r2);
      lds_barrier();
    }
    if (k.prof && t == 0) {
      const uint64_t c1 = cycles();
      pa[4] += c1 - c0;
      pa[16] += 1;
      c0 = c1;
    }
    sp_skip();
  }
  // the next layer's RA and unit passes into the registers this layer's have left
  const uint8_t* ptt_next = lnext->ptt;
  const uint32_t nwords = wave_words(lnext);
  r1 = fetch_words<RG::RAA, RG::RAN>(ptt_next);
  ru = fetch_words<RG::RUA, RG::RUN>(ptt_next, (int)(nwords & 15u));
  // ---- stage C1: down_proj by residual row (units in the model's order) into dsum
  down_rows<BF, E4>(gt, rdw);
  sp_arrive(2);
  lds_barrier();
  sp_depart(2);
  if (k.prof && t == 0) {
    const uint64_t c1 = cycles();
    pa[5] += c1 - c0;
    c0 = c1;
  }
  rdw = fetch_words<RG::RBA, RG::RBN>(ptt_next, (int)(nwords >> 4));
  // ---- stage C2: the residual add on the thread's rows (:791), the LDS copy, and this
  // thread's terms of the next sum of squares (rows past H stay +0)
  {
    const v4f* d4 = reinterpret_cast<const v4f*>(smem + L_DSUM);
    const v4f da = d4[t], db = d4[NT + t];
    const v4f ra = rd4<BF>(da), rb = rd4<BF>(db);
    ha = rd4<BF>(v4f{ha.x + ra.x, ha.y + ra.y, ha.z + ra.z, ha.w + ra.w});
    hb = rd4<BF>(v4f{hb.x + rb.x, hb.y + rb.y, hb.z + rb.z, hb.w + rb.w});
    v4f* h4 = reinterpret_cast<v4f*>(smem + L_H);
    h4[t] = ha;
    h4[NT + t] = hb;
    clear_gate_flags(k);  // for the next layer's gates (this layer's flags are read by now)
    sum512_begin(sq_terms<BF>(ha, hb), LF(L_WSUM) + 8 * par, 3);
  }
  if (k.prof && t == 0) {
    const uint64_t c1 = cycles();
    pa[1] += c1 - c0;
    pa[15] = c1;
  }
  return true;
}

// the residual rows of this thread to the trace (a test aid)
__device__ __forceinline__ void trace_rows(float* tr, int H, const v4f& ha, const v4f& hb) {
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if (4 * t + k < H) tr[4 * t + k] = ha[k];
    if (2048 + 4 * t + k < H) tr[2048 + 4 * t + k] = hb[k];
  }
}

// ---------------------------------------------------------------------------------------------
template <bool BF, bool E4, bool TR>
__device__ void run_chain(const lxm_params& pg) {
  using RG = Regions<E4>;
  const int t = threadIdx.x;
  // the parameter block in LDS: read there at every layer, it costs an LDS read, where the
  // compiler would reload it from global memory through the scalar cache (it does not keep the
  // block in scalar registers across the layer loop)
  static_assert(sizeof(lxm_params) <= 512 && sizeof(lxm_params) % 4 == 0, "params in LDS");
  for (int k = t; k < (int)(sizeof(lxm_params) / 4); k += NT)
    reinterpret_cast<uint32_t*>(smem + L_PARAMS)[k] = gp(reinterpret_cast<const uint32_t*>(&pg))[k];
  __syncthreads();
  const lxm_params& p = *reinterpret_cast<const lxm_params*>(smem + L_PARAMS);
  const ChainK k{p.hidden, p.n_layers, p.nk, p.nv, p.nv / p.nk, p.ring, p.rring, p.prof != nullptr};
  const int H = k.H;
  int* flags = LI(L_FLAGS);
  float* h = LF(L_H);
  float* hist = LF(L_HIST);
  LtEnt* lt = reinterpret_cast<LtEnt*>(smem + L_LT);
  // every LDS word starts finite (zero): gathers may read slots no table names
  for (int k = t; k < L_CHAIN_END / 16; k += NT)
    if (k < L_PARAMS / 16 || k >= L_GATES / 16) reinterpret_cast<v4u*>(smem)[k] = v4u{0, 0, 0, 0};
  __syncthreads();
  // the gate section, resident for the launch (the packer pads it to whole 16-byte words)
  {
    const GAS v4u* src = gp(reinterpret_cast<const v4u*>(p.gates));
    v4u* dst = reinterpret_cast<v4u*>(smem + L_GATES);
    for (int k = t; k < p.gate_bytes / 16; k += NT) dst[k] = src[k];
  }
  const int64_t gsec = p.gates - p.blob;
  for (int L = t; L < p.n_layers; L += NT) {
    const lxm_layer ly = ldg(p.layers + L);
    lt[L].ptt = p.blob + ly.ptt;
    lt[L].goff = (int32_t)(ly.gate - gsec);
    *reinterpret_cast<int64_t*>(lt[L].words) = ly.pt_words;
  }
  __syncthreads();
  // the live query/key channels' windows from the conv state (positions 1..3); each decay's
  // -exp(A_log), a constant of its value head, formed once here in the LDS copy (the gates read
  // it in A_log's place: the same cr_exp a step would evaluate)
  for (int L = 0; L < p.n_layers; L++) {
    uint8_t* gt = smem + L_GATES + lt[L].goff;
    const lxm_gate& hd = *reinterpret_cast<const lxm_gate*>(gt);
    const lxm_qkc* qk = reinterpret_cast<const lxm_qkc*>(gt + hd.qk);
    for (int j = t; j < hd.n_qk; j += NT)
      for (int s = 0; s < 3; s++)
        hist[3 * (hd.qk_base + j) + s] = conv_at<BF>(p.conv[L], (int64_t)qk[j].chan * 4 + 1 + s);
    lxm_dec* dec = reinterpret_cast<lxm_dec*>(gt + hd.dec);
    for (int j = t; j < hd.n_dec; j += NT) dec[j].A_log = -cr_exp(dec[j].A_log);
  }
  uint64_t* pa = reinterpret_cast<uint64_t*>(smem + L_PROF);
  if (t < 32) pa[t] = 0;
  clear_gate_flags(k);
  __syncthreads();
  // the first layer's tables; then always one layer ahead
  typename RG::RA r1 = fetch_words<RG::RAA, RG::RAN>(lt[0].ptt);
  typename RG::RU ru = fetch_words<RG::RUA, RG::RUN>(lt[0].ptt, (int)(wave_words(lt) & 15u));
  typename RG::RB rdw = fetch_words<RG::RBA, RG::RBN>(lt[0].ptt, (int)(wave_words(lt) >> 4));
  // the final norm's weights of this thread's rows (padded to MAXH)
  const v4f wfa = *reinterpret_cast<const v4f*>(p.w1_final + 4 * t);
  const v4f wfb = *reinterpret_cast<const v4f*>(p.w1_final + 2048 + 4 * t);
  int tok = p.forced[0];
  uint32_t seq = 0;
  const uint32_t nh = (uint32_t)(p.n_blocks - 1);
  int par = 0;
  for (int i = 0; i < p.n_tokens; i++) {
    if (tok < 0 || tok >= p.vocab) tok = 0;  // the host checks forced tokens; preds are in range
    if (t == 0 && p.inputs) p.inputs[i] = tok;
    if (k.prof && t == 0) pa[15] = cycles();
    // the input's embedding row (the rows past it are +0 already, and stay so)
    for (int c = t; c < H; c += NT) h[c] = 0.0f;
    lds_barrier();
    {
      const int64_t a = p.emb_ptr[tok], b = p.emb_ptr[tok + 1];
      for (int64_t e = a + t; e < b; e += NT) {
        int col;
        float w;
        Ent<E4>::gat(reinterpret_cast<const uint8_t*>(p.emb_ent), e, col, w);
        *reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(h) + (col & OFF_MASK)) = w;
      }
    }
    lds_barrier();
    v4f ha = reinterpret_cast<const v4f*>(h)[t], hb = reinterpret_cast<const v4f*>(h)[NT + t];
    float ss = hidden_ss<BF>(ha, hb);
    if (k.prof && t == 0) {
      const uint64_t c = cycles();
      pa[0] += c - pa[15];
      pa[15] = c;
    }
    sp_skip();
    for (int L = 0; L < k.nl; L++) {
      const int Ln = L + 1 < k.nl ? L + 1 : 0;
      if (!layer<BF, E4>(p, k, L, i, ss, par, ha, hb, r1, ru, rdw, lt + Ln, seq)) return;
      if constexpr (TR) trace_rows(p.trace + ((size_t)i * k.nl + L) * H, H, ha, hb);
      ss = sum512_take(LF(L_WSUM) + 8 * par);
      par ^= 1;
    }
    // the final norm (lx/lx/hf.py:179-184: model.norm then the tied head), to the helpers
    {
      const float r = norm_r(ss, H, p.rms_eps);
      st4_rlx(p.hn, 4 * t, norm4<BF>(ha, r, wfa));
      st4_rlx(p.hn, 2048 + 4 * t, norm4<BF>(hb, r, wfb));
    }
    drain();
    __syncthreads();
    if (k.prof && t == 0) {
      const uint64_t c = cycles();
      pa[6] += c - pa[15];
      pa[15] = c;
    }
    seq++;
    if (t < NGRP) st_rlx(p.sync + S_EV + 32 * t, seq << 8);
    {  // every helper's stamped key, then the first maximum
      unsigned long long best = 0;
      const bool ok = wait_keys(p.sync, (int)nh, seq & KEY_STAMP, p.err, 1,
                                reinterpret_cast<unsigned long long*>(flags + F_KEYW), &best);
      if (t == 0) {
        int pred = 0;
        if (ok) {
          pred = argmax_idx19(best);
          p.preds[i] = pred;
        }
        flags[F_OK] = ok;
        flags[F_TOK] = pred;
        if (k.prof) {
          const uint64_t c = cycles();
          pa[7] += c - pa[15];
          pa[15] = c;
          pa[17] += 1;
        }
      }
    }
    __syncthreads();
    if (!flags[F_OK]) return;
    tok = i + 1 < p.n_forced ? p.forced[i + 1] : flags[F_TOK];
  }
  if (k.prof && t < 32) p.prof[t] = pa[t];
#ifdef LXM_SUBPROF
  if (k.prof && t < 16 * SP_NS) p.prof[32 + 4 * p.n_blocks + t] = sp_base()[t];
#endif
  // every ring write visible to the other blocks, then let them write the conv windows
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (t == 0) __hip_atomic_store(gp(p.sync + S_DONE), 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// The helpers.

// HEAD: this helper's vocabulary rows against the final normed residual; its best key, stamped
// with the event's low bits, into its own slot (the chain reads every slot).
// The dense head columns' tables in a helper's LDS (after its rows' entries): the rows' code
// words, a byte per hidden column (how many dense columns lie below it), the dense columns, their
// inputs at the current event, their 4-value tables.
struct HeadDense {
  const unsigned long long* code;
  const uint8_t* rank;
  const int32_t* dcol;
  float* xd;
  const float* tab;
};
__host__ __device__ inline int a16(int64_t n) { return (int)((n + 15) & ~(int64_t)15); }
__device__ inline HeadDense head_dense(uint8_t* base, int nr, int H) {
  uint8_t* rk = base + a16(8 * (int64_t)nr);
  uint8_t* dc = rk + a16(H);
  return {reinterpret_cast<const unsigned long long*>(base), rk,
          reinterpret_cast<const int32_t*>(dc), reinterpret_cast<float*>(dc + 128),
          reinterpret_cast<const float*>(dc + 256)};
}

// One head row with dense columns: its sparse entries (columns outside the dense set, ascending)
// and its dense columns' coded values, merged in ascending column order, from +0.
template <bool BF, bool E4>
__device__ __forceinline__ float dense_row(const uint8_t* lent, int a, int n, const float* hn,
                                           const HeadDense& hd, unsigned long long cw, int nd) {
  float s = 0.0f;
  int j = 0;
  for (int e = 0; e < n; e++) {
    int i;
    float w;
    Ent<E4>::at(lent, a + e, i, w);
    i &= OFF_MASK;
    for (const int nb = hd.rank[i >> 2]; j < nb; j++) {
      const float wd = hd.tab[4 * j + (int)((cw >> (2 * j)) & 3ull)];
      s = wd != 0.0f ? acc<BF>(s, hd.xd[j], wd) : s;
    }
    s = acc<BF>(s, at_b(hn, i), w);
  }
  for (; j < nd; j++) {
    const float wd = hd.tab[4 * j + (int)((cw >> (2 * j)) & 3ull)];
    s = wd != 0.0f ? acc<BF>(s, hd.xd[j], wd) : s;
  }
  return s;
}

template <bool BF, bool E4>
__device__ void head_rows(const lxm_params& p, uint32_t stamp, const int32_t* lptr,
                          const uint8_t* lent, int r0, int nr, uint8_t* hx, const HeadDense& hd) {
  const int t = threadIdx.x, H = p.hidden, nd = p.n_hd;
  float* hn = reinterpret_cast<float*>(hx + HX_X);
  unsigned long long* wk = reinterpret_cast<unsigned long long*>(hx + HX_BS);
  {  // the thread's columns requested together (one round trip, not one per column)
    float v[MAXH / NT];
#pragma unroll
    for (int k = 0; k < MAXH / NT; k++) v[k] = t + k * NT < H ? ld_rlxf(p.hn + t + k * NT) : 0.0f;
#pragma unroll
    for (int k = 0; k < MAXH / NT; k++)
      if (t + k * NT < H) hn[t + k * NT] = v[k];
  }
  __syncthreads();
  unsigned long long best = 0;
  if (nd == 0) {
    for (int k = t; k < nr; k += NT) {
      const float v = rd<BF>(dot<BF, E4, 4, 0>(lent, lptr[k], lptr[k + 1] - lptr[k], hn));
      const unsigned long long key = argmax_key19(v, r0 + k);
      best = key > best ? key : best;
    }
  } else {
    if (t < nd) hd.xd[t] = hn[hd.dcol[t]];
    __syncthreads();
    for (int k = t; k < nr; k += NT) {
      const float v = rd<BF>(dense_row<BF, E4>(lent, lptr[k], lptr[k + 1] - lptr[k], hn, hd,
                                               hd.code[k], nd));
      const unsigned long long key = argmax_key19(v, r0 + k);
      best = key > best ? key : best;
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((t & 63) == 0) wk[t >> 6] = best;
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < NW; w++) best = wk[w] > best ? wk[w] : best;
    __hip_atomic_store(gp(reinterpret_cast<unsigned long long*>(p.sync + S_KEY + 32 * blockIdx.x)),
                       best | stamp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// GDN, first part: value head vh of layer L at this step (torch_recurrent_gated_delta_rule
// :330-380 with l2norm :242-245 in the model dtype, Qwen3_5RMSNormGated :168-184), by the
// head's owner. Writes the head's gated-norm output (zeros when it has none) to p.ybuf.
template <bool BF, bool E4>
__device__ void gdn_head(const lxm_params& p, int L, int step, int vh, bool out, uint32_t seq,
                         uint8_t* hx) {
  const int t = threadIdx.x, H = p.hidden, R = p.nv / p.nk, kh = vh / R;
  const int wv = t >> 6, lane = t & 63;
  float* qd = reinterpret_cast<float*>(hx + HX_QD);
  float* kd = reinterpret_cast<float*>(hx + HX_KD);
  float* qn = reinterpret_cast<float*>(hx + HX_QN);
  float* kn = reinterpret_cast<float*>(hx + HX_KN);
  float* vb = reinterpret_cast<float*>(hx + HX_V);
  float* zb = reinterpret_cast<float*>(hx + HX_Z);
  float* gwl = reinterpret_cast<float*>(hx + HX_GW);
  float* dl = reinterpret_cast<float*>(hx + HX_DL);
  float* bs = reinterpret_cast<float*>(hx + HX_BS);
  int* misc = reinterpret_cast<int*>(hx + HX_MISC);
  unsigned long long* y = p.ybuf + (size_t)vh * VD;  // (stamped with seq)
#ifdef LXM_SUBPROF
  // (the profiling build: wall-clock checkpoints of this step, summed per helper in LDS and
  // written out at the launch's end)
  uint64_t* gpr = p.prof ? reinterpret_cast<uint64_t*>(hx + HX_MISC + 64) : nullptr;
  const uint64_t g0 = wall();
#define GH_MARK(k) \
  if (gpr && t == 0) gpr[k] += wall() - g0
#else
#define GH_MARK(k)
#endif
  const uint32_t tf = ld_rlx(p.mb_task + vh);
  if (tf == 0) {  // the step leaves this head alone: state unchanged, output exactly 0
    if (out && t < VD) st64_rlx(y + t, seq, 0.0f);
    return;
  }
  const float e = ld_rlxf(p.mb_e + vh);
  const bool live = (tf & 1) != 0, dec = (tf & 4) != 0;
  const lxm_layer ly = reinterpret_cast<const lxm_layer*>(hx + HX_LT)[L];
  // the layer's state pointer requested at the start (a global load; it is used after the
  // value channels, on the step's path)
  float* const recL = gp(p.rec)[L];
  // the value channels', z rows' and beta row's descriptors, requested first (they do not
  // depend on the step's data)
  lxm_chan ch{};
  lxm_row zr{}, br{};
  if (live) {
    if (t < VD)
      ch = ldg(reinterpret_cast<const lxm_chan*>(p.blob + ly.chan) + 2 * p.nk * KD + vh * VD + t);
    else if (t < 2 * VD)
      zr = ldg(reinterpret_cast<const lxm_row*>(p.blob + ly.z_row) + vh * VD + t - VD);
    else if (t == 2 * VD)
      br = ldg(reinterpret_cast<const lxm_row*>(p.blob + ly.b_row) + vh);
  }
  const uint8_t* gtab = p.blob + ly.gate;
  const lxm_gate hd = ldg(reinterpret_cast<const lxm_gate*>(gtab));
#ifdef LXM_SUBPROF
  if (gpr && t == 0) {
    gpr[5] += 1;
    if (dec) gpr[7] += 1;
  }
#endif
  // This key head's dense query (wave NW - 2) and key (wave NW - 1), each gathered and then
  // l2-normed in the model dtype by its own wave, D(x * D(rsqrt(D(D(sum D(x*x)) + 1e-6)))), the
  // query scaled by 1/sqrt(256) in fp32 (:352-353), while waves 0-4 form the value channels, the
  // z rows and beta below. Without a live query or key both stay 0.
  if (wv >= NW - 2) {
    const bool isk = wv == NW - 1;
    float* x = isk ? kd : qd;
    float* o = isk ? kn : qn;
    int n = 0;
    if (live) {
      for (int i = lane; i < KD; i += 64) x[i] = 0.0f;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const lxm_qkc* qk = reinterpret_cast<const lxm_qkc*>(gtab + hd.qk);
      for (int j = lane; j < hd.n_qk; j += 64) {
        const int sl = gp(&qk[j].slot)[0];
        if ((sl >> 9) == kh && ((sl & 256) != 0) == isk) x[sl & 255] = ld_rlxf(p.mb_qk + j);
      }
      // (one wave's LDS accesses run in order: its reads below see its writes above)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      float s = 0.0f;
      for (int i = lane; i < KD; i += 64) s = s + rd<BF>(x[i] * x[i]);
      s = rd<BF>(sum64(s));
      const float inv = rd<BF>(rsqrt_(rd<BF>(s + 1e-6f)));
      for (int b = 0; b < KD; b += 64) {
        float v = rd<BF>(x[b + lane] * inv);
        if (!isk) v = v * 0.0625f;
        o[b + lane] = v;
        n += __popcll(__ballot(v != 0.0f));
      }
    } else {
      for (int b = 0; b < KD; b += 64) o[b + lane] = 0.0f;
    }
    if (lane == 0) misc[isk ? 1 : 0] = n;
  }
  GH_MARK(0);
  // the value channels' conv outputs (the window's earlier inputs from the ring, or from the
  // conv state before this launch), the in_proj_z rows and beta = sigmoid(b) (:497)
  if (live) {
    const uint8_t* qent = p.blob + ly.qkv_ent;
    const uint8_t* w1in = p.blob + ly.w1_in;
    const float* h0 = ring_at(p, step, L);
    const float r0 = ld_rlxf(rr_at(p, step, L));
    if (t < VD) {
      // window k = 3 - s holds step - s's input: from the ring (one pass over the channel's
      // entries for every such step), or from the conv state before this launch
      const int chan = 2 * p.nk * KD + vh * VD + t;
      const float* hs[4];
      float rs[4], win[4], sm[4];
      bool on[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int s = 3 - k;
        on[k] = s == 0 || (ch.taps[k] != 0.0f && step - s >= 0);
        hs[k] = ring_at(p, step - s, L);
        rs[k] = r0;
        win[k] = 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 3; k++) {
        const int s = 3 - k;
        if (on[k]) rs[k] = ld_rlxf(rr_at(p, step - s, L));
        else if (ch.taps[k] != 0.0f) win[k] = conv_at<BF>(p.conv[L], (int64_t)chan * 4 + 4 - (s - step));
      }
      rdot4<BF, E4>(qent, ch.start, ch.len, hs, rs, on, w1in, sm);
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (on[k]) win[k] = rd<BF>(sm[k]);
      float yv = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (ch.taps[k] != 0.0f) yv = yv + ch.taps[k] * win[k];
      vb[t] = silu_rd<BF>(rd<BF>(yv));  // (bf16: the fast exact path, as the chain's units)
    } else if (t < 2 * VD) {
      const int j = t - VD;
      // (silu of the gate, for the gated norm: formed here, beside the value channels' longer
      // windows, rather than on the output's path)
      // (and the gated norm's weight into LDS: not a global load on the output's path)
      const float w = gp(reinterpret_cast<const float*>(p.blob + ly.gnorm))[j];
      zb[j] = silu(rd<BF>(rdot<BF, E4, true>(p.blob + ly.z_ent, zr.start, zr.len, h0, r0, w1in)));
      gwl[j] = w;
    } else if (t == 2 * VD) {
      const float b = rd<BF>(rdot<BF, E4, true>(p.blob + ly.b_ent, br.start, br.len, h0, r0, w1in));
      misc[2] = (int)__float_as_uint(rd<BF>(sigmoid(b)));
    }
  }
  __syncthreads();
  GH_MARK(1);
  const int nq = misc[0], nk = misc[1];
  const float beta = __uint_as_float((uint32_t)misc[2]);
  // The state tile: thread (cg, rb) holds columns 4cg..4cg+3 of rows 16rb..16rb+15, i.e. one
  // of ATen's 16-row cascade blocks (torch .sum(-2) on the CPU: blocks of 16 rows, each from +0
  // in order, the block sums from +0 in order; only rows with a nonzero factor add terms). Only
  // those rows are read: the whole tile (128 KB) streamed into one CU was measured slower.
  {
    const int cg = t & 31, rb = t >> 5;
    GAS v4f* S4 = gp(reinterpret_cast<v4f*>(recL + (size_t)vh * KD * VD));
    // (the block's rows with a nonzero key factor and with a nonzero query factor, as masks
    // from 16-byte LDS reads, so that the rows' loads are issued back to back and the loops
    // below branch on registers; each loop reads its factors four at a time)
    const v4f* kn4 = reinterpret_cast<const v4f*>(kn + rb * 16);
    const v4f* qn4 = reinterpret_cast<const v4f*>(qn + rb * 16);
    uint32_t km = 0, qm = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const v4f a = kn4[q], b = qn4[q];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        km |= (uint32_t)(a[c] != 0.0f) << (4 * q + c);
        qm |= (uint32_t)(b[c] != 0.0f) << (4 * q + c);
      }
    }
    const uint32_t need = dec ? 0xffffu : (km | qm);
    v4f s[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = rb * 16 + i;
      s[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if ((need >> i) & 1) s[i] = S4[r * (VD / 4) + cg];
    }
    if (dec) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        s[i].x = s[i].x * e;
        s[i].y = s[i].y * e;
        s[i].z = s[i].z * e;
        s[i].w = s[i].w * e;
      }
    }
    if (nk > 0) {
      v4f a = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      v4f kf[4];
#pragma unroll
      for (int q = 0; q < 4; q++) kf[q] = kn4[q];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float f = kf[i >> 2][i & 3];
        if ((km >> i) & 1) {
          a.x = a.x + s[i].x * f;
          a.y = a.y + s[i].y * f;
          a.z = a.z + s[i].z * f;
          a.w = a.w + s[i].w * f;
        }
      }
      reinterpret_cast<v4f*>(bs + rb * VD)[cg] = a;
      __syncthreads();
      if (t < VD) {
        float kv = 0.0f;
#pragma unroll
        for (int b = 0; b < 16; b++) kv = kv + bs[b * VD + t];
        dl[t] = (vb[t] - kv) * beta;
      }
      __syncthreads();
      const v4f d = reinterpret_cast<const v4f*>(dl)[cg];
#pragma unroll
      for (int q = 0; q < 4; q++) kf[q] = kn4[q];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float f = kf[i >> 2][i & 3];
        if ((km >> i) & 1) {
          s[i].x = s[i].x + f * d.x;
          s[i].y = s[i].y + f * d.y;
          s[i].z = s[i].z + f * d.z;
          s[i].w = s[i].w + f * d.w;
        }
      }
    }
    GH_MARK(2);
    if (nq > 0) {
      v4f a = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      v4f qf[4];
#pragma unroll
      for (int q = 0; q < 4; q++) qf[q] = qn4[q];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float f = qf[i >> 2][i & 3];
        if ((qm >> i) & 1) {
          a.x = a.x + s[i].x * f;
          a.y = a.y + s[i].y * f;
          a.z = a.z + s[i].z * f;
          a.w = a.w + s[i].w * f;
        }
      }
      __syncthreads();  // the kv sums above have read bs
      reinterpret_cast<v4f*>(bs + rb * VD)[cg] = a;
      __syncthreads();
      // (a live query makes the event's output live, so out holds here.) One wave forms o for
      // dims lane and lane + 64 (the block sums in order), then the gated norm on this value
      // head, gate z: y = D(D(w * D(o * r)) * silu(z)), issued before any wave stores the
      // state's rows, so that the output does not queue behind them in the CU's memory pipeline
      if (wv == 0) {
        float ov[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          float o = 0.0f;
#pragma unroll
          for (int b = 0; b < 16; b++) o = o + bs[b * VD + lane + 64 * h];
          ov[h] = rd<BF>(o);
        }
        float sq = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) sq = sq + ov[h] * ov[h];
        sq = sum64(sq);
        const float rr = rsqrt_(sq / (float)VD + hd.geps);
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int j = lane + 64 * h;
          const float t1 = rd<BF>(ov[h] * rr);
          const float t2 = rd<BF>(gwl[j] * t1);
          st64_rlx(y + j, seq, rd<BF>(t2 * zb[j]));
        }
      }
      GH_MARK(4);
      __syncthreads();
    } else if (out) {  // no live query: o = 0, and so is every term the head gives out_proj
      if (wv == 0)
        for (int j = lane; j < VD; j += 64) st64_rlx(y + j, seq, 0.0f);
      GH_MARK(4);
      __syncthreads();
    }
    // the state's written rows (each thread stores the blocks it alone reads at the next step,
    // so its own later loads see them; a drain before the head's completion stamp covers them
    // where the chain waits for the states)
    const uint32_t wrote = dec ? 0xffffu : km;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = rb * 16 + i;
      if ((wrote >> i) & 1) S4[r * (VD / 4) + cg] = s[i];
    }
  }
  GH_MARK(3);
#ifdef LXM_SUBPROF
  if (gpr && t == 0 && dec) gpr[6] += wall() - g0;
#endif
}
#undef GH_MARK

// GDN, second part: out_proj rows ra..rb (all value heads' outputs, ascending dims, from +0),
// rounded once, to p.xo. out_prep reads the rows' static tables into LDS (before the wait for
// the heads' outputs); out_rows then reads the outputs the entries name and sums.
template <bool BF, bool E4>
__device__ int out_prep(const lxm_params& p, int L, int ra, int rb, uint8_t* hx) {
  const int t = threadIdx.x;
  int* op = reinterpret_cast<int*>(hx + HX_OP);
  uint8_t* oe = hx + HX_OE;
  const lxm_layer ly = reinterpret_cast<const lxm_layer*>(hx + HX_LT)[L];
  const GAS int32_t* gptr = gp(reinterpret_cast<const int32_t*>(p.blob + ly.out_ptr));
  const int e0 = gptr[ra], ne = gptr[rb] - e0;  // the packer keeps ne <= LXM_OUT_MAX
  if (t <= rb - ra) op[t] = gptr[ra + t] - e0;
  for (int k = t; k < ne; k += NT) {
    int d;
    float w;
    Ent<E4>::gat(p.blob + ly.out_ent, e0 + k, d, w);
    if constexpr (E4) reinterpret_cast<uint32_t*>(oe)[k] = (uint32_t)d | (__float_as_uint(w) & 0xffff0000u);
    else reinterpret_cast<uint2*>(oe)[k] = make_uint2((uint32_t)d, __float_as_uint(w));
  }
  return ne;
}
template <bool BF, bool E4>
__device__ bool out_rows(const lxm_params& p, int ra, int rb, int ne, uint32_t seq, uint8_t* hx) {
  const int t = threadIdx.x;
  int* op = reinterpret_cast<int*>(hx + HX_OP);
  uint8_t* oe = hx + HX_OE;
  float* oy = reinterpret_cast<float*>(hx + HX_OY);
  int* misc = reinterpret_cast<int*>(hx + HX_MISC);
  static_assert(LXM_OUT_MAX <= 2 * NT, "two entries per thread");
  {  // the head outputs the entries name, once every one carries this event's stamp
    int idx[2];
    float yv[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int k = t + i * NT;
      idx[i] = -1;
      if (k < ne) {
        int d;
        float w;
        Ent<E4>::at(oe, k, d, w);
        idx[i] = d;
      }
    }
    if (!wait_words<2>(p.ybuf, idx, seq, p.err, 5, yv)) return false;
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (t + i * NT < ne) oy[t + i * NT] = yv[i];
  }
  lds_barrier();
  if (t < rb - ra) {
    // the row's entries in order, four at a time (slots past the row weigh 0; oy is finite)
    const int a = op[t], n = op[t + 1] - a;
    float s = 0.0f;
    for (int k0 = 0; k0 < n; k0 += 4) {
      float w[4], x[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int d;
        Ent<E4>::at(oe, a + k0 + j, d, w[j]);
        w[j] = k0 + j < n ? w[j] : 0.0f;
        x[j] = oy[a + k0 + j];
      }
#pragma unroll
      for (int j = 0; j < 4; j++) s = acc<BF>(s, x[j], w[j]);
    }
    st_rlxf(p.xo + ra + t, rd<BF>(s));
  }
  return true;
}

template <bool BF, bool E4>
__device__ void run_helper(const lxm_params& pg) {
  uint8_t* lds = smem;
  const int t = threadIdx.x, b = blockIdx.x;
  const int r0 = pg.head_rows[b], r1 = pg.head_rows[b + 1], nr = r1 - r0;
  const int64_t e0 = pg.head_ptr[r0], ne = pg.head_ptr[r1] - e0;
  // the scratch regions first (constant offsets: the head's normed input at 0), the head
  // tables after them
  uint8_t* hx = lds;
  int32_t* lptr = reinterpret_cast<int32_t*>(lds + HX_END);
  uint8_t* lent = lds + HX_END + (((size_t)(nr + 1) * 4 + 15) & ~(size_t)15);
  int* misc = reinterpret_cast<int*>(hx + HX_MISC);
  // every LDS word starts finite (zero): gathers may read slots no table names
  for (int k = t; k < (HX_END + pg.head_lds + 256) / 16; k += NT)
    reinterpret_cast<v4u*>(lds)[k] = v4u{0, 0, 0, 0};
  __syncthreads();
  // the parameter block into LDS: the event path reads its pointers by ds_reads, not by flat
  // loads from global memory (which would also wait on the vector memory counter)
  static_assert(sizeof(lxm_params) <= 512 && sizeof(lxm_params) % 4 == 0, "params in LDS");
  for (int k = t; k < (int)(sizeof(lxm_params) / 4); k += NT)
    reinterpret_cast<uint32_t*>(hx + HX_PARAMS)[k] = gp(reinterpret_cast<const uint32_t*>(&pg))[k];
  __syncthreads();
  const lxm_params& p = *reinterpret_cast<const lxm_params*>(hx + HX_PARAMS);
  const int H = p.hidden, nh = p.n_blocks - 1;
  for (int k = t; k <= nr; k += NT) lptr[k] = (int32_t)(p.head_ptr[r0 + k] - e0);
  // the layer table (an event then reads its layer's offsets from LDS, not from global memory)
  for (int L = t; L < p.n_layers; L += NT)
    reinterpret_cast<lxm_layer*>(hx + HX_LT)[L] = ldg(p.layers + L);
  {
    const uint32_t* src = p.head_ent + e0 * (Ent<E4>::SZ / 4);
    uint32_t* dst = reinterpret_cast<uint32_t*>(lent);
    for (int64_t k = t; k < ne * (Ent<E4>::SZ / 4); k += NT) dst[k] = src[k];
  }
  // the dense head columns' tables (after the entries; none without dense columns)
  uint8_t* ldense = lent + a16(ne * Ent<E4>::SZ);
  const HeadDense hd = head_dense(ldense, nr, H);
  if (p.n_hd > 0) {
    unsigned long long* code = const_cast<unsigned long long*>(hd.code);
    for (int k = t; k < nr; k += NT) code[k] = p.head_code[r0 + k];
    int32_t* dcol = const_cast<int32_t*>(hd.dcol);
    float* tab = const_cast<float*>(hd.tab);
    if (t < p.n_hd) dcol[t] = p.head_dcol[t];
    if (t < 4 * p.n_hd) tab[t] = p.head_dtab[t];
    uint8_t* rank = const_cast<uint8_t*>(hd.rank);
    for (int c = t; c < H; c += NT) {
      int nb = 0;
      for (int j = 0; j < p.n_hd; j++) nb += p.head_dcol[j] < c ? 1 : 0;
      rank[c] = (uint8_t)nb;
    }
  }
  // out_proj rows of this helper: an even split of the residual rows over LXM_OUT_HELPERS
  // helpers (fewer on a smaller grid): the helpers after the value heads' owners when enough
  // remain, so that every out_proj helper reads its tables and polls the heads' outputs while
  // the heads work (an owner would start only after its own head's step); else the first ones
  const int no = nh < LXM_OUT_HELPERS ? nh : LXM_OUT_HELPERS;
  const int rp = (H + no - 1) / no;
  const int ob = b - 1 - (nh - p.nv >= no ? p.nv : 0);  // out_proj index (helper ob of no)
  const bool oh = ob >= 0 && ob < no;
  const int ra = oh && ob * rp < H ? ob * rp : H, rb = ra + rp < H ? ra + rp : H;
  const int vh = b - 1;
  const bool owner = vh < p.nv;
  const int grp = b % NGRP;
  __syncthreads();
  uint64_t pr[4] = {0, 0, 0, 0};
#ifdef LXM_SUBPROF
  if (t < 8) reinterpret_cast<uint64_t*>(hx + HX_MISC + 64)[t] = 0;
  __syncthreads();
#endif
  uint32_t last = 0;
  int step = 0;
  while (step < p.n_tokens) {
    const uint64_t w0 = PROF_ON ? cycles() : 0;
    if (t == 0) {
      uint32_t w = 0;
      misc[5] = spin_ne(p.sync + S_EV + 32 * grp, last, &w, p.err, 2);
      misc[4] = (int)w;
    }
    __syncthreads();
    if (!misc[5]) return;
    const uint32_t w = (uint32_t)misc[4];
    last = w;
    uint64_t w1 = 0;
    if (PROF_ON) {
      w1 = cycles();
      pr[0] += w1 - w0;
    }
    if (!(w & EV_GDN)) {
      // (the head's rows read the parameter block from global memory: the LDS copy, read
      // between the row tables' LDS reads, measured slower there)
      head_rows<BF, E4>(pg, (w >> 8) & KEY_STAMP, lptr, lent, r0, nr, hx, hd);
      if (PROF_ON) pr[1] += cycles() - w1;
      step++;
    } else {
      // (a helper that is neither a value-head owner nor an out_proj helper has nothing to do,
      // and may even miss a GDN event: only HEAD events need every helper)
      const int L = (int)((w >> 2) & 63);
      const bool out = (w & EV_OUT) != 0;
      const uint32_t seq = (w >> 8) & SEQ_MASK;
#ifdef LXM_SUBPROF
      uint64_t* evh = PROF_ON ? reinterpret_cast<uint64_t*>(p.prof) + 32 + 4 * p.n_blocks + SP_EV + 4 + 4 * b
                              : nullptr;
      if (evh && t == 0) evh[0] += wall();
#endif
      if (owner) {
        // (its output goes out as stamped words; without a live query the chain waits for
        // every head's state instead, so the head then drains and stamps it)
        gdn_head<BF, E4>(p, L, step, vh, out, seq, hx);
        if (!out) {
          drain();
          __syncthreads();
          if (t == 0) st_rlx(p.sync + S_OWN + 32 * vh, seq);
        }
#ifdef LXM_SUBPROF
        if (evh && t == 0) evh[1] += wall();
#endif
      }
      uint64_t w2 = 0;
      if (PROF_ON) {
        w2 = cycles();
        pr[2] += w2 - w1;
      }
      if (out && oh && rb > ra) {  // the out_proj helpers: their rows, as stamped words,
        // from every value head's stamped output
        const int ne = out_prep<BF, E4>(p, L, ra, rb, hx);
        if (!out_rows<BF, E4>(p, ra, rb, ne, seq, hx)) return;
#ifdef LXM_SUBPROF
        if (evh && t == 0) evh[2] += wall();
#endif
        drain();
        __syncthreads();
      }
      if (out && oh) {
#ifdef LXM_SUBPROF
        if (evh && t == 0) evh[3] += wall();
#endif
        if (t == 0) st_rlx(p.sync + S_XO + 32 * ob, seq);
      }
      if (PROF_ON) pr[3] += cycles() - w2;
    }
  }
  if (PROF_ON && t == 0)
    for (int k = 0; k < 4; k++) p.prof[32 + 4 * b + k] = pr[k];
#ifdef LXM_SUBPROF
  if (PROF_ON && t == 0)
    for (int k = 0; k < 8; k++)
      reinterpret_cast<uint64_t*>(p.prof)[32 + 8 * p.n_blocks + SP_EV + 4 + 8 * b + k] =
          reinterpret_cast<const uint64_t*>(hx + HX_MISC + 64)[k];
#endif
  if (t == 0) misc[5] = spin_ge(p.sync + S_DONE, 1u, p.err, 3);
  __syncthreads();
  if (misc[5]) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Every conv window once, at the end: [P(n-4), P(n-3), P(n-2), P(n-1)] per channel, P(s) the
// channel's projection of step s's GDN norm output (the ring), or the launch's initial window
// for s < 0 (causal_conv1d_update's state after n steps, :210-211).
template <bool BF, bool E4>
__device__ void write_windows(const lxm_params& p) {
  const int64_t total = (int64_t)p.n_layers * p.n_conv;
  const int64_t per = (total + p.n_blocks - 1) / p.n_blocks;
  const int64_t a = (int64_t)blockIdx.x * per, b = a + per < total ? a + per : total;
  const int n = p.n_tokens;
  for (int64_t g = a + threadIdx.x; g < b; g += NT) {
    const int L = (int)(g / p.n_conv), c = (int)(g % p.n_conv);
    const lxm_layer ly = ldg(p.layers + L);
    const lxm_chan ch = ldg(reinterpret_cast<const lxm_chan*>(p.blob + ly.chan) + c);
    void* cs = p.conv[L];
    float w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int s = n - 4 + k;
      if (s >= 0) {
        // the channel's projection of step s's GDN norm output, formed per entry from the ring
        // (the lanes of a wave can hold two layers' channels: each reads its own layer's row)
        const uint8_t* w1in = p.blob + ly.w1_in;
        w[k] = rd<BF>(rdot<BF, E4, false>(p.blob + ly.qkv_ent, ch.start, ch.len, ring_at(p, s, L),
                                   ld_rlxf(rr_at(p, s, L)), w1in));
      } else {
        w[k] = conv_at<BF>(cs, (int64_t)c * 4 + 4 + s);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) conv_put<BF>(cs, (int64_t)c * 4 + k, w[k]);
  }
}

// TR: the launch records the trace (every layer's residual; a test aid), which the production
// instantiation leaves out of the layer loop
template <bool BF, bool E4, bool TR>
__global__ void __launch_bounds__(NT, 1) lxm_decode(const lxm_params* __restrict__ pp) {
  const lxm_params& p = *pp;
  if (blockIdx.x == 0) run_chain<BF, E4, TR>(p);
  else run_helper<BF, E4>(p);
  __syncthreads();
  if (__hip_atomic_load(gp(p.err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
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
    case 7: r = silu_bf16(bf16r(v)); break;
    default: r = bf16r(v); break;
  }
  y[i] = r;
}

__global__ void __launch_bounds__(NT) k_sum(int kind, const float* x, int n, float* out) {
  __shared__ float wsum[32];
  const float* row = x + (size_t)blockIdx.x * n;
  if (kind == 0) {
    float s = 0.0f;
    for (int part = 0; part < 2; part++)
      for (int j = 0; j < 4; j++) {
        const int i = 2048 * part + 4 * (int)threadIdx.x + j;
        if (i < n) s = s + row[i];
      }
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
// The no-allocation launch's per-device scratch: the parameter block's device copy and every run
// buffer, at fixed 256-byte-aligned offsets (each GPU holds its own copy of the array).
#define SC_PARAMS 0
#define SC_SYNC 512
#define SC_KEYS (SC_SYNC + 4 * LXM_NSYNC)
#define SC_HN (SC_KEYS + 256)
#define SC_XO (SC_HN + 4 * MAXH)
#define SC_MBQK (SC_XO + 4 * MAXH)
#define SC_MBTASK (SC_MBQK + 4 * LXM_MAXQKL)
#define SC_MBE (SC_MBTASK + 4 * LXM_SCRATCH_MAXNV)
#define SC_YBUF (SC_MBE + 4 * LXM_SCRATCH_MAXNV)
#define SC_RRING (SC_YBUF + 8 * LXM_SCRATCH_MAXNV * VD)
#define SC_RING (SC_RRING + 4 * 4 * LXM_SCRATCH_MAXL)
#define SC_END (SC_RING + 4 * 4 * LXM_SCRATCH_MAXL * MAXH)
static_assert(sizeof(lxm_params) <= SC_SYNC, "the parameter block fits its slot");
static_assert(SC_END == LXM_SCRATCH_BYTES, "LXM_SCRATCH_BYTES matches the layout");
static_assert(SC_KEYS % 256 == 0 && SC_RING % 256 == 0 && SC_YBUF % 256 == 0, "aligned slots");

static __device__ __align__(256) uint8_t scratch[LXM_SCRATCH_BYTES];

// the parameter block into the scratch's slot, and the words that must start at zero cleared:
// the sync area, the head keys, the value heads' stamped outputs and the caller's error word
__global__ void __launch_bounds__(256) k_noalloc_prep(lxm_params p, uint8_t* sc) {
  if (threadIdx.x == 0) *reinterpret_cast<lxm_params*>(sc + SC_PARAMS) = p;
  uint32_t* sync = reinterpret_cast<uint32_t*>(sc + SC_SYNC);
  for (int i = threadIdx.x; i < LXM_NSYNC; i += blockDim.x) sync[i] = 0u;
  for (int i = threadIdx.x; i < p.nv * VD; i += blockDim.x) p.ybuf[i] = 0ull;
  if (threadIdx.x < 2) reinterpret_cast<unsigned long long*>(sc + SC_KEYS)[threadIdx.x] = 0ull;
  if (threadIdx.x == 0) *p.err = 0;
}

static const void* decode_fn(const lxm_params* p) {
  const bool tr = p->trace != nullptr;
  return p->bf16 ? (tr ? (const void*)lxm_decode<true, true, true>
                       : (const void*)lxm_decode<true, true, false>)
         : p->e4 ? (tr ? (const void*)lxm_decode<false, true, true>
                       : (const void*)lxm_decode<false, true, false>)
                 : (tr ? (const void*)lxm_decode<false, false, true>
                       : (const void*)lxm_decode<false, false, false>);
}

static hipError_t launch_decode(const void* fn, const lxm_params* pd, int n_blocks, int lds_bytes,
                                hipStream_t stream) {
  void* args[] = {&pd};
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
  if (e != hipSuccess) return e;
  return hipLaunchCooperativeKernel(fn, dim3(n_blocks), dim3(NT), args, (unsigned)lds_bytes, stream);
}

#define SC_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static uint8_t* g_scratch[SC_MAX_DEVICES];  // the scratch's device address, per device

// the current device's scratch address (hipGetSymbolAddress once per device, with it current)
static hipError_t scratch_ptr(uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= SC_MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

extern "C" {

int lxm_lds_base(void) { return L_CHAIN_END; }

int lxm_helper_lds(int head_lds) { return HX_END + head_lds + 256; }  // (reads past the tables)

// the shapes the sync area and the stamped keys hold
static bool launch_ok(const lxm_params* p, int n_blocks) {
  return p && n_blocks >= 2 && n_blocks <= LXM_MAXBLOCKS && p->n_blocks == n_blocks &&
         p->n_tokens >= 0 && (int64_t)p->n_tokens * (p->n_layers + 1) < (int64_t)SEQ_MASK &&
         p->vocab <= LXM_MAXVOCAB && p->nv >= 1 && p->nv <= LXM_SCRATCH_MAXNV && p->nk >= 1 &&
         p->nk <= F_KEYW - F_KH && p->n_hd >= 0 && p->n_hd <= LXM_HEAD_DENSE &&
         (p->n_hd == 0 || (p->head_dcol && p->head_dtab && p->head_code));
}

int lxm_run(const lxm_params* p_host, const lxm_params* p_dev, int n_blocks, int lds_bytes,
            void* stream) {
  if (!launch_ok(p_host, n_blocks)) return (int)hipErrorInvalidValue;
  return (int)launch_decode(decode_fn(p_host), p_dev, n_blocks, lds_bytes, (hipStream_t)stream);
}

int lxm_run_noalloc(const lxm_params* p_host, int n_blocks, int lds_bytes, void* stream) {
  if (!launch_ok(p_host, n_blocks) || !p_host->err || p_host->n_layers < 1 ||
      p_host->n_layers > LXM_SCRATCH_MAXL || p_host->hidden > MAXH)
    return (int)hipErrorInvalidValue;
  uint8_t* sc = nullptr;
  hipError_t e = scratch_ptr(&sc);
  if (e != hipSuccess) return (int)e;
  lxm_params p = *p_host;
  p.ring = reinterpret_cast<float*>(sc + SC_RING);
  p.rring = reinterpret_cast<float*>(sc + SC_RRING);
  p.hn = reinterpret_cast<float*>(sc + SC_HN);
  p.sync = reinterpret_cast<uint32_t*>(sc + SC_SYNC);
  p.keys = reinterpret_cast<unsigned long long*>(sc + SC_KEYS);
  p.mb_task = reinterpret_cast<uint32_t*>(sc + SC_MBTASK);
  p.mb_e = reinterpret_cast<float*>(sc + SC_MBE);
  p.mb_qk = reinterpret_cast<float*>(sc + SC_MBQK);
  p.ybuf = reinterpret_cast<unsigned long long*>(sc + SC_YBUF);
  p.xo = reinterpret_cast<float*>(sc + SC_XO);
  hipLaunchKernelGGL(k_noalloc_prep, dim3(1), dim3(256), 0, (hipStream_t)stream, p, sc);
  e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return (int)launch_decode(decode_fn(&p), reinterpret_cast<const lxm_params*>(sc + SC_PARAMS),
                            n_blocks, lds_bytes, (hipStream_t)stream);
}

int lxm_max_blocks(int lds_bytes) {
  int dev = 0, cus = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipFuncSetAttribute((const void*)lxm_decode<true, true, false>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lxm_decode<true, true, false>, NT, lds_bytes) !=
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
