/* linuxformer on MI355X: the stock forward's chunked delta rule (T > 1), C ABI.
 *
 * torch_chunk_gated_delta_rule (transformers/models/qwen3_5/modeling_qwen3_5.py:249-327, the
 * T > 1 path of Qwen3_5GatedDeltaNet.forward, :517-529; in the reference, fla's
 * chunk_gated_delta_rule called from lx/lx/fast.py:342-345) for one chunk of up to 64 positions
 * of many value heads: the within-chunk WY form (the 64 x 64 key Gram matrix, its unit lower
 * triangular inverse, the decayed key and value combinations) and the chunk's step of the state
 * S <- S exp(g_last) + (k exp(g_last - g))^T v_new, every matrix product on MFMA (fp32 16x16x4).
 * A caller runs the chunks of a sequence in order; the state carries from one call to the next.
 * Results equal the stock chunked form's up to the order of its fp32 sums (no canonical order
 * exists for a matrix product); in the exact regime (one-hot keys, beta in {0, 1}, no decay,
 * dyadic values) they equal the recurrent step bit for bit. All buffers belong to the caller.
 */
#ifndef LXM_CHUNK_H
#define LXM_CHUNK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LXM_CHUNK 64 /* positions per chunk (the stock chunk_size) */

typedef struct lxm_chunk_io {
  const float* q;    /* query of position t, key head kh, dim d: q[t x qk_ts + kh x qk_hs + d];
                        l2-normed and already times 1 / sqrt(256) (the stock scale) */
  const float* k;    /* key, the same layout (l2-normed) */
  const float* v;    /* value of position t, value slot h, dim d: v[t x v_ts + h x 128 + d] */
  const float* beta; /* beta[t x g_ts + h x g_hs] */
  const float* g;    /* log decay g[t x gl_ts + h] (the stock g, before exp) */
  float* S;          /* slot h's state: S + ((h / rl) x rfull + h % rl) x 256 x 128, (256, 128)
                        row-major float32, updated in place */
  float* o;          /* output o[t x o_ts + h x 128 + d] */
  int64_t qk_ts, qk_hs, v_ts, g_ts, g_hs, gl_ts, o_ts;
  int32_t n;       /* positions in this chunk, 1 .. 64 */
  int32_t n_slots; /* value heads (slots) */
  int32_t rl;      /* slots per key head (slot h reads key head h / rl) */
  int32_t rfull;   /* state heads per key head (>= rl) */
  int32_t kl;      /* live key dims, a multiple of 16, <= 128: q and k dims from kl on are
                      zero, and so must be S's rows from kl on (the kernel neither reads nor
                      decays them) */
  int32_t o_bf16;  /* 1: o rounded to bf16 (the stock casts the output to the model dtype) */
} lxm_chunk_io;

/* One chunk of every slot on stream (one workgroup per slot and 32 state columns). q, k, v and S
   are read 16 bytes at a time: each must be 16-byte aligned and qk_ts, qk_hs and v_ts multiples of
   4. Returns a hipError_t (hipErrorInvalidValue for sizes outside the limits above or a misaligned
   pointer or stride). */
int lxm_gdn_chunk(const lxm_chunk_io* io, void* stream);

#ifdef __cplusplus
}
#endif
#endif
