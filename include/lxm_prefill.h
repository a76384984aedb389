/* linuxformer on MI355X: the verified-mode forward of the chip layers, C ABI.
 *
 * lx.fast's Fast (lx/lx/fast.py:252-361 forward/layer, :544-550 head_argmax, :365-540 decode)
 * runs T known tokens through every chip layer at once and takes the head's argmax at every
 * position (session.py:86-116: prediction i is for token i + 1). The reference reaches its
 * kernels from Python (cuBLAS projections, fla's chunk_gated_delta_rule); here the same roles
 * are a few native entry points over caller-owned buffers. Semantics: each position sees
 * exactly the stock decode step (the recurrent delta rule, token by token), so a verified
 * prefill of T tokens leaves the predictions and the states that T forced decode steps leave,
 * bit for bit. (The reference runs fla's chunked rule here and relies on the circuit's values
 * being exact in fp32 for the two to agree, lx/lx/fast.py:17-20; on general values the chunked
 * and recurrent forms round apart, and this library keeps the decode's.) All buffers belong to
 * the caller; the library allocates nothing. Every entry
 * point returns a hipError_t (0 on success).
 *
 * The residual stream lives in HBM as tiles of LXM_PF_TT tokens: element (t, c) of a (T, hidden)
 * stream at ((t / TT) * hidden + c) * TT + t % TT, in the model dtype (bf16 or fp32), so one
 * 16-byte (fp32) or 8-byte (bf16) load gives a column for the tile's tokens.
 */
#ifndef LXM_PREFILL_H
#define LXM_PREFILL_H

#include <stdint.h>

#include "lxm.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LXM_PF_TT 4      /* tokens per residual tile */
#define LXM_PF_MAXKS 16  /* key-head slots of one layer (the layer's live key heads) */
#define LXM_PF_MAXVS 128 /* value-head slots of one layer (live key heads' value heads, decays) */
#define LXM_PF_UPT 4     /* MLP units per thread of the tile kernel (units <= 4 x 512) */
#define LXM_PF_SLICES 8  /* head row slices, one per XCD */

/* One sparse entry of the prefill's tables: off is a byte offset into the vector the row is
   applied to (16 x column for the tile-shaped vectors in LDS, 4 x index for flat ones); w the
   weight. Every table is followed by 4 entries of padding (off 0, w 0). */
typedef struct lxm_pf_ent { int32_t off; float w; } lxm_pf_ent;

typedef struct lxm_pf_unit { int32_t gs, gn, us, un; } lxm_pf_unit;          /* gate, up rows */
typedef struct lxm_pf_drow { int32_t row, start, len, pad; } lxm_pf_drow;    /* down / out rows */
typedef struct lxm_pf_qk {   /* a query/key channel of a live key head with a nonzero tap */
  int32_t chan, kslot, pos;  /* conv channel; key slot; 0..255 query, 256..511 key */
  int32_t start, len, pad[3];
  float taps[4];
} lxm_pf_qk;
typedef struct lxm_pf_dec {  /* a value head whose decay can be nonzero */
  int32_t vslot, start, len; /* in_proj_a row (len 0: a = 0) */
  float dt_bias, A_log;
  int32_t pad[3];
} lxm_pf_dec;
typedef struct lxm_pf_vs {   /* a value-head slot */
  int32_t vh, kslot, dslot, pad; /* kslot -1: no live key head (decay only); dslot -1: no decay */
} lxm_pf_vs;
typedef struct lxm_pf_vc {   /* a value channel of a slot: in_proj_qkv row and conv taps */
  int32_t start, len;
  float taps[4];
} lxm_pf_vc;

/* One layer's tables: byte offsets into the plan's blob; entry starts index the layer's
   lxm_pf_ent array at `ent`. A candidate record (one per position the layer may touch) holds
   {tok, live key slots, 2 x pad}, qn[n_ks][256], kn[n_ks][256], v[n_vs][128] (then the delta
   rule's output o), z[n_vs][128], beta[n_vs], e[n_vs], proc[n_vs] (int), padded to 16 bytes:
   rec_bytes. */
typedef struct lxm_pf_layer {
  int64_t ent;       /* lxm_pf_ent[] */
  int64_t w1_in;     /* float[hidden]: 1 + input_layernorm.weight */
  int64_t w1_post;   /* float[hidden]: 1 + post_attention_layernorm.weight */
  int64_t units;     /* lxm_pf_unit[n_units]: gate/up entries over the MLP norm (16 x column) */
  int64_t drows;     /* lxm_pf_drow[n_drows]: down_proj rows, entries 16 x unit position */
  int64_t qk;        /* lxm_pf_qk[n_qk] */
  int64_t dec;       /* lxm_pf_dec[n_dec] */
  int64_t vs;        /* lxm_pf_vs[n_vs] */
  int64_t vc;        /* lxm_pf_vc[n_vs * 128] (slots with a live key head) */
  int64_t zrow;      /* lxm_row[n_vs * 128]: in_proj_z rows */
  int64_t brow;      /* lxm_row[n_vs]: in_proj_b rows */
  int64_t orows;     /* lxm_pf_drow[n_orows]: out_proj rows, entries 4 x (vslot * 128 + dim) */
  int64_t cc;        /* lxm_row[n_conv]: every conv channel's in_proj_qkv row (the windows) */
  int64_t gnorm;     /* float[128]: the gated norm's weight */
  int64_t entn;      /* float[] parallel to ent: for entries over a norm's output (the MLP units',
                        the query/key channels', the decays'), the norm weight 1 + w of the entry's
                        column, which the tile kernel applies as it gathers; else 0 */
  int32_t n_units, n_drows, n_qk, n_dec, n_ks, n_vs, n_orows, rec_bytes;
  int32_t kh[LXM_PF_MAXKS]; /* key head of each key slot */
  float eps, geps;
  int32_t reach, pad;       /* reach: the earliest conv tap any live query/key channel has (0..3) */
} lxm_pf_layer;

typedef struct lxm_pf_params {
  int32_t hidden, n_layers, nk, nv, n_conv, vocab, bf16;
  int32_t T, ntiles;           /* positions; tiles = ceil(T / LXM_PF_TT) */
  int32_t max_rec;             /* bytes of the largest layer's record */
  float rms_eps;
  int32_t head_long;           /* 1: some head row has more than 4 entries (head_more is read); 0:
                                  none (head_more is not read) */
  const lxm_pf_layer* layers;  /* device, n_layers */
  const lxm_pf_layer* layers_host; /* the same in host memory (the launcher's counts) */
  const uint8_t* blob;         /* device */
  float* const* rec;           /* device array of n_layers pointers: (nv, 256, 128) float */
  void* const* conv;           /* device array of n_layers pointers: (n_conv, 4) model dtype */
  const float* w1_final;       /* (hidden): 1 + the final norm's weight */
  const int64_t* emb_ptr;      /* (vocab + 1): the embedding rows */
  const lxm_pf_ent* emb_ent;   /* off = column, w = value */
  const int32_t* head_slice;   /* (LXM_PF_SLICES + 1): head row ranges, one per XCD */
  const int32_t* head_more;    /* (vocab, 2): the head's rows (columns with nonzero final
                                  weight): row r's first 4 entries at head_ent[4 r ..] (padded);
                                  the rest of a longer row at head_ent[head_more[2 r] ..], a
                                  multiple of 4 entries (padded), head_more[2 r + 1] of them
                                  ((0, 0): none); fewer than 2^31 entries in all */
  const lxm_pf_ent* head_ent;  /* off = 16 x column; padding: off = 16 x hidden, w = 0 */
  const int32_t* tokens;       /* (T): the positions' token ids (embedding) */
  void* h;                     /* (ntiles, hidden, TT) model dtype: the residual stream */
  void* hn;                    /* same layout: the head's normed input */
  float* r1;                   /* (T): each position's input-norm factor of the current layer */
  uint32_t* mask;              /* (T): key slots with a nonzero query/key projection; bit 31 a decay */
  int32_t* cand;               /* (T): the current layer's candidate positions, ascending */
  uint32_t* cmask;             /* (T): their key slots to evaluate */
  int32_t* count;              /* (n_layers + 1): candidates per layer */
  uint8_t* recs;               /* (T x max_rec): candidate records */
  unsigned long long* keys;    /* (T): argmax keys */
  int32_t* preds;              /* (T) */
  int32_t* err;                /* (1): 1 a token id out of range; 2 the head kernel's LDS tile
                                  not at LDS address 0 (a build fault). Sticky: the kernels only
                                  set it, the caller zeroes it before a call (Prefill.embed does).
                                  A bad token's position is embedded as zeros and the layers
                                  still run, so the cache has changed when err reads 1. */
} lxm_pf_params;

/* Fast.forward / Fast.layer (fast.py:252-269): layers [l0, l1) over the T positions of p->h, in
   place, updating the conv windows and recurrent states of those layers. */
int lxm_pf_layers(const lxm_pf_params* p_host, const lxm_pf_params* p_dev, int l0, int l1,
                  void* stream);
/* Fast.head_argmax (fast.py:544-550): the final norm of p->h into p->hn, the tied head over the
   vocabulary rows, the first maximum per position into p->preds (ties to the lower index, NaN
   above everything: torch.argmax). */
int lxm_pf_head(const lxm_pf_params* p_host, const lxm_pf_params* p_dev, void* stream);
/* The embedding rows of p->tokens into p->h (the stock embed_tokens on the chip rows). */
int lxm_pf_embed(const lxm_pf_params* p_host, const lxm_pf_params* p_dev, void* stream);
/* Layout conversion: dir 0 (T, hidden) row-major -> tiles (p->h), dir 1 tiles -> row-major. x is
   in the model dtype. */
int lxm_pf_tiles(const lxm_pf_params* p_host, const void* x, void* y, int dir, void* stream);
/* LDS bytes the tile kernel needs for a model dtype (bf16 != 0), the hidden size and a layer's
   MLP units (it is launched with them; the device allows lxm_max_lds()). */
int lxm_pf_lds(int bf16, int hidden, int n_units);

#ifdef __cplusplus
}
#endif
#endif
