/* linuxformer on MI355X: the chip layers' persistent greedy-decode kernel, C ABI.
 *
 * The drop-in boundary for lx.mega's native library. The reference binds its CUDA library with
 * ctypes (lx/lx/mk_build.py:40-57, lx/lx/mega.py:202) and calls five entry points
 * (lx/csrc/mega.cu:864-893); each has a counterpart here with the same role and error
 * convention (a hipError_t returned as int, 0 on success). All buffers belong to the caller
 * (torch tensors on the Python side); the library allocates nothing.
 *
 * Entry formats in the packed tables ("e4", always for bf16 models, and for fp32 models whose
 * packed values are all exact in bf16): one uint32, index (16 bits) | bf16 value bits << 16,
 * norm weights as their bf16 bits; otherwise two uint32, index then the float's bits, norm
 * weights as 1 + w in fp32.
 */
#ifndef LXM_H
#define LXM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LXM_NT 512          /* threads per workgroup */
#define LXM_MAXH 4096       /* hidden size limit */
#define LXM_KD 256          /* key head dim (the chip's, and the padded text layers') */
#define LXM_VD 128          /* value head dim */
#define LXM_RMAX 8          /* value heads per key head */
#define LXM_MAXU 2048       /* MLP units per layer */
#define LXM_MAXQK 1024      /* live query/key channels, all layers */
#define LXM_MAXQKL 512      /* live query/key channels of one layer */
#define LXM_MAXDEC 512      /* decaying value heads of one layer */
#define LXM_GATE_MAX 65536  /* bytes of the gate section (resident in the chain's LDS) */
#define LXM_NSYNC 19456     /* uint32 words of the sync area (event words, per-writer stamps) */
#define LXM_MAXBLOCKS 256   /* workgroups of a launch, at most (the chain and 255 helpers) */
#define LXM_MAXVOCAB 524288 /* vocabulary rows, at most (a token index fits 19 bits) */
#define LXM_OUT_MAX 1024    /* out_proj entries of the rows one helper workgroup computes */
#define LXM_OUT_HELPERS 64  /* helper workgroups that compute out_proj's rows */
#define LXM_OUT_ROWS 64     /* out_proj rows one of them computes, at most */
#define LXM_HEAD_DENSE 32   /* dense head columns (2-bit coded), at most */

/* The chain workgroup's per-thread table of one layer (packed by linuxformer_amd/chain.py):
   LXM_PT_WORDS x LXM_NT 16-byte words, word j of thread t at (j * LXM_NT + t) * 16, prefetched
   into the thread's registers one layer ahead. Slots (uint32) in a fixed layout: the MLP norm's
   weights of the thread's residual rows (4t..4t+3, 2048+4t..2048+4t+3), meta words, two unit
   passes (gate/up entries interleaved) and down-row passes; see the kernel's PT<E4>. */
#define LXM_PT_WORDS 15

/* One layer's gate tables: the live query/key channels and the decaying value heads, and the
   long units and rows of the chain's per-thread table (resident in the chain's LDS for a launch;
   the helpers read the gate tables from global memory). Offsets are bytes
   from the start of this header, 16-byte aligned. */
typedef struct lxm_gate {
  int32_t n_qk, n_dec, qk_base; /* qk_base: the layer's first q/k history slot */
  int32_t qk;              /* lxm_qkc[n_qk] */
  int32_t dec;             /* lxm_dec[n_dec] */
  int32_t ent;             /* entries of the q/k and decay rows (column byte offsets) */
  int32_t ent_w1;          /* the GDN norm's weight at each entry's column (e4 bf16 bits,
                              else 1 + w as fp32) */
  int32_t size;            /* bytes */
  float eps, geps;
  int32_t long_u, long_r;  /* lxm_longu[n_long_u], lxm_longr[n_long_r] */
  int32_t long_ent;        /* their entries */
  int32_t n_long_u, n_long_r, pad;
} lxm_gate;

/* A unit too long for the chain's register passes: its rows' entries (column byte offsets into
   the MLP norm's output) in the layer's long entries. */
typedef struct lxm_longu { int32_t act, gs, gn, us, un, pad[3]; } lxm_longu;
/* A residual row too long for the down passes: entries are unit byte offsets into act. */
typedef struct lxm_longr { int32_t row, start, len, pad; } lxm_longr;

typedef struct lxm_qkc {   /* a live query/key channel (its conv taps are not all zero) */
  int32_t slot;            /* key head * 512 + (0 query | 256 key) + position */
  int32_t chan;            /* conv channel */
  int32_t start, len;      /* in_proj_qkv row: entries in the gate tables */
  float taps[4];
} lxm_qkc;

typedef struct lxm_dec {   /* a value head whose decay can be nonzero */
  int32_t vh, start, len;  /* in_proj_a row: entries in the gate tables */
  float dt_bias, A_log;
  int32_t pad[3];
} lxm_dec;

typedef struct lxm_chan {  /* a conv channel: in_proj_qkv row (cold entries) and taps */
  int32_t start, len;
  float taps[4];
} lxm_chan;

typedef struct lxm_row { int32_t start, len; } lxm_row;

/* One layer: byte offsets into the packed blob. */
typedef struct lxm_layer {
  int64_t ptt;             /* the chain's per-thread table */
  int64_t pt_words;        /* byte w: the words of its unit region (low nibble) and down region
                              (high nibble) wave w loads (the rest of its slots are unused) */
  int64_t gate;            /* lxm_gate + its tables (inside the gate section) */
  int64_t chan;            /* lxm_chan[n_conv] */
  int64_t qkv_ent;         /* entries (column) */
  int64_t b_row, b_ent;    /* lxm_row[nv], entries (column) */
  int64_t z_row, z_ent;    /* lxm_row[nv * vd], entries (column) */
  int64_t out_ptr;         /* int32[hidden + 1]: out_proj by residual row */
  int64_t out_ent;         /* entries (value dim, all heads: vh * vd + j), ascending per row */
  int64_t gnorm;           /* float[vd] */
  int64_t w1_in;           /* the GDN norm's weights (hidden), w1_post's format */
} lxm_layer;

typedef struct lxm_params {
  int32_t hidden, n_layers, nk, kd, nv, vd, n_conv, vocab, bf16, n_blocks;
  float rms_eps;
  int32_t head_lds;        /* bytes of head tables a helper workgroup stages: its rows' pointers
                              (rows + 1 int32), their entries, and with dense columns (n_hd > 0)
                              the rows' code words (8 bytes each), a column-rank byte per hidden
                              column, the dense columns, their inputs and their tables (768
                              bytes); each part from a 16-byte boundary */
  int32_t e4;              /* the entry format (above) */
  int32_t gate_bytes;      /* bytes of the gate section (every layer's lxm_gate tables) */
  const lxm_layer* layers; /* device, n_layers */
  const uint8_t* blob;     /* device */
  const uint8_t* gates;    /* device: the gate section, inside blob */
  float* const* rec;       /* device array of n_layers pointers: (nv, kd, vd) float */
  void* const* conv;       /* device array of n_layers pointers: (n_conv, 4) model dtype */
  const int64_t* emb_ptr;  /* (vocab + 1): the embedding rows (all columns) */
  const uint32_t* emb_ent;
  const float* w1_final;   /* (hidden): 1 + the final norm's weight */
  const int32_t* head_rows;/* (n_blocks + 1): block b's vocabulary rows */
  const int64_t* head_ptr; /* (vocab + 1): head entries (columns with nonzero final weight) */
  const uint32_t* head_ent;
  const int32_t* forced;
  int32_t n_forced, n_tokens;
  int32_t* preds;          /* (n_tokens) */
  int32_t* inputs;         /* (n_tokens) or null: each step's input as embedded */
  float* trace;            /* (n_tokens, n_layers, hidden) or null: residual after each layer */
  float* ring;             /* (4, n_layers, LXM_MAXH): the last 4 steps' layer inputs */
  float* rring;            /* (4, n_layers): their norm factors r */
  float* hn;               /* (hidden): the head's normed input, chain -> helpers */
  uint32_t* sync;          /* LXM_NSYNC words, zero at launch */
  unsigned long long* keys;/* (2): reserved (the head's keys travel in the sync area) */
  int32_t* err;            /* (1), zero at launch; nonzero: a spin timed out (1..) */
  unsigned long long* prof; /* null, or 32 + 4 x n_blocks counters (phase cycles, see the kernel) */
  uint32_t* mb_task;       /* (nv): a GDN event's task per value head, chain -> helpers */
  float* mb_e;             /* (nv): its decay factor exp(g) */
  float* mb_qk;            /* (LXM_MAXQKL): the layer's live query/key channel values */
  unsigned long long* ybuf; /* (nv, vd), zero at launch: each value head's gated-norm output,
                              a stamped word (the value's fp32 bits low, the GDN event's
                              sequence number high) */
  float* xo;               /* (LXM_MAXH): out_proj's rows, rounded, helpers -> chain */
  int32_t n_qk_total;
  /* Dense head columns (the reference keeps its head's all-nonzero columns as 2-bit codes,
     lx/csrc/mega.cu:96-101, :551-563; lx/lx/mega.py:354-376): n_hd <= LXM_HEAD_DENSE columns,
     head_dcol (ascending hidden indices), each with a table of 4 values head_dtab[4 j + c]
     (bf16-exact for e4 models), and per vocabulary row one word head_code (column j's code at
     bits 2j, 2j + 1). head_ptr / head_ent then hold only the other columns. A row's logit adds
     its terms in ascending column order, the dense ones merged in, from +0 (a code whose value
     is 0 adds nothing). n_hd 0: the pointers may be null. */
  int32_t n_hd;
  const int32_t* head_dcol;
  const float* head_dtab;
  const unsigned long long* head_code;
} lxm_params;

/* mk_run (lx/csrc/mega.cu:867-874): launch the persistent decode, cooperatively, n_blocks
   workgroups of LXM_NT threads with lds_bytes of LDS each, on stream (a hipStream_t). p_host
   is the parameter block in host memory, p_dev the same bytes in device memory (the kernel
   reads its parameters from there). Returns a hipError_t. */
int lxm_run(const lxm_params* p_host, const lxm_params* p_dev, int n_blocks, int lds_bytes,
            void* stream);
/* (A launch numbers its events, at most n_tokens x (n_layers + 1), below 2^24: longer launches
   are refused with hipErrorInvalidValue.) */
/* mk_smem_base (mega.cu:865): LDS bytes the kernel needs besides the staged head tables. */
int lxm_lds_base(void);
/* LDS bytes a helper workgroup needs with head_lds bytes of head tables (the launch's LDS is
   the larger of this and lxm_lds_base()). */
int lxm_helper_lds(int head_lds);
/* mk_max_ctas (mega.cu:876-883): co-resident workgroups at lds_bytes (occupancy x CUs). */
int lxm_max_blocks(int lds_bytes);
/* mk_max_smem (mega.cu:885-890): LDS bytes a workgroup may use. */
int lxm_max_lds(void);
/* mk_last_error (mega.cu:892). */
int lxm_last_error(void);
/* the device's compute units */
int lxm_device_cus(void);

/* Test exports (mk_test.cu:136-160's roles): the kernels' own arithmetic on device arrays.
   fn: 0 exp, 1 silu, 2 sigmoid, 3 softplus, 4 rsqrt, 5 log1p, 6 bf16 rounding, 7 silu of the
   input rounded to bf16, rounded to bf16 (the decode's fast path for bf16 models). */
int lxm_t_elem(int fn, const float* x, float* y, long n, void* stream);
/* kind 0: the 512-lane hidden sum, kind 1: the 64-lane head sum, of each of rows rows of n
   values (x row-major); out (rows). */
int lxm_t_sum(int kind, const float* x, int n, int rows, float* out, void* stream);

/* No counterpart in the reference: lxm_run for callers that cannot allocate device memory (tight
   serving loops, harnesses that forbid hipMalloc). It is a cooperative launch, which is not
   recorded into a captured HIP graph here; no test captures it. The run buffers
   (ring, rring, hn, sync, keys, mb_task, mb_e, mb_qk, ybuf, xo) and the parameter block's device
   copy come from a static array of LXM_SCRATCH_BYTES per GPU (held until the process ends); the
   corresponding fields of *p_host are ignored, everything else (tables, states, forced, preds,
   inputs, trace, prof) and err (zeroed by this call) are the caller's, as for lxm_run. Allocates
   nothing; clears what must start at zero with a kernel on the stream (no memset). Limits:
   n_layers <= LXM_SCRATCH_MAXL, nv <= LXM_SCRATCH_MAXNV (hipErrorInvalidValue beyond them, and
   for a missing err). Calls on one GPU share its array: calls that overlap in time on one GPU
   race, so issue them on one stream (or wait between them). */
#define LXM_SCRATCH_MAXL 64
#define LXM_SCRATCH_MAXNV 256
#define LXM_SCRATCH_BYTES 4572928
int lxm_run_noalloc(const lxm_params* p_host, int n_blocks, int lds_bytes, void* stream);

/* Cross-workgroup synchronisation costs, measured with the decode's own primitives (agent-scope
   words, one polling thread per workgroup, bounded spins): kind 0, a grid barrier over n_blocks
   workgroups on 8 per-XCD counter copies; kind 1, a round trip between workgroup 0 and workgroup
   far (1: another XCD, 8: the same one). n_iter timed operations after a first; *out_us (device)
   gets microseconds per operation, or -1 when a wait timed out (then *err is nonzero). words
   (device, at least 320 uint32) and err (device) must be zero at launch. The role of the
   reference's barrier profile counters (lx/csrc/mega.cu:732-737); a cooperative launch. */
int lxm_t_sync(int kind, int n_iter, int n_blocks, int far, uint32_t* words, int32_t* err,
               float* out_us, void* stream);

#ifdef __cplusplus
}
#endif
#endif
