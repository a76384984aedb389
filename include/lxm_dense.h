/* linuxformer on MI355X: greedy decode of the dense padded text-view stack (benchmark config 4),
 * C ABI.
 *
 * The dense counterpart of lxm_run for stacks whose projections are dense (lx/lx/merge.py:82-120
 * pads the text layers' key heads from 128 to 256 dims and keeps 2 of every 8 value heads): one
 * decode step of every layer and the head per call, each layer as a few HBM-bound row kernels
 * (one wave per row: 64 lanes, each summing one 64th of the row's entries in order from +0, the
 * 64 sums combined by a pairwise tree at offsets 32..1; the oracle's dense order) around the
 * delta rule of the live value heads. The step counter, the fed-back token and the predictions
 * stay on the device, so a caller may capture one call in a graph and replay it per token. The
 * reference has no C entry point for this path (it decodes dense stacks with torch ops,
 * lx/lx/fast.py:365-540): the roles mirror lxm_run's. All buffers belong to the caller.
 *
 * Layouts (bf16 = uint16 bits): a projection set's rows are contiguous, row r's K entries (every
 * live column, ascending) at r x K, interleaved for the wave that reads them: with G = K / 64
 * entries per lane and G >= 8, entries 8q..8q+7 of lane l's G at (q x 64 + l) x 8 within the row
 * (G = 4: plain order). The embedding rows (the head's) likewise. Value heads of a key head kh: kh x 8 + r, live for
 * r < rl (their state and windows change); the other heads and the zero-padded key dims must
 * hold zero state and windows (they then stay zero, as the stock layer leaves them).
 */
#ifndef LXM_DENSE_H
#define LXM_DENSE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lxm_dn_layer {
  const uint16_t* proj;    /* rows: q (nk x kl), k (nk x kl), v (nk x rl x 128), z (nk x rl x 128),
                              b (nk x rl), a (nk x rl); each of hidden entries */
  const uint16_t* conv_qk; /* (2, nk, kl, 4): the live query/key channels' taps */
  const uint16_t* conv_v;  /* (nk, rl, 128, 4) */
  const float* A_log;      /* (nv) */
  const float* dt_bias;    /* (nv) */
  const float* gnorm;      /* (128): the gated norm's weight */
  const float* ln_in;      /* (hidden): input_layernorm's raw weight w (the kernels form 1 + w) */
  const float* ln_post;    /* (hidden) */
  const uint16_t* out;     /* (hidden, nk x rl x 128): out_proj over the live value dims */
  const uint16_t* gate;    /* (inter, hidden) */
  const uint16_t* up;      /* (inter, hidden) */
  const uint16_t* down;    /* (hidden, inter) */
  float* rec;              /* (nv, 256, 128): the layer's recurrent state (in place) */
  uint16_t* conv;          /* (n_conv, 4) bf16: the layer's conv windows (in place) */
} lxm_dn_layer;

typedef struct lxm_dn_params {
  int32_t hidden, n_layers, nk, kl, nv, rl, inter, vocab, n_conv;
  float rms_eps, geps;
  int32_t n_forced, n_steps, pad;
  const lxm_dn_layer* layers; /* device, n_layers */
  const lxm_dn_layer* layers_host; /* the same in host memory (the launcher's weight pointers) */
  const uint16_t* embed;      /* (vocab, hidden): the embedding, tied to the head */
  const float* w_final;       /* (hidden): the final norm's raw weight */
  const int32_t* forced;      /* (n_forced): step i's input is forced[i], else the last prediction */
  int32_t* preds;             /* (n_steps) */
  int32_t* step;              /* (1): the next step's index (advanced by each call) */
  int32_t* tok;               /* (1): the last prediction */
  float* h;                   /* (hidden): the residual */
  float* xn;                  /* (hidden + inter): the MLP's act at +hidden (the norms are formed
                                 inside the kernels that read them) */
  float* P;                   /* (rows of proj): the projections */
  float* on;                  /* (nk x rl x 128): the live heads' delta-rule outputs o (the out_proj
                                 kernel forms the gated norm); nk x rl <= 32 */
  unsigned long long* keys;   /* (2): the head's argmax key (lxm_dn_run alternates between the two
                                 by step parity; both zero before a run) */
  int32_t* err;               /* (1): 1 a forced token out of range, 2 a wait of lxm_dn_run timed out */
  uint32_t* sync;             /* (256): lxm_dn_run's barrier counters, zero before each run */
  unsigned long long* prof;   /* null, or (the sub-phase profiling build only) lxm_dn_run's phase
                                 clock: per workgroup b at prof + 32 b, for each phase k (the
                                 projections, the delta rule, out_proj, SwiGLU, down_proj, the
                                 head) 3 sums over the run of 100 MHz wall-clock ticks: input
                                 staged, rows summed, barrier passed */
} lxm_dn_params;

/* One greedy step (embedding, every layer, the head's first maximum, the token fed back) on
   stream, as five kernels per layer (a caller may capture one call in a graph and replay it).
   p_host: the block in host memory (launch shapes); p_dev: the same bytes on the device.
   Returns a hipError_t. */
int lxm_dn_step(const lxm_dn_params* p_host, const lxm_dn_params* p_dev, void* stream);

/* n greedy steps in one cooperative launch of one workgroup per CU (the same results as n calls
   of lxm_dn_step): the layers' phases are separated by grid barriers; in each workgroup a control
   wave polls them and stages each phase's input in LDS while seven stream waves hold their next
   phase's weight rows in flight. Before the call: sync[0..255] = 0, keys[0..1] =
   0, *err = 0; afterwards *err != 0 reports a bad forced token (1) or a timed-out wait (2). Needs
   nk x rl x 4 <= the device's CUs and (hidden, live value dims, inter) = (2560, 4096, 9216) or
   (256, 512, 512). Returns a hipError_t. */
int lxm_dn_run(const lxm_dn_params* p_host, const lxm_dn_params* p_dev, int n, void* stream);

/* The batched prefill's buffers (device, caller-owned; PB = LXM_DN_PB tokens per batch). */
#define LXM_DN_PB 16
typedef struct lxm_dn_pbuf {
  float* h;    /* (PB, hidden): the batch's residuals */
  uint16_t* xn; /* (PB, hidden) bf16: a norm's output, in the weights' interleaved order */
  float* P;    /* (PB, rows of proj): the projections */
  float* qk;   /* (PB, nk, 2, 256): the normed query (times 1/16) and key */
  float* v;    /* (PB, nk x rl x 128): the values after the conv */
  float* g;    /* (PB, nk x rl, 2): beta and exp(g) */
  float* live; /* (PB, nk, 2): 1 where the query / key has a nonzero element */
  float* o;    /* (PB, nk x rl x 128): the delta rule's outputs */
  uint16_t* ys;  /* (PB, nk x rl x 128) bf16: the gated norm's output, interleaved */
  uint16_t* act; /* (PB, inter) bf16: SwiGLU's output, interleaved */
  float* gl;     /* (PB, nk x rl): the log decays (lxm_dn_prefill_chunked only; else unused) */
} lxm_dn_pbuf;

/* T forced tokens (device int32) through every layer without the head, in batches of LXM_DN_PB:
   the states and windows afterwards are those T calls of lxm_dn_step with these forced tokens
   leave, bit for bit (each weight row is read once per batch; every sum keeps the step's
   order). The stock generate's prefill role (the prompt before the first prediction, here with
   the decode's per-token arithmetic); a caller then steps from the next token. A token out of
   range sets *err = 1 (row 0 is used). Supports (hidden, live value dims, inter) = (2560, 4096,
   9216) or (256, 512, 512). Returns a hipError_t. */
int lxm_dn_prefill(const lxm_dn_params* p_host, const int32_t* tokens, int T,
                   const lxm_dn_pbuf* buf, void* stream);

/* The stock forward's prompt (transformers' T > 1 path, Qwen3_5GatedDeltaNet.forward :517-529:
   torch_chunk_gated_delta_rule, chunks of 64 from the prompt's first token) for T forced tokens
   through every layer without the head: each chunk of LXM_CHUNK (64) tokens goes through every
   layer, its delta rule as one call of lxm_gdn_chunk (include/lxm_chunk.h; MFMA), the row
   kernels on its LXM_DN_PB-token slices. The projections, norms, conv, MLP and out_proj are
   those of lxm_dn_prefill bit for bit on the same inputs; the delta rule's outputs and states
   are the chunked form's (equal to the recurrent step's up to the order of fp32 sums).
   buf's arrays hold LXM_CHUNK tokens (the sizes above with PB = 64) and buf->gl is set. The
   predictions a caller then takes from steps are the stock generate's after a T-token prompt.
   Returns a hipError_t. */
int lxm_dn_prefill_chunked(const lxm_dn_params* p_host, const int32_t* tokens, int T,
                           const lxm_dn_pbuf* buf, void* stream);

#ifdef __cplusplus
}
#endif
#endif
