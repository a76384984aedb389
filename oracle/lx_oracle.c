/* TEST INFRASTRUCTURE ONLY -- the checker, never the product.
 *
 * A CPU restatement, in plain C, of the stock decode of linuxformer's chip layers: the
 * transformers Qwen3_5 decoder layer run token by token in the "chip view"
 * (lx/lx/hf.py:169-176: no positions, no masks), then the tied output head's argmax
 * (lx/lx/hf.py:179-184), with the next input fed back as lx.mega runs it (lx/csrc/mega.cu:852-858,
 * lx/lx/mega.py:529-535). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may
 * load this library; the HIP product path never does.
 *
 * Each step follows, op for op, the stock module it restates (TF = transformers 5.15
 * models/qwen3_5/modeling_qwen3_5.py):
 *   Qwen3_5RMSNorm                TF:720-737   x * rsqrt(mean(x^2) + eps), * (1 + w), to dtype
 *   Qwen3_5GatedDeltaNet.forward  TF:432-543   projections, causal_conv1d_update (TF:199-216),
 *                                              beta = sigmoid(b), g = -exp(A_log) softplus(a + dt)
 *   torch_recurrent_gated_delta_rule TF:330-380 with l2norm (TF:242-245) in the input dtype
 *   Qwen3_5RMSNormGated           TF:168-184
 *   Qwen3_5MLP                    TF:704-717
 *   Qwen3_5DecoderLayer.forward   TF:753-793
 *
 * The rounding contract (what "bit-exact" means between this file and the HIP kernels):
 *   - every elementary op is one IEEE binary32 op, rounded to nearest even, never contracted
 *     into an fma (built with -ffp-contract=off); "D(x)" rounds to the model dtype (bf16: round
 *     to nearest even with NaN -> 0x7fc0, as c10::BFloat16 does; fp32: identity);
 *   - exp, log1p are this file's own functions: evaluated in binary64 (exp: Cody-Waite reduction
 *     by ln 2 and a degree-13 Taylor polynomial; log1p: 2 atanh series) and rounded once to
 *     binary32 (correctly rounded except within ~1e-15 relative of a rounding boundary);
 *     silu(x) = x / (1 + exp(-x)), sigmoid(x) = 1 / (1 + exp(-x)), softplus(x) = x > 20 ? x :
 *     log1p(exp(x)), rsqrt(x) = 1 / sqrt(x) -- the compositions ATen's CPU kernels use;
 *   - dot products and row sums add their terms in ascending index order, from +0; a term
 *     whose factor is an exact zero is skipped (it can change only the sign of a zero sum);
 *   - the delta rule's sums over the state's rows (kv and o, TF:372 and :375, torch's .sum(-2))
 *     follow ATen's CPU cascade for a reduction over a non-contiguous dimension: rows in blocks
 *     of 16, each block summed in order from +0, the block sums added in order from +0 (this
 *     order does not depend on the CPU's vector width, and torch's sum matches it bit for bit);
 *   - sums over a hidden vector (RMSNorm's sum of squares) use 512 lanes: lane l adds
 *     x[4l..4l+3], then x[2048+4l..2048+4l+3], in order from +0; the lanes of each group of 64
 *     are combined by a
 *     pairwise tree at offsets 32, 16, 8, 4, 2, 1 (lane i takes i + off); the 8 group totals by
 *     a tree at offsets 4, 2, 1. Sums over a head (128 or 256 values) use one group of 64 lanes.
 *     Means divide the sum by the count (ATen's CPU mean is sum().div_(n)).
 *   - a matrix marked dense (blocks = 64; the dense padded text-view stack, whose projections a
 *     GPU sums across a wave) sums each row's stored entries (every live column, zeros included;
 *     a multiple of 64) in 64 equal consecutive groups, each in order from +0, and combines the
 *     64 group sums by the pairwise tree at offsets 32, 16, 8, 4, 2, 1. The stock forward's dense
 *     GEMV order (oneDNN, cuBLAS) is a library choice with no canonical form; this one is fixed
 *     here and shared with the dense kernels.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ rounding primitives */

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

static inline float bf16r(float x) {
  uint32_t u = fbits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bitsf(0x7fc00000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bitsf(u & 0xffff0000u);
}

static int g_bf16 = 1; /* model dtype of the current call */
static inline float D(float x) { return g_bf16 ? bf16r(x) : x; }

/* The flush mode (off by default; never the contract the kernels follow): bf16 matrix products
   treat denormal inputs as zero and flush denormal sums to zero, as oneDNN's bf16 GEMM does on
   CPUs with AMX / AVX512-BF16 (the stock forward's F.linear on such hosts). It lets the tests
   show that this flushing is the only difference between the contract and the stock forward. */
static int g_flush = 0;
void ox_set_flush(int on) { g_flush = on; }
static inline int tiny(float x) { return x != 0.0f && fabsf(x) < 0x1p-126f; }

static inline double pow2i(int k) { /* 2^k, -1022 <= k <= 1023 */
  uint64_t u = (uint64_t)(k + 1023) << 52;
  double d; memcpy(&d, &u, 8); return d;
}

/* exp(x) in binary64 for -110 <= x <= 89 (relative error ~5e-16) */
static double exp_d(double x) {
  const double LOG2E = 0x1.71547652b82fep+0;
  const double LN2_HI = 0x1.62e42fee00000p-1, LN2_LO = 0x1.a39ef35793c76p-33;
  double kd = floor(x * LOG2E + 0.5);
  double r = (x - kd * LN2_HI) - kd * LN2_LO;
  double p = 0x1.6124613a86d09p-33;
  p = p * r + 0x1.1eed8eff8d898p-29;
  p = p * r + 0x1.ae64567f544e4p-26;
  p = p * r + 0x1.27e4fb7789f5cp-22;
  p = p * r + 0x1.71de3a556c734p-19;
  p = p * r + 0x1.a01a01a01a01ap-16;
  p = p * r + 0x1.a01a01a01a01ap-13;
  p = p * r + 0x1.6c16c16c16c17p-10;
  p = p * r + 0x1.1111111111111p-7;
  p = p * r + 0x1.5555555555555p-5;
  p = p * r + 0x1.5555555555555p-3;
  p = p * r + 0x1.0000000000000p-1;
  p = p * r + 1.0;
  p = p * r + 1.0;
  return p * pow2i((int)kd);
}

float ox_expf(float x) {
  if (x != x) return x;
  if (x > 89.0f) return INFINITY;
  if (x < -110.0f) return 0.0f;
  return (float)exp_d((double)x);
}

/* log(u) in binary64 for finite u >= 1 */
static double log_d(double u) {
  const double LN2_HI = 0x1.62e42fee00000p-1, LN2_LO = 0x1.a39ef35793c76p-33;
  uint64_t b; memcpy(&b, &u, 8);
  int m = (int)((b >> 52) & 0x7ff) - 1023;
  b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull; /* f in [1, 2) */
  double f; memcpy(&f, &b, 8);
  if (f > 0x1.6a09e667f3bcdp+0) { f = f * 0.5; m += 1; } /* f in [sqrt(1/2), sqrt(2)] */
  double s = (f - 1.0) / (f + 1.0);
  double s2 = s * s;
  double p = 0x1.642c8590b2164p-5;
  p = p * s2 + 0x1.8618618618618p-5;
  p = p * s2 + 0x1.af286bca1af28p-5;
  p = p * s2 + 0x1.e1e1e1e1e1e1ep-5;
  p = p * s2 + 0x1.1111111111111p-4;
  p = p * s2 + 0x1.3b13b13b13b14p-4;
  p = p * s2 + 0x1.745d1745d1746p-4;
  p = p * s2 + 0x1.c71c71c71c71cp-4;
  p = p * s2 + 0x1.2492492492492p-3;
  p = p * s2 + 0x1.999999999999ap-3;
  p = p * s2 + 0x1.5555555555555p-2;
  p = p * s2 + 1.0;
  double lf = (2.0 * s) * p;
  return (double)m * LN2_HI + ((double)m * LN2_LO + lf);
}

/* log1p(y) for y >= 0 (the only arguments softplus gives it) */
float ox_log1pf(float y) {
  if (y != y) return y;
  if (y == INFINITY) return y;
  double yd = (double)y;
  if (yd < 0x1p-29) return (float)(yd - (yd * yd) * 0.5);
  return (float)log_d(1.0 + yd);
}

float ox_silu(float x) { return x / (1.0f + ox_expf(-x)); }
float ox_sigmoid(float x) { return 1.0f / (1.0f + ox_expf(-x)); }
float ox_softplus(float x) { return x > 20.0f ? x : ox_log1pf(ox_expf(x)); }
float ox_rsqrt(float x) { return 1.0f / sqrtf(x); }

/* elementwise exports for the tests: fn 0 exp, 1 silu, 2 sigmoid, 3 softplus, 4 rsqrt,
   5 log1p, 6 bf16 rounding */
void ox_elem(int fn, const float* x, float* y, long n) {
  for (long i = 0; i < n; i++) {
    float v = x[i];
    switch (fn) {
      case 0: y[i] = ox_expf(v); break;
      case 1: y[i] = ox_silu(v); break;
      case 2: y[i] = ox_sigmoid(v); break;
      case 3: y[i] = ox_softplus(v); break;
      case 4: y[i] = ox_rsqrt(v); break;
      case 5: y[i] = ox_log1pf(v); break;
      default: y[i] = bf16r(v); break;
    }
  }
}

/* ------------------------------------------------------------------ canonical sums */

/* the 512-lane sum of n <= 4096 values: lane l adds x[4l .. 4l+3] then x[2048+4l .. 2048+4l+3]
   (those < n) in order from +0; lanes pair within groups of 64 at offsets 32..1, the 8 group
   totals at offsets 4, 2, 1 */
float ox_sum_h(const float* x, int n) {
  float p[512], w[8];
  if (n > 4096) return __builtin_nanf("");
  for (int l = 0; l < 512; l++) {
    float s = 0.0f;
    for (int part = 0; part < 2; part++)
      for (int j = 0; j < 4; j++) {
        const int i = 2048 * part + 4 * l + j;
        if (i < n) s = s + x[i];
      }
    p[l] = s;
  }
  for (int g = 0; g < 8; g++) {
    float* q = p + 64 * g;
    for (int off = 32; off >= 1; off >>= 1)
      for (int i = 0; i < off; i++) q[i] = q[i] + q[i + off];
    w[g] = q[0];
  }
  for (int off = 4; off >= 1; off >>= 1)
    for (int i = 0; i < off; i++) w[i] = w[i] + w[i + off];
  return w[0];
}

/* the 64-lane sum of n values (a head's 128 or 256) */
float ox_sum_64(const float* x, int n) {
  float q[64];
  for (int l = 0; l < 64; l++) {
    float s = 0.0f;
    for (int i = l; i < n; i += 64) s = s + x[i];
    q[l] = s;
  }
  for (int off = 32; off >= 1; off >>= 1)
    for (int i = 0; i < off; i++) q[i] = q[i] + q[i + off];
  return q[0];
}

/* ------------------------------------------------------------------ the model */

typedef struct {
  int hidden, n_layers, nk, kd, nv, vd, conv, inter, vocab, bf16;
  float rms_eps, gated_eps;
} ox_dims;

typedef struct { /* CSR: row r's entries ptr[r] .. ptr[r + 1] - 1, columns ascending */
  int nrows, ncols;
  const int64_t* ptr;
  const int32_t* col;
  const float* val;
  int blocks;      /* 0: each row summed in order; 64: the dense order (entries per row % 64 == 0) */
  int pad;
} ox_csr;

typedef struct {
  ox_csr qkv, z, b, a, out, gate, up, down;
  const float* conv_w;  /* (n_conv, conv) */
  const float* A_log;   /* (nv,) */
  const float* dt_bias; /* (nv,) */
  const float* gnorm;   /* (vd,) */
  const float* ln_in;   /* (hidden,) raw weights w */
  const float* ln_post;
} ox_layer;

typedef struct {
  ox_dims d;
  const ox_layer* layers;
  ox_csr embed;             /* (vocab, hidden): the embedding, also the tied output head */
  const float* final_norm;  /* (hidden,) */
} ox_model;

typedef struct {
  float *xn, *P, *z, *b, *a, *y, *beta, *g, *qn, *kn, *o, *on, *out, *sq, *kv, *delta, *act,
      *gt, *up, *logits;
  int *proc;
} ox_ws;

static void* xalloc(size_t n) { void* p = calloc(n ? n : 1, 1); if (!p) abort(); return p; }

static void ws_init(ox_ws* w, const ox_dims* d) {
  int C = 2 * d->nk * d->kd + d->nv * d->vd;
  w->xn = xalloc(4 * (size_t)d->hidden);
  w->P = xalloc(4 * (size_t)C);
  w->y = xalloc(4 * (size_t)C);
  w->z = xalloc(4 * (size_t)d->nv * d->vd);
  w->b = xalloc(4 * (size_t)d->nv);
  w->a = xalloc(4 * (size_t)d->nv);
  w->beta = xalloc(4 * (size_t)d->nv);
  w->g = xalloc(4 * (size_t)d->nv);
  w->qn = xalloc(4 * (size_t)d->nk * d->kd);
  w->kn = xalloc(4 * (size_t)d->nk * d->kd);
  w->o = xalloc(4 * (size_t)d->nv * d->vd);
  w->on = xalloc(4 * (size_t)d->nv * d->vd);
  w->out = xalloc(4 * (size_t)d->hidden);
  w->sq = xalloc(4 * (size_t)(d->kd > d->vd ? d->kd : d->vd));
  w->kv = xalloc(4 * (size_t)d->vd);
  w->delta = xalloc(4 * (size_t)d->vd);
  w->act = xalloc(4 * (size_t)d->inter);
  w->gt = xalloc(4 * (size_t)d->inter);
  w->up = xalloc(4 * (size_t)d->inter);
  w->logits = xalloc(4 * (size_t)d->vocab);
  w->proc = xalloc(4 * (size_t)d->nv);
}

static void ws_free(ox_ws* w) {
  void* ps[] = {w->xn, w->P, w->y, w->z, w->b, w->a, w->beta, w->g, w->qn, w->kn, w->o, w->on,
                w->out, w->sq, w->kv, w->delta, w->act, w->gt, w->up, w->logits, w->proc};
  for (size_t i = 0; i < sizeof(ps) / sizeof(ps[0]); i++) free(ps[i]);
}

/* sum over row r's entries of x[col] * w (unrounded): ascending columns from +0, or for a dense
   matrix per group of n / 64 consecutive entries, then the group sums' pairwise tree (lane i
   takes i + off) */
static float row_dot(const ox_csr* m, int r, const float* x) {
  if (!m->blocks) {
    float s = 0.0f;
    if (g_flush && g_bf16) {
      for (int64_t e = m->ptr[r]; e < m->ptr[r + 1]; e++) {
        float xv = x[m->col[e]];
        if (xv == 0.0f || tiny(xv)) continue;
        s = s + xv * m->val[e];
        if (tiny(s)) s = copysignf(0.0f, s);
      }
      return s;
    }
    for (int64_t e = m->ptr[r]; e < m->ptr[r + 1]; e++) {
      float xv = x[m->col[e]];
      if (xv == 0.0f) continue;
      s = s + xv * m->val[e];
    }
    return s;
  }
  float p[64] = {0};
  const int64_t e0 = m->ptr[r], n = m->ptr[r + 1] - e0, g = n / 64;
  if (n % 64) abort(); /* the packer keeps every live column of a dense row */
  for (int64_t e = e0; e < e0 + n; e++) {
    float xv = x[m->col[e]];
    if (xv == 0.0f) continue;
    const int b = (int)((e - e0) / g);
    p[b] = p[b] + xv * m->val[e];
  }
  for (int off = 32; off >= 1; off >>= 1)
    for (int i = 0; i < off; i++) p[i] = p[i] + p[i + off];
  return p[0];
}

/* test export: x . w over n terms in a row's order (blocks 0: in order; 64: the dense order) */
float ox_row_dot(int blocks, int n, const float* x, const float* w) {
  int64_t ptr[2] = {0, n};
  int32_t* col = malloc(sizeof(int32_t) * (n ? n : 1));
  if (!col) abort();
  for (int i = 0; i < n; i++) col[i] = i;
  ox_csr m = {1, n, ptr, col, w, blocks, 0};
  float r = row_dot(&m, 0, x);
  free(col);
  return r;
}

/* out[r] = D(row r . x); rows are independent, so they are spread over the host's threads (each
   row's own sum keeps its order) */
static void csr_mv(const ox_csr* m, const float* x, float* out) {
#pragma omp parallel for schedule(static) if (m->nrows >= 2048)
  for (int r = 0; r < m->nrows; r++) out[r] = D(row_dot(m, r, x));
}

/* Qwen3_5RMSNorm(h) (TF:720-737): r = rsqrt(mean(h^2) + eps); xn = D((h * r) * (1 + w)) */
static void rms_norm(const float* h, int H, float eps, const float* w, float* sq, float* xn) {
  for (int i = 0; i < H; i++) sq[i] = h[i] * h[i];
  float ss = ox_sum_h(sq, H);
  float r = ox_rsqrt(ss / (float)H + eps);
  for (int i = 0; i < H; i++) xn[i] = D((h[i] * r) * (1.0f + w[i]));
}

/* sum over rows i of col[i * stride] * f[i] (f[i] != 0 only), in ATen's outer-sum cascade:
   blocks of 16 rows, each from +0 in order, the block sums from +0 in order */
static float row_sum(const float* col, int stride, const float* f, int n) {
  float tot = 0.0f;
  for (int b = 0; b < n; b += 16) {
    float s = 0.0f;
    int any = 0;
    for (int i = b; i < b + 16 && i < n; i++) {
      if (f[i] == 0.0f) continue;
      s = s + col[(size_t)i * stride] * f[i];
      any = 1;
    }
    if (any) tot = tot + s;
  }
  return tot;
}

/* l2norm(x) (TF:242-245) in the model dtype: x * rsqrt(sum(x * x) + 1e-6), each op rounded */
static void l2norm_D(const float* x, int n, float* sq, float* out) {
  for (int i = 0; i < n; i++) sq[i] = D(x[i] * x[i]);
  float s = D(ox_sum_64(sq, n));
  float inv = D(ox_rsqrt(D(s + 1e-6f)));
  for (int i = 0; i < n; i++) out[i] = D(x[i] * inv);
}

/* torch_recurrent_gated_delta_rule (TF:330-380) for one token, use_qk_l2norm_in_kernel: q, k
   (nk, kd) and v (nv, vd) in the model dtype, g (nv) fp32, beta (nv) model dtype, the state S
   (nv, kd, vd) fp32 updated in place; value head vh reads key head vh / (nv / nk) (the stock
   repeat_interleave). Outputs o (nv, vd) in the model dtype into w->o; w->proc[vh] is 0 for a
   head the step leaves alone (exp(g) = 1, q = k = 0: state unchanged, output exactly 0), 1 for a
   decay only, 2 for a head with a live query or key. Returns whether any head had one. */
static int rec_heads(const ox_dims* d, const float* qall, const float* kall, const float* vall,
                     const float* g, const float* betas, float* S, ox_ws* w) {
  const int kd = d->kd, vd = d->vd, nk = d->nk, nv = d->nv, R = nv / nk;
  int any = 0;
  int klive[64];
  for (int kh = 0; kh < nk; kh++) {
    const float* q = qall + (size_t)kh * kd;
    const float* k = kall + (size_t)kh * kd;
    int live = 0;
    for (int i = 0; i < kd; i++) live |= (q[i] != 0.0f) | (k[i] != 0.0f);
    klive[kh] = live;
    float* qn = w->qn + (size_t)kh * kd;
    float* kn = w->kn + (size_t)kh * kd;
    if (live) {
      l2norm_D(q, kd, w->sq, qn);
      l2norm_D(k, kd, w->sq, kn);
      for (int i = 0; i < kd; i++) qn[i] = qn[i] * 0.0625f; /* 1 / sqrt(256) */
    }
  }
  /* value heads are independent: each owns its state tile, output and flag */
#pragma omp parallel for schedule(dynamic) reduction(| : any) if (nv >= 16)
  for (int vh = 0; vh < nv; vh++) {
    const int kh = vh / R, live = klive[kh];
    const float* qn = w->qn + (size_t)kh * kd;
    const float* kn = w->kn + (size_t)kh * kd;
    float* Sv = S + (size_t)vh * kd * vd;
    float* o = w->o + (size_t)vh * vd;
    float delta[256];
    const float e = ox_expf(g[vh]);
    w->proc[vh] = live || e != 1.0f;
    for (int j = 0; j < vd; j++) o[j] = 0.0f;
    if (!w->proc[vh]) continue;
    if (e != 1.0f)
      for (size_t i = 0; i < (size_t)kd * vd; i++) Sv[i] = Sv[i] * e;
    if (!live) continue; /* q = 0: output exactly 0 */
    const float* v = vall + (size_t)vh * vd;
    const float beta = betas[vh];
    for (int j = 0; j < vd; j++) {
      float s = row_sum(Sv + j, vd, kn, kd);
      delta[j] = (v[j] - s) * beta;
    }
    for (int i = 0; i < kd; i++) {
      if (kn[i] == 0.0f) continue;
      for (int j = 0; j < vd; j++) Sv[(size_t)i * vd + j] = Sv[(size_t)i * vd + j] + kn[i] * delta[j];
    }
    for (int j = 0; j < vd; j++) o[j] = D(row_sum(Sv + j, vd, qn, kd));
    w->proc[vh] = 2;
    any = 1;
  }
  return any;
}

/* channels c0 .. c1 - 1 of causal_conv1d_update: each window shifts in P[c]; y[c] is formed
   unless live (non-null) marks the channel's key head idle (channels (c - c0) / per of a key
   head) */
static void conv_channels(const ox_layer* ly, float* cs, ox_ws* w, int c0, int c1,
                          const int* live, int K, int per) {
#pragma omp parallel for schedule(static) if (c1 - c0 >= 2048)
  for (int c = c0; c < c1; c++) {
    float* win = cs + (size_t)c * K;
    if (fbits(w->P[c]) == 0u) { /* a window of +0s stays so and gives +0 (a sum of zeros from
                                   +0); a -0 (a tiny negative rounded) must still shift */
      uint32_t any = 0u;
      for (int i = 0; i < K; i++) any |= fbits(win[i]);
      if (!any) { w->y[c] = 0.0f; continue; }
    }
    for (int i = 0; i + 1 < K; i++) win[i] = win[i + 1];
    win[K - 1] = w->P[c];
    if (live && !live[(c - c0) / per]) { w->y[c] = 0.0f; continue; }
    const float* tw = ly->conv_w + (size_t)c * K;
    float s = 0.0f;
    for (int i = 0; i < K; i++) s = s + tw[i] * win[i];
    const float ds = D(s);
    w->y[c] = D(ds == 0.0f ? ds : ox_silu(ds)); /* silu(+-0) = +-0: skips the exp */
  }
}

/* one chip layer's decode step on the residual h (TF:753-793), updating its conv window cs
   (n_conv, conv) and recurrent state S (nv, kd, vd) in place */
static void layer_step(const ox_model* m, int L, float* h, float* cs, float* S, ox_ws* w,
                       float* hsq) {
  const ox_dims* d = &m->d;
  const ox_layer* ly = &m->layers[L];
  const int H = d->hidden, K = d->conv, kd = d->kd, vd = d->vd, nk = d->nk, nv = d->nv;
  const int C = 2 * nk * kd + nv * vd;

  /* ---- linear attention (TF:432-543) */
  rms_norm(h, H, d->rms_eps, ly->ln_in, hsq, w->xn);
  csr_mv(&ly->qkv, w->xn, w->P);
  csr_mv(&ly->b, w->xn, w->b);
  csr_mv(&ly->a, w->xn, w->a);
  /* causal_conv1d_update (TF:199-216): window <- [window[1:], P]; y = silu(D(sum w_i x_i)).
     Every window shifts; a value channel's output is formed only under a key head whose query
     or key is nonzero (the delta rule reads no other head's values) */
  const int QK = 2 * nk * kd;
  conv_channels(ly, cs, w, 0, QK, NULL, K, kd * (nv / nk));
  int vlive[64];
  for (int kh = 0; kh < nk; kh++) {
    int live = 0;
    for (int i = 0; i < kd; i++)
      live |= (w->y[(size_t)kh * kd + i] != 0.0f) | (w->y[(size_t)(nk + kh) * kd + i] != 0.0f);
    vlive[kh] = live;
  }
  conv_channels(ly, cs, w, QK, C, vlive, K, vd * (nv / nk));
  for (int v = 0; v < nv; v++) {
    w->beta[v] = D(ox_sigmoid(w->b[v]));
    float sp = ox_softplus(w->a[v] + ly->dt_bias[v]);
    w->g[v] = (-ox_expf(ly->A_log[v])) * sp;
  }
  /* the recurrent step per value head (TF:330-380); query and key heads repeat R times */
  int any_proc = rec_heads(d, w->y, w->y + (size_t)nk * kd, w->y + (size_t)2 * nk * kd, w->g,
                           w->beta, S, w);
  for (int vh = 0; vh < nv; vh++) {
    float* on = w->on + (size_t)vh * vd;
    if (w->proc[vh] != 2) {
      for (int j = 0; j < vd; j++) on[j] = 0.0f;
      continue;
    }
    const float* o = w->o + (size_t)vh * vd;
    /* Qwen3_5RMSNormGated (TF:168-184) on this value head, gate z */
    for (int j = 0; j < vd; j++) w->sq[j] = o[j] * o[j];
    float ss = ox_sum_64(w->sq, vd);
    float rr = ox_rsqrt(ss / (float)vd + d->gated_eps);
    float zrow[256];
    for (int j = 0; j < vd; j++) /* in_proj_z rows of this head */
      zrow[j] = D(row_dot(&ly->z, vh * vd + j, w->xn));
    for (int j = 0; j < vd; j++) {
      float t1 = D(o[j] * rr);
      float t2 = D(ly->gnorm[j] * t1);
      on[j] = D(t2 * ox_silu(zrow[j]));
    }
  }
  /* out_proj, then the residual add (all rows: a row with no term adds +0) */
  if (any_proc) {
    csr_mv(&ly->out, w->on, w->out);
  } else {
    for (int i = 0; i < H; i++) w->out[i] = 0.0f;
  }
  for (int i = 0; i < H; i++) h[i] = D(h[i] + w->out[i]);

  /* ---- MLP (TF:704-717) */
  rms_norm(h, H, d->rms_eps, ly->ln_post, hsq, w->xn);
  csr_mv(&ly->gate, w->xn, w->gt);
  csr_mv(&ly->up, w->xn, w->up);
  for (int u = 0; u < d->inter; u++) {
    const float gt = w->gt[u];
    w->act[u] = D(D(gt == 0.0f ? gt : ox_silu(gt)) * w->up[u]); /* silu(+-0) = +-0 */
  }
  csr_mv(&ly->down, w->act, w->out);
  for (int i = 0; i < H; i++) h[i] = D(h[i] + w->out[i]);
}

/* the final norm and the tied head's first maximum (NaN counts as the maximum, as
   torch.argmax takes it) */
static int head_argmax(const ox_model* m, const float* h, ox_ws* w, float* hsq) {
  const ox_dims* d = &m->d;
  rms_norm(h, d->hidden, d->rms_eps, m->final_norm, hsq, w->xn);
  csr_mv(&m->embed, w->xn, w->logits);
  int best = 0;
  float bv = w->logits[0];
  for (int v = 1; v < d->vocab; v++) {
    float x = w->logits[v];
    if (bv != bv) break;
    if (x != x || x > bv) { bv = x; best = v; }
  }
  return best;
}

/* The residual stream of token tok: its embedding row (D values). */
static void embed_row(const ox_model* m, int tok, float* h) {
  const ox_csr* e = &m->embed;
  for (int i = 0; i < m->d.hidden; i++) h[i] = 0.0f;
  for (int64_t k = e->ptr[tok]; k < e->ptr[tok + 1]; k++) h[e->col[k]] = e->val[k];
}

/* n greedy decode steps: step i's input is forced[i] (i < n_forced) or step i - 1's
   prediction (lx/lx/mega.py:529-535). conv (n_layers, n_conv, conv) and rec (n_layers, nv, kd,
   vd) are updated in place. trace (optional, n x n_layers x hidden): the residual after each
   layer. Returns 0, or -1 on a token id out of range. */
int ox_decode(const ox_model* m, float* conv, float* rec, const int* forced, int n_forced, int n,
              int* preds, int* inputs, float* trace) {
  const ox_dims* d = &m->d;
  g_bf16 = d->bf16;
  const int H = d->hidden, C = 2 * d->nk * d->kd + d->nv * d->vd;
  ox_ws w;
  ws_init(&w, d);
  float* h = xalloc(4 * (size_t)H);
  float* hsq = xalloc(4 * (size_t)H);
  int tok = n_forced > 0 ? forced[0] : 0, rc = 0;
  for (int i = 0; i < n; i++) {
    if (tok < 0 || tok >= d->vocab) { rc = -1; break; }
    if (inputs) inputs[i] = tok;
    embed_row(m, tok, h);
    for (int L = 0; L < d->n_layers; L++) {
      layer_step(m, L, h, conv + (size_t)L * C * d->conv, rec + (size_t)L * d->nv * d->kd * d->vd,
                 &w, hsq);
      if (trace) memcpy(trace + ((size_t)i * d->n_layers + L) * H, h, 4 * (size_t)H);
    }
    int p = head_argmax(m, h, &w, hsq);
    preds[i] = p;
    tok = i + 1 < n_forced ? forced[i + 1] : p;
  }
  free(h);
  free(hsq);
  ws_free(&w);
  return rc;
}

/* One layer's step on a given residual h (in place) -- the per-layer comparison against the
   stock decoder layer. */
void ox_layer_step(const ox_model* m, int L, float* h, float* conv_L, float* rec_L) {
  g_bf16 = m->d.bf16;
  ox_ws w;
  ws_init(&w, &m->d);
  float* hsq = xalloc(4 * (size_t)m->d.hidden);
  layer_step(m, L, h, conv_L, rec_L, &w, hsq);
  free(hsq);
  ws_free(&w);
}

/* The head on residual rows h (T, hidden): logits (T, vocab) if given, and the argmax. */
void ox_head(const ox_model* m, const float* h, int T, float* logits, int* pred) {
  g_bf16 = m->d.bf16;
  ox_ws w;
  ws_init(&w, &m->d);
  float* hsq = xalloc(4 * (size_t)m->d.hidden);
  for (int t = 0; t < T; t++) {
    pred[t] = head_argmax(m, h + (size_t)t * m->d.hidden, &w, hsq);
    if (logits) memcpy(logits + (size_t)t * m->d.vocab, w.logits, 4 * (size_t)m->d.vocab);
  }
  free(hsq);
  ws_free(&w);
}

/* torch_recurrent_gated_delta_rule for one token (the test of the delta rule alone): q, k
   (nk, kd), v (nv, vd), beta (nv) in the model dtype (bf16 != 0), g (nv) fp32; S (nv, kd, vd)
   updated in place; o (nv, vd) written. */
void ox_rec_step(int nk, int nv, int bf16, const float* q, const float* k, const float* v,
                 const float* g, const float* beta, float* S, float* o) {
  ox_dims d;
  memset(&d, 0, sizeof d);
  d.nk = nk; d.nv = nv; d.kd = 256; d.vd = 128; d.hidden = 1; d.n_layers = 1; d.conv = 4;
  d.inter = 1; d.vocab = 1; d.bf16 = bf16;
  g_bf16 = bf16;
  ox_ws w;
  ws_init(&w, &d);
  rec_heads(&d, q, k, v, g, beta, S, &w);
  memcpy(o, w.o, 4 * (size_t)nv * 128);
  ws_free(&w);
}

/* ---------------------------------------------------------------------------------------------
   torch_chunk_gated_delta_rule (TF:249-327), the stock forward's T > 1 delta rule, for one value
   head over positions 0 .. T - 1 in chunks of C from position 0 (the sequence padded with zero
   positions to a multiple of C, as F.pad does): everything in fp32 (the function casts its
   inputs to float32). q, k (T, K) are the l2-normed query and key (use_qk_l2norm_in_kernel is
   applied by the caller, in the model dtype), v (T, V), g (T) the log decays, beta (T); S (K, V)
   the initial state, overwritten with the final state; o (T, V) the fp32 outputs (the caller
   casts them to the model dtype). The matrix products sum in index order from +0; the
   cumulative sum of g accumulates in binary64 and rounds each prefix (ATen's CPU cumsum for
   float). Returns 0, or -1 if C > 64 or K, V > 256. */
int ox_chunk_gdr(int T, int K, int V, int C, const float* q, const float* k, const float* v,
                 const float* g, const float* beta, float* S, float* o) {
  if (C > 64 || C < 1 || K > 256 || V > 256) return -1;
  const float scale = (float)(1.0 / sqrt((double)K));
  float* A = xalloc(4 * 64 * 64);      /* attn, then (I - A)^-1 form */
  float* Dm = xalloc(4 * 64 * 64);     /* decay_mask */
  float* A2 = xalloc(4 * 64 * 64);     /* (q k^T) * decay_mask */
  float* U = xalloc(4 * (size_t)64 * V);  /* value = attn @ v_beta */
  float* W = xalloc(4 * (size_t)64 * K);  /* k_cumdecay = attn @ (k_beta exp(gc)) */
  float* kb = xalloc(4 * (size_t)64 * K); /* k_beta, then k_beta exp(gc) */
  float* vb = xalloc(4 * (size_t)64 * V); /* v_beta */
  float* qs = xalloc(4 * (size_t)64 * K); /* q * scale */
  float* vn = xalloc(4 * (size_t)64 * V); /* v_new */
  float* Sn = xalloc(4 * (size_t)K * V);
  float gc[64], row[64];
  for (int c0 = 0; c0 < T; c0 += C) {
    const int n = T - c0 < C ? T - c0 : C; /* live positions; the rest are the zero padding */
    /* the chunk's inputs, padded with zeros to C positions */
    double acc = 0.0;
    for (int i = 0; i < C; i++) {
      const int t = c0 + i;
      const float gi = i < n ? g[t] : 0.0f, bi = i < n ? beta[t] : 0.0f;
      acc += (double)gi;
      gc[i] = (float)acc;
      for (int d = 0; d < K; d++) {
        const float qi = i < n ? q[(size_t)t * K + d] : 0.0f, ki = i < n ? k[(size_t)t * K + d] : 0.0f;
        qs[i * K + d] = qi * scale;
        kb[i * K + d] = ki * bi;
      }
      for (int d = 0; d < V; d++) vb[i * V + d] = (i < n ? v[(size_t)t * V + d] : 0.0f) * bi;
    }
    /* decay_mask = exp(tril(gc_i - gc_j)), zero above the diagonal */
    for (int i = 0; i < C; i++)
      for (int j = 0; j < C; j++) Dm[i * 64 + j] = j <= i ? ox_expf(gc[i] - gc[j]) : 0.0f;
    /* attn = -((k_beta @ k^T) * decay_mask), zero on and above the diagonal */
    for (int i = 0; i < C; i++)
      for (int j = 0; j < C; j++) {
        if (j >= i) { A[i * 64 + j] = 0.0f; continue; }
        float s = 0.0f;
        for (int d = 0; d < K; d++) {
          const float kj = c0 + j < T ? k[(size_t)(c0 + j) * K + d] : 0.0f;
          s = s + kb[i * K + d] * kj;
        }
        A[i * 64 + j] = -(s * Dm[i * 64 + j]);
      }
    /* row i += row i (before the update) @ attn[:i, :i] (rows < i already updated) */
    for (int i = 1; i < C; i++) {
      for (int j = 0; j < i; j++) row[j] = A[i * 64 + j];
      for (int j = 0; j < i; j++) {
        float s = 0.0f;
        for (int m = 0; m < i; m++) s = s + row[m] * A[m * 64 + j];
        A[i * 64 + j] = row[j] + s;
      }
    }
    for (int i = 0; i < C; i++) A[i * 64 + i] = A[i * 64 + i] + 1.0f;
    /* value = attn @ v_beta; k_cumdecay = attn @ (k_beta * exp(gc)) */
    for (int i = 0; i < C; i++) {
      const float e = ox_expf(gc[i]);
      for (int d = 0; d < K; d++) kb[i * K + d] = kb[i * K + d] * e;
    }
    for (int i = 0; i < C; i++) {
      for (int d = 0; d < V; d++) {
        float s = 0.0f;
        for (int m = 0; m < C; m++) s = s + A[i * 64 + m] * vb[m * V + d];
        U[i * V + d] = s;
      }
      for (int d = 0; d < K; d++) {
        float s = 0.0f;
        for (int m = 0; m < C; m++) s = s + A[i * 64 + m] * kb[m * K + d];
        W[i * K + d] = s;
      }
    }
    /* attn2 = (q @ k^T) * decay_mask (zero above the diagonal) */
    for (int i = 0; i < C; i++)
      for (int j = 0; j < C; j++) {
        float s = 0.0f;
        for (int d = 0; d < K; d++) {
          const float kj = c0 + j < T ? k[(size_t)(c0 + j) * K + d] : 0.0f;
          s = s + qs[i * K + d] * kj;
        }
        A2[i * 64 + j] = s * Dm[i * 64 + j];
      }
    /* v_new = value - k_cumdecay @ S; o = (q exp(gc)) @ S + attn2 @ v_new */
    for (int i = 0; i < C; i++) {
      const float e = ox_expf(gc[i]);
      for (int d = 0; d < V; d++) {
        float s = 0.0f;
        for (int m = 0; m < K; m++) s = s + W[i * K + m] * S[(size_t)m * V + d];
        vn[i * V + d] = U[i * V + d] - s;
      }
      for (int d = 0; d < V; d++) {
        float s = 0.0f;
        for (int m = 0; m < K; m++) s = s + (qs[i * K + m] * e) * S[(size_t)m * V + d];
        if (i < n) o[(size_t)(c0 + i) * V + d] = s;
      }
    }
    for (int i = 0; i < n; i++)
      for (int d = 0; d < V; d++) {
        float s = 0.0f;
        for (int m = 0; m < C; m++) s = s + A2[i * 64 + m] * vn[m * V + d];
        o[(size_t)(c0 + i) * V + d] = o[(size_t)(c0 + i) * V + d] + s;
      }
    /* S = S * exp(gc[-1]) + (k * exp(gc[-1] - gc))^T @ v_new */
    const float el = ox_expf(gc[C - 1]);
    for (int i = 0; i < C; i++) row[i] = ox_expf(gc[C - 1] - gc[i]);
    for (int m = 0; m < K; m++)
      for (int d = 0; d < V; d++) {
        float s = 0.0f;
        for (int i = 0; i < C; i++) {
          const float ki = c0 + i < T ? k[(size_t)(c0 + i) * K + m] : 0.0f;
          s = s + (ki * row[i]) * vn[i * V + d];
        }
        Sn[(size_t)m * V + d] = S[(size_t)m * V + d] * el + s;
      }
    memcpy(S, Sn, 4 * (size_t)K * V);
  }
  free(A); free(Dm); free(A2); free(U); free(W); free(kb); free(vb); free(qs); free(vn); free(Sn);
  return 0;
}

/* The stock forward over T tokens at once (transformers' T > 1 path, Qwen3_5GatedDeltaNet.forward
   TF:454-543 with causal_conv1d_fn over the cached window and torch_chunk_gated_delta_rule in
   chunks of C from the cached state), layer after layer, without the head: each position's norms,
   projections, conv, l2norms, gated norm, out_proj and MLP are the decode step's; the delta rule
   is ox_chunk_gdr per value head over the T positions, its fp32 outputs cast to the model dtype.
   conv (n_layers, n_conv, conv) and rec (n_layers, nv, kd, vd) are updated in place; h (T, hidden)
   holds the embedding rows on entry and the last layer's outputs on return; trace (optional,
   T x n_layers x hidden) gets every layer's output. */
void ox_prefill_chunked(const ox_model* m, float* conv, float* rec, float* h, int T, int C,
                        float* trace) {
  const ox_dims* d = &m->d;
  g_bf16 = d->bf16;
  const int H = d->hidden, K = d->conv, kd = d->kd, vd = d->vd, nk = d->nk, nv = d->nv;
  const int R = nv / nk, NC = 2 * nk * kd + nv * vd, QK = 2 * nk * kd;
  ox_ws w;
  ws_init(&w, d);
  float* hsq = xalloc(4 * (size_t)H);
  float* XN = xalloc(4 * (size_t)T * H);          /* the input norm's output per position */
  float* Y = xalloc(4 * (size_t)T * NC);          /* conv outputs */
  float* Qn = xalloc(4 * (size_t)T * nk * kd);    /* l2-normed queries and keys, per key head */
  float* Kn = xalloc(4 * (size_t)T * nk * kd);
  float* G = xalloc(4 * (size_t)T * nv);
  float* Bt = xalloc(4 * (size_t)T * nv);
  float* O = xalloc(4 * (size_t)T * nv * vd);     /* the delta rule's outputs (model dtype) */
  float* qh = xalloc(4 * (size_t)T * kd);
  float* kh_ = xalloc(4 * (size_t)T * kd);
  float* vh_ = xalloc(4 * (size_t)T * vd);
  float* gh = xalloc(4 * (size_t)T);
  float* bh = xalloc(4 * (size_t)T);
  float* oh = xalloc(4 * (size_t)T * vd);
  for (int L = 0; L < d->n_layers; L++) {
    const ox_layer* ly = &m->layers[L];
    float* cs = conv + (size_t)L * NC * K;
    float* S = rec + (size_t)L * nv * kd * vd;
    /* per position: norm, projections, conv (the windows shift in position order), gates */
    for (int t = 0; t < T; t++) {
      float* ht = h + (size_t)t * H;
      rms_norm(ht, H, d->rms_eps, ly->ln_in, hsq, XN + (size_t)t * H);
      csr_mv(&ly->qkv, XN + (size_t)t * H, w.P);
      csr_mv(&ly->b, XN + (size_t)t * H, w.b);
      csr_mv(&ly->a, XN + (size_t)t * H, w.a);
      conv_channels(ly, cs, &w, 0, NC, NULL, K, 1);
      memcpy(Y + (size_t)t * NC, w.y, 4 * (size_t)NC);
      for (int v = 0; v < nv; v++) {
        Bt[(size_t)t * nv + v] = D(ox_sigmoid(w.b[v]));
        G[(size_t)t * nv + v] = (-ox_expf(ly->A_log[v])) * ox_softplus(w.a[v] + ly->dt_bias[v]);
      }
      for (int k = 0; k < nk; k++) { /* l2norm in the model dtype (zero stays zero) */
        l2norm_D(w.y + (size_t)k * kd, kd, w.sq, Qn + ((size_t)t * nk + k) * kd);
        l2norm_D(w.y + (size_t)(nk + k) * kd, kd, w.sq, Kn + ((size_t)t * nk + k) * kd);
      }
    }
    /* the chunked delta rule per value head over the T positions */
    for (int v = 0; v < nv; v++) {
      const int k = v / R;
      for (int t = 0; t < T; t++) {
        memcpy(qh + (size_t)t * kd, Qn + ((size_t)t * nk + k) * kd, 4 * (size_t)kd);
        memcpy(kh_ + (size_t)t * kd, Kn + ((size_t)t * nk + k) * kd, 4 * (size_t)kd);
        memcpy(vh_ + (size_t)t * vd, Y + (size_t)t * NC + QK + (size_t)v * vd, 4 * (size_t)vd);
        gh[t] = G[(size_t)t * nv + v];
        bh[t] = Bt[(size_t)t * nv + v];
      }
      ox_chunk_gdr(T, kd, vd, C, qh, kh_, vh_, gh, bh, S + (size_t)v * kd * vd, oh);
      for (int t = 0; t < T; t++)
        for (int j = 0; j < vd; j++) O[((size_t)t * nv + v) * vd + j] = D(oh[(size_t)t * vd + j]);
    }
    /* per position: gated norm, out_proj, residual; the MLP */
    for (int t = 0; t < T; t++) {
      float* ht = h + (size_t)t * H;
      const float* xn = XN + (size_t)t * H;
      for (int v = 0; v < nv; v++) {
        const float* o = O + ((size_t)t * nv + v) * vd;
        float* on = w.on + (size_t)v * vd;
        for (int j = 0; j < vd; j++) w.sq[j] = o[j] * o[j];
        float ss = ox_sum_64(w.sq, vd);
        float rr = ox_rsqrt(ss / (float)vd + d->gated_eps);
        for (int j = 0; j < vd; j++) {
          float zj = D(row_dot(&ly->z, v * vd + j, xn));
          float t1 = D(o[j] * rr);
          float t2 = D(ly->gnorm[j] * t1);
          on[j] = D(t2 * ox_silu(zj));
        }
      }
      csr_mv(&ly->out, w.on, w.out);
      for (int i = 0; i < H; i++) ht[i] = D(ht[i] + w.out[i]);
      rms_norm(ht, H, d->rms_eps, ly->ln_post, hsq, w.xn);
      csr_mv(&ly->gate, w.xn, w.gt);
      csr_mv(&ly->up, w.xn, w.up);
      for (int u = 0; u < d->inter; u++) {
        const float gt = w.gt[u];
        w.act[u] = D(D(gt == 0.0f ? gt : ox_silu(gt)) * w.up[u]);
      }
      csr_mv(&ly->down, w.act, w.out);
      for (int i = 0; i < H; i++) ht[i] = D(ht[i] + w.out[i]);
      if (trace) memcpy(trace + ((size_t)t * d->n_layers + L) * H, ht, 4 * (size_t)H);
    }
  }
  void* ps[] = {hsq, XN, Y, Qn, Kn, G, Bt, O, qh, kh_, vh_, gh, bh, oh};
  for (size_t i = 0; i < sizeof(ps) / sizeof(ps[0]); i++) free(ps[i]);
  ws_free(&w);
}

/* The embedding rows of tokens (T) into h (T, hidden); 0, or -1 on a token out of range. */
int ox_embed(const ox_model* m, const int* tokens, int T, float* h) {
  for (int t = 0; t < T; t++) {
    if (tokens[t] < 0 || tokens[t] >= m->d.vocab) return -1;
    embed_row(m, tokens[t], h + (size_t)t * m->d.hidden);
  }
  return 0;
}
