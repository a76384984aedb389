// The decode's float arithmetic on gfx950, one rounding at a time.
//
// Every op is a single IEEE binary32 op rounded to nearest even; the library is built with
// -ffp-contract=off, so a*b+c is never fused, and without fast-math, so nothing is reordered;
// f32 division and sqrt are the correctly rounded sequences (clang's HIP default). exp and
// log1p are evaluated in binary64 and rounded once to binary32: exp by a Cody-Waite reduction
// with ln 2 split in two and a degree-13 Taylor polynomial for exp(r), |r| <= ln2/2; log by
// f in [sqrt(1/2), sqrt(2)] and the series 2 atanh(s) = 2 (s + s^3/3 + ... + s^23/23). The
// compositions silu(x) = x / (1 + exp(-x)), sigmoid(x) = 1 / (1 + exp(-x)),
// softplus(x) = x > 20 ? x : log1p(exp(x)) and rsqrt(x) = 1 / sqrt(x) are those of ATen's CPU
// kernels for torch.nn.functional.silu/sigmoid/softplus and torch.rsqrt, which the stock
// forward (transformers/models/qwen3_5/modeling_qwen3_5.py:168-184, :242-245, :497-499,
// :727) calls; the results agree with ATen's on every bf16 input.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lxm {

__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t fbits(float x) { return __float_as_uint(x); }

// round to bf16, nearest even, by gfx950's v_cvt_pk_bf16_f32; returned widened to f32. Equal to
// c10::BFloat16's rounding on every non-NaN input, denormals included; a NaN stays a NaN (the
// hardware keeps its sign and leading payload bits where c10 returns 0x7fc0; no NaN arises
// from finite inputs in the decode)
__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ float bf16f(uint32_t hi16) { return bitsf(hi16 << 16); }
// the same for two values by one conversion (one v_cvt_pk_bf16_f32 for the pair)
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x2 bf16r2(f32x2 v) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
  return f32x2{bitsf(u << 16), bitsf(u & 0xffff0000u)};
}

// the model dtype's rounding
template <bool BF>
__device__ __forceinline__ float rd(float x) {
  if constexpr (BF) return bf16r(x);
  else return x;
}

__device__ __forceinline__ double pow2i(int k) {
  return __longlong_as_double((long long)(k + 1023) << 52);
}

__device__ __forceinline__ float cr_exp(float x) {
  if (x != x) return x;
  if (x > 89.0f) return __builtin_inff();
  if (x < -110.0f) return 0.0f;
  const double xd = (double)x;
  const double kd = __builtin_floor(xd * 0x1.71547652b82fep+0 + 0.5);
  const double r = (xd - kd * 0x1.62e42fee00000p-1) - kd * 0x1.a39ef35793c76p-33;
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
  return (float)(p * pow2i((int)kd));
}

__device__ __forceinline__ double log_ge1(double u) {
  long long b = __double_as_longlong(u);
  int m = (int)((b >> 52) & 0x7ff) - 1023;
  double f = __longlong_as_double((b & 0x000fffffffffffffll) | 0x3ff0000000000000ll);
  if (f > 0x1.6a09e667f3bcdp+0) {
    f = f * 0.5;
    m += 1;
  }
  const double s = (f - 1.0) / (f + 1.0);
  const double s2 = s * s;
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
  const double lf = (2.0 * s) * p;
  return (double)m * 0x1.62e42fee00000p-1 + ((double)m * 0x1.a39ef35793c76p-33 + lf);
}

// log1p(y), y >= 0
__device__ __forceinline__ float cr_log1p(float y) {
  if (y != y) return y;
  if (y == __builtin_inff()) return y;
  const double yd = (double)y;
  if (yd < 0x1p-29) return (float)(yd - (yd * yd) * 0.5);
  return (float)log_ge1(1.0 + yd);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + cr_exp(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + cr_exp(-x)); }

// bf16r(silu(g)) for a bf16 value g (every MLP unit and conv output rounds silu's result to
// bf16 at once), equal bit for bit to the exact sequence above. A fast evaluation first:
// exp(-g) = 2^(-g*log2 e) with log2 e split in two (LH keeps 15 significant bits, so g * LH is
// exact for g's 8), each power by the hardware's exp2, then g * rcp(1 + e); its result lies
// within a few units in the last place of the exact sequence's. Where it lies within 64 units
// of a bf16 rounding boundary (low half 0x8000), or |g| >= 64, the exact sequence decides (for
// g >= 64, 1 + exp(-g) rounds to 1 and silu(g) = g). Tested on every bf16 input.
__device__ __forceinline__ float silu_bf16(float g) {
  if (g >= 64.0f) return bf16r(g);
  if (!(g > -64.0f)) return bf16r(silu(g));
  const float LH = __uint_as_float(0x3fb8aa00u), LL = __uint_as_float(0x36eca570u);
  const float e = __builtin_amdgcn_exp2f(g * -LH) * __builtin_amdgcn_exp2f(g * -LL);
  const float q = g * __builtin_amdgcn_rcpf(1.0f + e);
  if ((fbits(q) & 0xffffu) - 0x7fc0u < 0x80u) return bf16r(silu(g));
  return bf16r(q);
}
// silu rounded to the model dtype (bf16: the fast path above; fp32: the exact sequence)
template <bool BF>
__device__ __forceinline__ float silu_rd(float g) {
  if constexpr (BF) return silu_bf16(g);
  else return silu(g);
}
__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : cr_log1p(cr_exp(x)); }
__device__ __forceinline__ float rsqrt_(float x) { return 1.0f / __builtin_sqrtf(x); }

// s + x * w, rounded once as the oracle's s + D(x * w): for bf16 models x and w are bf16
// values, whose product is exact in fp32, so one fused op gives the same bits
template <bool BF>
__device__ __forceinline__ float acc(float s, float x, float w) {
  if constexpr (BF) return __builtin_fmaf(x, w, s);
  else return s + x * w;
}

// a workgroup barrier ordering LDS only: global loads in flight (the next tables or weight rows)
// stay in flight across it
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A wave's tree sum: lane 0 ends with the sum that __shfl_down at offsets 32, 16, ..., 1
// leaves there (lane l adds lane l + off). Offsets 32 and 16 by gfx950's permlane swaps, 8..1
// by DPP row shifts; no LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float wave_tree(float s) {
  const uint32_t u = __float_as_uint(s);
  s = s + __uint_as_float(__builtin_amdgcn_permlane32_swap(u, u, false, false)[1]);
  const uint32_t v = __float_as_uint(s);
  s = s + __uint_as_float(__builtin_amdgcn_permlane16_swap(v, v, false, false)[1]);
  s = s + dpp_f<0x108>(s);  // row_shl:8
  s = s + dpp_f<0x104>(s);
  s = s + dpp_f<0x102>(s);
  s = s + dpp_f<0x101>(s);
  return s;
}

// the 64-lane head sum over one wave: lane l's partial (elements l, l + 64, ...), offsets
// 32..1; every lane gets the sum
__device__ __forceinline__ float sum64(float s) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                       __builtin_bit_cast(int, wave_tree(s))));
}

// (value, index) -> one key whose unsigned maximum is torch.argmax's pick: the larger value,
// then the lower index; NaN above everything; -0 counted as +0
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  uint32_t u = fbits(v);
  uint32_t o;
  if ((u & 0x7fffffffu) > 0x7f800000u) o = 0xffffffffu;
  else {
    if ((u & 0x7fffffffu) == 0) u = 0;
    o = (u >> 31) ? ~u : (u | 0x80000000u);
  }
  return ((unsigned long long)o << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int argmax_idx(unsigned long long key) {
  return (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}
// the same order with the index in 19 bits (bits 13..31) and the low 13 bits free for a stamp:
// (value, lower index) for indices below 2^19
__device__ __forceinline__ unsigned long long argmax_key19(float v, int idx) {
  const unsigned long long k = argmax_key(v, 0);
  return (k & 0xffffffff00000000ull) | ((unsigned long long)(0x7ffffu - (uint32_t)idx) << 13);
}
__device__ __forceinline__ int argmax_idx19(unsigned long long key) {
  return (int)(0x7ffffu - (uint32_t)((key >> 13) & 0x7ffffu));
}

}  // namespace lxm
