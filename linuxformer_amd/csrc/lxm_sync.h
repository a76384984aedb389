// Cross-workgroup data on MI355X (gfx950): agent-scope relaxed loads and stores (sc1: coherent
// across the 8 XCDs, whose L2s are not), the drain before a workgroup signals, and the bounded
// spin every wait uses (a wall-clock limit that sets the run's error word, so every workgroup
// leaves and the grid drains).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define TIMEOUT_TICKS 300000000ull  // 3 s of the 100 MHz wall clock

#define GAS __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ GAS T* gp(T* q) {
  return (GAS T*)q;
}
template <class T>
__device__ __forceinline__ const GAS T* gp(const T* q) {
  return (const GAS T*)q;
}

// a struct from global memory through global loads (a generic copy would be flat loads)
template <class T>
__device__ __forceinline__ T ldg(const T* q) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  T r;
  const GAS uint32_t* src = gp(reinterpret_cast<const uint32_t*>(q));
  uint32_t* dst = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); i++) dst[i] = src[i];
  return r;
}
typedef float v4f __attribute__((ext_vector_type(4)));

// agent-scope relaxed atomics: sc1 loads and stores on gfx950, coherent across the XCDs
__device__ __forceinline__ uint32_t ld_rlx(const uint32_t* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_rlx(uint32_t* p, uint32_t v) {
  __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_rlxf(const float* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_rlxf(float* p, float v) {
  __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void add_rlx(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_add(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// every earlier memory op of this wave has completed (its stores are visible at agent scope
// when they were agent-scope atomics)
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint64_t wall() { return __builtin_amdgcn_s_memrealtime(); }


// a pointer the whole wave shares, in scalar registers (a buffer resource built from it is
// uniform: no waterfall loop around the store)
__device__ __forceinline__ float* wave_ptr(float* q) {
  const uint64_t u = reinterpret_cast<uint64_t>(q);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<float*>(((uint64_t)hi << 32) | lo);
}
// 16 bytes from global memory at agent scope (a buffer load with the sc1 policy)
__device__ __forceinline__ v4f ld4_rlx(const float* base, int idx) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, idx * 4, 0, 16));
}

// spin (one thread) until the counter reaches target (modulo 2^32); false on timeout or
// another block's error
__device__ inline bool spin_ge(const uint32_t* p, uint32_t target, int32_t* err, int code) {
  const uint64_t t0 = wall();
  while ((int32_t)(ld_rlx(p) - target) < 0) {
    __builtin_amdgcn_s_sleep(2);
    if (__hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    if (wall() - t0 > TIMEOUT_TICKS) {
      __hip_atomic_fetch_max(gp(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
  return true;
}
