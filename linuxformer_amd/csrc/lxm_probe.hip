// Cross-workgroup synchronisation costs on MI355X, measured with the primitives the decode and
// dense kernels use (lxm_sync.h): agent-scope relaxed words polled by one thread per workgroup
// with the same bounded spin (s_sleep between polls, a 3 s wall-clock limit that sets the error
// word). The decode's latency bound is built from these figures.
//
// kind 0: a grid barrier over every workgroup of the launch: each arrives on one of 8 counter
//         copies (blockIdx % 8, 128 bytes apart: the per-XCD copies lxm_dn_run uses) and polls
//         their sum; the figure is microseconds per barrier.
// kind 1: a round trip between workgroup 0 and workgroup `far` (workgroups are dealt to the 8
//         XCDs in turn, so far = 1 sits on another XCD and far = 8 on the same one): 0 writes i,
//         far waits for it and writes i back, 0 waits; microseconds per round trip.
// Both time n_iter operations after a first one (which absorbs the launch's skew), on the
// 100 MHz wall clock of workgroup 0.
#include "lxm_sync.h"

#include "../../include/lxm.h"

namespace {

constexpr int NCOPY = 8;
constexpr int W_PING = 8 * 32, W_PONG = 9 * 32;

__device__ bool spin_sum(const uint32_t* p, uint32_t target, int32_t* err) {
  const uint64_t t0 = wall();
  for (;;) {
    uint32_t sum = 0;
#pragma unroll
    for (int g = 0; g < NCOPY; g++) sum += ld_rlx(p + 32 * g);
    if ((int32_t)(sum - target) >= 0) return true;
    __builtin_amdgcn_s_sleep(2);
    if (__hip_atomic_load(gp(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    if (wall() - t0 > TIMEOUT_TICKS) {
      __hip_atomic_fetch_max(gp(err), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

__global__ void __launch_bounds__(64) k_sync(int kind, int n_iter, int far, uint32_t* words,
                                             int32_t* err, float* out) {
  if (threadIdx.x != 0) return;
  const uint32_t nb = gridDim.x, b = blockIdx.x;
  uint64_t t0 = 0;
  bool ok = true;
  if (kind == 0) {
    uint32_t* mine = words + 32 * (b % NCOPY);
    for (int i = 0; i <= n_iter && ok; i++) {
      if (i == 1) t0 = wall();
      add_rlx(mine, 1u);
      ok = spin_sum(words, (uint32_t)(i + 1) * nb, err);
    }
  } else if (b == 0) {
    for (int i = 0; i <= n_iter && ok; i++) {
      if (i == 1) t0 = wall();
      st_rlx(words + W_PING, (uint32_t)(i + 1));
      ok = spin_ge(words + W_PONG, (uint32_t)(i + 1), err, 2);
    }
  } else if ((int)b == far) {
    for (int i = 0; i <= n_iter && ok; i++) {
      ok = spin_ge(words + W_PING, (uint32_t)(i + 1), err, 3);
      if (ok) st_rlx(words + W_PONG, (uint32_t)(i + 1));
    }
  }
  if (b == 0) out[0] = ok ? (float)(wall() - t0) * 0.01f / (float)n_iter : -1.0f;
}

}  // namespace

extern "C" int lxm_t_sync(int kind, int n_iter, int n_blocks, int far, uint32_t* words,
                          int32_t* err, float* out_us, void* stream) {
  if (kind < 0 || kind > 1 || n_iter < 1 || n_blocks < 1 || n_blocks > 1024) return (int)hipErrorInvalidValue;
  if (kind == 1 && (far < 1 || far >= n_blocks)) return (int)hipErrorInvalidValue;
  void* args[] = {&kind, &n_iter, &far, &words, &err, &out_us};
  return (int)hipLaunchCooperativeKernel((const void*)k_sync, dim3(n_blocks), dim3(64), args, 0,
                                         (hipStream_t)stream);
}
