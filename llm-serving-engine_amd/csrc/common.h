// Shared helpers of the gfx950 kernels: error reporting for the C ABI, launch checks and
// wavefront (64-lane) reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "llmserve_hip.h"

namespace lsh {

// Records the calling thread's last error message (read by llmserve_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks the status of the launch just enqueued.
int launch_status(const char* what);

constexpr int kWave = 64;

// Butterfly sum / max over the lanes whose index differs only in the bits of [lo, 64):
// lane groups of size `lo` stay separate. All lanes get the result.
template <int LO = 1>
__device__ __forceinline__ float wave_sum_from(float v) {
#pragma unroll
  for (int o = 32; o >= LO; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

template <int LO = 1>
__device__ __forceinline__ float wave_max_from(float v) {
#pragma unroll
  for (int o = 32; o >= LO; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Sum over the `W` consecutive lanes of each group of W (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

}  // namespace lsh

#define LSH_CHECK(cond, ...)                 \
  do {                                       \
    if (!(cond)) {                           \
      ::lsh::set_error(__VA_ARGS__);         \
      return LLMSERVE_ERR_INVALID;           \
    }                                        \
  } while (0)
