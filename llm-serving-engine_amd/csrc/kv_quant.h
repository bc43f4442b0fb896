// Quantization of one (token, kv head) row of the int8 KV cache (QuantizedKV.quantize,
// reference attention.py:153-157, with the key-smoothing division of attention.py:243-245):
//   x' = smooth ? x / smooth : x;  s = max(amax |x'|, 1e-8) / 127  (clamp, then divide);
//   q = clamp(round_half_even(x' / s), -127, 127)
// One wavefront per row; lane i holds elements i, i + 64, ... (N of them). IEEE division and
// rintf, no contraction (none of these operations is a multiply-add): bit-exact with torch's
// CPU ops.
#pragma once

#include "common.h"

namespace lsh {

template <int N>
__device__ __forceinline__ void kv_quant_row(const float (&x)[N], const float* smooth, int D,
                                             int8_t* out, float* scale_out) {
  const int lane = threadIdx.x % kWave;
  float v[N];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int d = lane + i * kWave;
    v[i] = (d < D && smooth) ? x[i] / smooth[d] : x[i];
    if (d < D) amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max_from<1>(amax);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int d = lane + i * kWave;
    if (d < D) out[d] = static_cast<int8_t>(fminf(fmaxf(rintf(v[i] / s), -127.f), 127.f));
  }
  if (lane == 0) *scale_out = s;
}

// kv_quant_row for a full row (D = 64 N) whose smoothing factors are already in registers
// (sm[i] for element lane + 64 i, used when `smooth`): the same operations, the same bits.
template <int N>
__device__ __forceinline__ void kv_quant_row_smoothed(const float (&x)[N], const float (&sm)[N],
                                                      bool smooth, int8_t* out, float* scale_out) {
  const int lane = threadIdx.x % kWave;
  float v[N];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = smooth ? x[i] / sm[i] : x[i];
    amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max_from<1>(amax);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
#pragma unroll
  for (int i = 0; i < N; ++i)
    out[lane + i * kWave] = static_cast<int8_t>(fminf(fmaxf(rintf(v[i] / s), -127.f), 127.f));
  if (lane == 0) *scale_out = s;
}

}  // namespace lsh
