// Per-head RMSNorm and rotate-half RoPE of one (token, head) row held by a wavefront, shared
// by the post-qkv decode kernels (fused_ops.cpp:101-127 of the reference: rope_qk_ with the
// Qwen3 q/k norms).
#pragma once

#include "common.h"

namespace lsh {

// One wavefront per (token, head). Lane l holds elements d = l + 64 i (i < N = max(1, D / 64));
// when D < 64 the lanes >= D hold nothing.
// Per-head RMSNorm (norm_row with the head's weight), then out[d] = x[d] c[d] - x[d + D/2]
// s[d] for d < D/2 and x[d] c[d] + x[d - D/2] s[d] above (rotate_half, fused_ops.cpp:121-124).
template <int N>
__device__ __forceinline__ void norm_rope(float (&v)[N], const float* w, const float* c,
                                          const float* s, int D, float eps) {
  const int lane = threadIdx.x % kWave;
  if (w) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (lane + i * kWave < D) ss += v[i] * v[i];
    ss = lsh::wave_sum_from<1>(ss);
    const float inv = 1.f / sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int d = lane + i * kWave;
      if (d < D) v[i] = w[d] * (v[i] * inv);
    }
  }
  const int half = D / 2;
  float p[N];  // partner element d +- D/2
  if (half % kWave == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = v[(i + (half / kWave)) % N];
  } else {  // D = 64: the partner is 32 lanes away; D = 32 / 16: within the first lanes
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = __shfl_xor(v[i], half, kWave);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int d = lane + i * kWave;
    if (d < D) v[i] = d < half ? v[i] * c[d] - p[i] * s[d] : v[i] * c[d] + p[i] * s[d];
  }
}

}  // namespace lsh
