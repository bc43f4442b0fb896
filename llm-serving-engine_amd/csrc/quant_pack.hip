// Load-time quantizers (int8 rows, int4 groups with AWQ fold + nibble packing) and the int8
// KV-cache quantize-and-scatter.
//
// These must reproduce the reference's torch CPU arithmetic bit for bit, so:
//  * every division is an IEEE correctly rounded fp32 division (the build passes
//    -fhip-fp32-correctly-rounded-divide-sqrt; never a reciprocal multiply);
//  * rounding is round-half-to-even (rintf -> v_rndne_f32), as torch.round;
//  * no multiply-add contraction anywhere in this file (torch runs each op on its own);
//  * fp32 denormals are kept (gfx950 default, as the CPU).
// min/max reductions are order independent, so the reduction shape does not matter.
#pragma clang fp contract(off)

#include "common.h"
#include "kv_quant.h"

namespace {

using lsh::kWave;
constexpr int kMaxKvRow = 256;  // head_dim limit of the KV quantizer (one wavefront per row)

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
  return fminf(fmaxf(v, lo), hi);
}

// One 256-thread workgroup per output row n (quant.py:41-43).
__global__ __launch_bounds__(256) void int8_quantize_rows(const float* __restrict__ w,
                                                          int8_t* __restrict__ q,
                                                          float* __restrict__ scale,
                                                          int64_t K) {
  const int64_t n = blockIdx.x;
  const float* row = w + n * K;
  float amax = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(row[k]));
  amax = lsh::wave_max_from<1>(amax);
  __shared__ float red[4];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8): divide, then clamp.
  const float s = fmaxf(amax / 127.0f, 1e-8f);
  if (threadIdx.x == 0) scale[n] = s;
  int8_t* qrow = q + n * K;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    qrow[k] = static_cast<int8_t>(clampf(rintf(row[k] / s), -127.f, 127.f));
}

// One wavefront per (row n, group g) (quant.py:82-90, AWQ fold quant.py:103-107, packing
// quant.py:113-116). Lanes stride over the group's input channels.
__global__ __launch_bounds__(256) void int4_quantize_groups(
    const float* __restrict__ w, const float* __restrict__ act, uint8_t* __restrict__ nib,
    float* __restrict__ gs, float* __restrict__ gz, int64_t N, int64_t K, int64_t group) {
  const int lane = threadIdx.x % kWave;
  const int64_t G = K / group;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (gid >= N * G) return;  // whole wave exits; the kernel has no barriers
  const int64_t n = gid / G, g = gid % G;
  const float* base = w + n * K + g * group;
  const float* sc = act ? act + g * group : nullptr;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t i = lane; i < group; i += kWave) {
    const float v = sc ? base[i] * sc[i] : base[i];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  }
  const float s = fmaxf((mx - mn) / 15.0f, 1e-8f);
  if (lane == 0) {
    gs[gid] = s;
    gz[gid] = mn + 8.0f * s;  // two roundings (8*s is exact, then the add)
  }
  uint8_t* out = nib + n * (K / 2) + g * group / 2;
  for (int64_t j = lane; j < group / 2; j += kWave) {
    float v0 = base[2 * j], v1 = base[2 * j + 1];
    if (sc) {
      v0 = v0 * sc[2 * j];
      v1 = v1 * sc[2 * j + 1];
    }
    const int q0 = static_cast<int>(clampf(rintf((v0 - mn) / s), 0.f, 15.f));
    const int q1 = static_cast<int>(clampf(rintf((v1 - mn) / s), 0.f, 15.f));
    out[j] = static_cast<uint8_t>(q0 | (q1 << 4));
  }
}

// inv_act_scale = 1.0 / act_scale (torch: act_scale.reciprocal() * 1.0, quant.py:104).
__global__ void reciprocal_kernel(const float* __restrict__ a, float* __restrict__ r, int64_t K) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < K) r[i] = 1.0f / a[i];
}

// One wavefront per (token t, kv head h): QuantizedKV.quantize + write (attention.py:153-162),
// with the smoothing division k / smooth fused in front (attention.py:245).
__global__ __launch_bounds__(256) void kv_quantize_write_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ slots,
    const float* __restrict__ smooth, int8_t* __restrict__ data, float* __restrict__ scale,
    int64_t T, int64_t Hk, int64_t D, int64_t num_slots) {
  const int lane = threadIdx.x % kWave;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (gid >= T * Hk) return;
  const int64_t t = gid / Hk, h = gid % Hk;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const float* xr = x + (t * Hk + h) * D;
  float v[kMaxKvRow / kWave];
#pragma unroll
  for (int i = 0; i < kMaxKvRow / kWave; ++i) {
    const int64_t d = lane + i * kWave;
    v[i] = d < D ? xr[d] : 0.f;
  }
  lsh::kv_quant_row(v, smooth ? smooth + h * D : nullptr, static_cast<int>(D),
                    data + (slot * Hk + h) * D, scale + slot * Hk + h);
}

constexpr int kWavesPerBlock = 4;

}  // namespace

extern "C" int llmserve_int8_quantize(const float* w, int8_t* q, float* scale, int64_t N,
                                      int64_t K, void* stream) {
  LSH_CHECK(N >= 0 && K >= 1, "int8_quantize: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  LSH_CHECK(N <= 0x7fffffff, "int8_quantize: N=%lld too large", (long long)N);
  if (N == 0) return LLMSERVE_OK;
  LSH_CHECK(w && q && scale, "int8_quantize: null pointer");
  hipLaunchKernelGGL(int8_quantize_rows, dim3(static_cast<unsigned>(N)), dim3(256), 0,
                     lsh::as_stream(stream), w, q, scale, K);
  return lsh::launch_status("int8_quantize");
}

extern "C" int llmserve_int4_quantize(const float* w, const float* act_scale, uint8_t* nibbles,
                                      float* g_scale, float* g_zero, float* inv_act_scale,
                                      int64_t N, int64_t K, int64_t group_size, void* stream) {
  LSH_CHECK(N >= 0 && K >= 1 && group_size >= 2, "int4_quantize: bad shape");
  LSH_CHECK(K % group_size == 0, "in_features %lld not divisible by group %lld", (long long)K,
            (long long)group_size);
  LSH_CHECK(group_size % 2 == 0, "int4_quantize: group_size must be even");
  const int64_t waves = N * (K / group_size);
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  LSH_CHECK(blocks <= 0x7fffffff, "int4_quantize: too many groups");
  hipStream_t st = lsh::as_stream(stream);
  if (act_scale && inv_act_scale) {
    hipLaunchKernelGGL(reciprocal_kernel, dim3(static_cast<unsigned>((K + 255) / 256)), dim3(256),
                       0, st, act_scale, inv_act_scale, K);
    const int rc = lsh::launch_status("int4_quantize(reciprocal)");
    if (rc) return rc;
  }
  if (waves == 0) return LLMSERVE_OK;
  LSH_CHECK(w && nibbles && g_scale && g_zero, "int4_quantize: null pointer");
  hipLaunchKernelGGL(int4_quantize_groups, dim3(static_cast<unsigned>(blocks)),
                     dim3(kWavesPerBlock * kWave), 0, st, w, act_scale, nibbles, g_scale, g_zero,
                     N, K, group_size);
  return lsh::launch_status("int4_quantize");
}

extern "C" int llmserve_kv_quantize_write(const float* x, const int64_t* slots,
                                          const float* smooth, int8_t* data, float* scale,
                                          int64_t T, int64_t Hk, int64_t D, int64_t num_slots,
                                          void* stream) {
  LSH_CHECK(T >= 0 && Hk >= 1 && D >= 1 && num_slots >= 0, "kv_quantize_write: bad shape");
  LSH_CHECK(D <= kMaxKvRow, "kv_quantize_write: head_dim %lld > %d", (long long)D, kMaxKvRow);
  const int64_t waves = T * Hk;
  if (waves == 0) return LLMSERVE_OK;
  LSH_CHECK(x && slots && data && scale, "kv_quantize_write: null pointer");
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  LSH_CHECK(blocks <= 0x7fffffff, "kv_quantize_write: too many rows");
  hipLaunchKernelGGL(kv_quantize_write_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(kWavesPerBlock * kWave), 0, lsh::as_stream(stream), x, slots, smooth,
                     data, scale, T, Hk, D, num_slots);
  return lsh::launch_status("kv_quantize_write");
}
