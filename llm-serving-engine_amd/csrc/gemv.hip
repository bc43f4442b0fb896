// Weight-only int8 / int4 GEMV for decode (M <= 16 per launch; the host loops over row tiles
// up to the 64-row limit).
//
// Decode is HBM-bound: each weight byte is read once, dequantized in registers and used for
// all M activation rows. Layout of the work:
//  * a 256-thread workgroup = 4 wavefronts; wavefront w owns R consecutive output rows;
//  * a row is streamed in segments of 64*V bytes: lane l loads bytes [l*V, l*V+V) of each
//    segment with one V-byte (dwordx4 / dwordx2 / dword) load, so every wave-level load is
//    one fully coalesced 64*V-byte run;
//  * the activations x (M x K fp32) are either staged once per workgroup in LDS (the int4
//    AWQ pre-scale x * inv_act_scale is applied while staging) or read directly from the
//    L1/L2-resident copy;
//  * each lane keeps R x MT partial sums; a butterfly over the 64 lanes (DPP/permute
//    shuffles) finishes the K reduction.
// The int4 path uses the reference's group decomposition
//   y = sum_g s * sum_{k in g} x q + (z - 8 s) * sum_{k in g} x   (int8_gemv.cpp:48-52)
// evaluated per lane slice (2V input channels, always inside one group).
// Shapes that do not meet the fast path's divisibility/alignment go to a generic kernel
// with scalar loads.
#include "common.h"

namespace {

using lsh::kWave;
constexpr int kWaves = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int V>
struct Vec;
template <>
struct Vec<16> {
  using T = u32x4;
  static constexpr int kWords = 4;
};
template <>
struct Vec<8> {
  using T = u32x2;
  static constexpr int kWords = 2;
};
template <>
struct Vec<4> {
  using T = uint32_t;
  static constexpr int kWords = 1;
};

__device__ __forceinline__ uint32_t word(const u32x4& v, int i) { return v[i]; }
__device__ __forceinline__ uint32_t word(const u32x2& v, int i) { return v[i]; }
__device__ __forceinline__ uint32_t word(const uint32_t& v, int) { return v; }

// Streaming (non-temporal) load of one lane's V weight bytes: weights are read once per call.
template <int V>
__device__ __forceinline__ typename Vec<V>::T load_vec(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename Vec<V>::T*>(p));
}

// Nibbles of byte b of word u: channel 2b (low) and 2b+1 (high) of the word's 8 channels.
__device__ __forceinline__ void unpack_nibbles(uint32_t u, float (&q)[8]) {
  const uint32_t lo = u & 0x0f0f0f0fu, hi = (u >> 4) & 0x0f0f0f0fu;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    q[2 * b] = static_cast<float>((lo >> (8 * b)) & 0xffu);
    q[2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xffu);
  }
}

// Sums acc[i] over the wave and stores lane-0's totals through `store(i, value)`.
template <int NV, typename F>
__device__ __forceinline__ void wave_reduce_store(float (&acc)[NV], int lane, F store) {
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = lsh::wave_sum_from<1>(acc[i]);
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane == (i & (kWave - 1))) store(i, acc[i]);
}

// Stages x[0:M, c0:c0+width] (times inv[k] when given) into LDS as fp32 rows of stride KC
// ([MT][KC]); rows >= M are zero-filled. Requires width % 4 == 0, width <= KC,
// c0 + width <= K and 16-byte aligned x / inv rows.
template <int MT>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x,
                                        const float* __restrict__ inv, int M, int K, int c0,
                                        int width, int KC) {
  const int k4 = width / 4;
  for (int i = threadIdx.x; i < MT * k4; i += blockDim.x) {
    const int m = i / k4, c = i - m * k4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < M) {
      v = reinterpret_cast<const float4*>(x + static_cast<int64_t>(m) * K + c0)[c];
      if (inv) {
        const float4 s = reinterpret_cast<const float4*>(inv + c0)[c];
        v.x = __fmul_rn(v.x, s.x);
        v.y = __fmul_rn(v.y, s.y);
        v.z = __fmul_rn(v.z, s.z);
        v.w = __fmul_rn(v.w, s.w);
      }
    }
    reinterpret_cast<float4*>(xs + m * KC)[c] = v;
  }
}

// With XLDS, xs holds the staged chunk [MT][KC] starting at channel c0.
template <int NX, bool XLDS>
__device__ __forceinline__ void read_x(float (&xv)[NX], const float* xs,
                                       const float* __restrict__ x,
                                       const float* __restrict__ inv, int m, int M, int K, int k,
                                       int c0, int KC) {
  if (XLDS) {
    const float4* p = reinterpret_cast<const float4*>(xs + m * KC + (k - c0));
#pragma unroll
    for (int i = 0; i < NX / 4; ++i) {
      const float4 v = p[i];
      xv[4 * i] = v.x;
      xv[4 * i + 1] = v.y;
      xv[4 * i + 2] = v.z;
      xv[4 * i + 3] = v.w;
    }
  } else {
    if (m >= M) {
#pragma unroll
      for (int i = 0; i < NX; ++i) xv[i] = 0.f;
      return;
    }
    const float4* p = reinterpret_cast<const float4*>(x + static_cast<int64_t>(m) * K + k);
    const float4* s = inv ? reinterpret_cast<const float4*>(inv + k) : nullptr;
#pragma unroll
    for (int i = 0; i < NX / 4; ++i) {
      float4 v = p[i];
      if (s) {
        const float4 t = s[i];
        v.x = __fmul_rn(v.x, t.x);
        v.y = __fmul_rn(v.y, t.y);
        v.z = __fmul_rn(v.z, t.z);
        v.w = __fmul_rn(v.w, t.w);
      }
      xv[4 * i] = v.x;
      xv[4 * i + 1] = v.y;
      xv[4 * i + 2] = v.z;
      xv[4 * i + 3] = v.w;
    }
  }
}

// ---------------------------------------------------------------------------------------
// int8: y[m, n] = scale[n] * sum_k x[m, k] q[n, k]
// ---------------------------------------------------------------------------------------
template <int MT, int V, int R, bool XLDS>
__global__ __launch_bounds__(256) void int8_gemv_fast(const float* __restrict__ x,
                                                      const int8_t* __restrict__ q,
                                                      const float* __restrict__ scale,
                                                      float* __restrict__ y, int M, int N,
                                                      int K, int KC) {
  extern __shared__ float xs[];
  using VT = typename Vec<V>::T;
  constexpr int W = Vec<V>::kWords;
  constexpr int SEG = kWave * V;  // input channels per segment
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const int nseg = K / SEG;
  const int spc = KC / SEG;  // segments per staged x chunk
  const uint8_t* qb = reinterpret_cast<const uint8_t*>(q);

  VT w[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w[r] = (row0 + r < N) ? load_vec<V>(qb + static_cast<int64_t>(row0 + r) * K + lane * V)
                          : VT{};
  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;

  int c0 = 0;
  for (int j = 0; j < nseg; ++j) {
    VT wn[R];
    if (j + 1 < nseg) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        wn[r] = (row0 + r < N) ? load_vec<V>(qb + static_cast<int64_t>(row0 + r) * K +
                                             (j + 1) * SEG + lane * V)
                               : VT{};
    }
    if (XLDS && j % spc == 0) {
      c0 = j * SEG;
      if (j) __syncthreads();
      stage_x<MT>(xs, x, nullptr, M, K, c0, min(KC, K - c0), KC);
      __syncthreads();
    }
    float wf[R][V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const uint32_t u = word(w[r], i);
#pragma unroll
        for (int b = 0; b < 4; ++b)
          wf[r][4 * i + b] = static_cast<float>(static_cast<int8_t>((u >> (8 * b)) & 0xffu));
      }
    const int k0 = j * SEG + lane * V;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float xv[V];
      read_x<V, XLDS>(xv, xs, x, nullptr, m, M, K, k0, c0, KC);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float a = acc[r * MT + m];
#pragma unroll
        for (int i = 0; i < V; ++i) a += xv[i] * wf[r][i];
        acc[r * MT + m] = a;
      }
    }
    if (j + 1 < nseg) {
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = wn[r];
    }
  }
  wave_reduce_store<R * MT>(acc, lane, [&](int i, float v) {
    const int r = i / MT, m = i % MT;
    if (m < M && row0 + r < N) y[static_cast<int64_t>(m) * N + row0 + r] = v * scale[row0 + r];
  });
}

// Any shape / alignment: one wave per output row, lanes stride over k with byte loads.
template <int MT>
__global__ __launch_bounds__(256) void int8_gemv_generic(const float* __restrict__ x,
                                                         const int8_t* __restrict__ q,
                                                         const float* __restrict__ scale,
                                                         float* __restrict__ y, int M, int N,
                                                         int K) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= N) return;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;
  const int8_t* qr = q + static_cast<int64_t>(row) * K;
  for (int k = lane; k < K; k += kWave) {
    const float wv = static_cast<float>(qr[k]);
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m < M) acc[m] += x[static_cast<int64_t>(m) * K + k] * wv;
  }
  wave_reduce_store<MT>(acc, lane, [&](int m, float v) {
    if (m < M) y[static_cast<int64_t>(m) * N + row] = v * scale[row];
  });
}

// ---------------------------------------------------------------------------------------
// int4: nibble byte j of a row holds q[2j] (low) and q[2j+1] (high); w = (q - 8) s + z.
// ---------------------------------------------------------------------------------------
template <int MT, int V, int R, bool XLDS>
__global__ __launch_bounds__(256) void int4_gemv_fast(
    const float* __restrict__ x, const float* __restrict__ inv, const uint8_t* __restrict__ nib,
    const float* __restrict__ gs, const float* __restrict__ gz, float* __restrict__ y, int M,
    int N, int K, int group, int KC) {
  extern __shared__ float xs[];
  using VT = typename Vec<V>::T;
  constexpr int W = Vec<V>::kWords;
  constexpr int KL = 2 * V;         // input channels per lane slice
  constexpr int SEG = kWave * KL;   // input channels per segment
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const int RB = K / 2;  // bytes per row
  const int G = K / group;
  const int nseg = K / SEG;
  const int spc = KC / SEG;

  VT w[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w[r] = (row0 + r < N) ? load_vec<V>(nib + static_cast<int64_t>(row0 + r) * RB + lane * V)
                          : VT{};
  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;

  int c0 = 0;
  for (int j = 0; j < nseg; ++j) {
    VT wn[R];
    if (j + 1 < nseg) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        wn[r] = (row0 + r < N) ? load_vec<V>(nib + static_cast<int64_t>(row0 + r) * RB +
                                             (j + 1) * kWave * V + lane * V)
                               : VT{};
    }
    if (XLDS && j % spc == 0) {
      c0 = j * SEG;
      if (j) __syncthreads();
      stage_x<MT>(xs, x, inv, M, K, c0, min(KC, K - c0), KC);
      __syncthreads();
    }
    const int k0 = j * SEG + lane * KL;
    const int g = k0 / group;
    float s[R], c[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = min(row0 + r, N - 1);
      s[r] = gs[static_cast<int64_t>(rr) * G + g];
      c[r] = gz[static_cast<int64_t>(rr) * G + g] - 8.f * s[r];
    }
    if constexpr (MT <= 2) {
      // x slice read once per m; nibbles unpacked per (m, row).
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[KL];
        read_x<KL, XLDS>(xv, xs, x, inv, m, M, K, k0, c0, KC);
        float xsum = 0.f;
#pragma unroll
        for (int i = 0; i < KL; ++i) xsum += xv[i];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < W; ++i) {
            float qf[8];
            unpack_nibbles(word(w[r], i), qf);
#pragma unroll
            for (int e = 0; e < 8; ++e) d += xv[8 * i + e] * qf[e];
          }
          acc[r * MT + m] += s[r] * d + c[r] * xsum;
        }
      }
    } else {
      // nibbles unpacked once per row; x slice re-read per row (LDS / L1).
      float xsum[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[KL];
        read_x<KL, XLDS>(xv, xs, x, inv, m, M, K, k0, c0, KC);
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < KL; ++i) t += xv[i];
        xsum[m] = t;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float qf[KL];
#pragma unroll
        for (int i = 0; i < W; ++i) {
          float t[8];
          unpack_nibbles(word(w[r], i), t);
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[8 * i + e] = t[e];
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float xv[KL];
          read_x<KL, XLDS>(xv, xs, x, inv, m, M, K, k0, c0, KC);
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < KL; ++i) d += xv[i] * qf[i];
          acc[r * MT + m] += s[r] * d + c[r] * xsum[m];
        }
      }
    }
    if (j + 1 < nseg) {
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = wn[r];
    }
  }
  wave_reduce_store<R * MT>(acc, lane, [&](int i, float v) {
    const int r = i / MT, m = i % MT;
    if (m < M && row0 + r < N) y[static_cast<int64_t>(m) * N + row0 + r] = v;
  });
}

template <int MT>
__global__ __launch_bounds__(256) void int4_gemv_generic(
    const float* __restrict__ x, const float* __restrict__ inv, const uint8_t* __restrict__ nib,
    const float* __restrict__ gs, const float* __restrict__ gz, float* __restrict__ y, int M,
    int N, int K, int group) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= N) return;
  const int G = K / group;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;
  const uint8_t* qr = nib + static_cast<int64_t>(row) * (K / 2);
  for (int k = lane; k < K; k += kWave) {
    const uint8_t b = qr[k / 2];
    const float qv = static_cast<float>((k & 1) ? (b >> 4) : (b & 0xf));
    const int g = k / group;
    const float s = gs[static_cast<int64_t>(row) * G + g];
    const float c = gz[static_cast<int64_t>(row) * G + g] - 8.f * s;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m < M) {
        float xv = x[static_cast<int64_t>(m) * K + k];
        if (inv) xv = __fmul_rn(xv, inv[k]);
        acc[m] += s * (xv * qv) + c * xv;
      }
  }
  wave_reduce_store<MT>(acc, lane, [&](int m, float v) {
    if (m < M) y[static_cast<int64_t>(m) * N + row] = v;
  });
}

// ---------------------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------------------
constexpr int kLdsBudget = 64 * 1024;  // bytes of staged x per workgroup

int pick_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// Rows per wave: spread small matrices over more waves, amortise x reads on large ones.
int pick_rows(int N, int MT) {
  if (MT >= 8) return 2;
  if (N >= 4 * 256 * kWaves) return 4;
  if (N >= 2 * 256 * kWaves) return 2;
  return 1;
}

// Widest lane vector (16/8/4 bytes) whose segment tiles a row exactly and whose staged x
// segment (MT rows x seg_channels) fits the LDS budget; 0 = generic kernel.
int pick_vec(int64_t row_bytes, int channels_per_byte, int MT) {
  for (int v : {16, 8, 4}) {
    const int64_t seg_channels = static_cast<int64_t>(kWave) * v * channels_per_byte;
    if (row_bytes % (kWave * v) == 0 && MT * seg_channels * 4 <= kLdsBudget) return v;
  }
  return 0;
}

// Staged chunk: as many whole segments as fit the budget.
int pick_chunk(int K, int seg, int MT) {
  const int max_segs = kLdsBudget / (MT * seg * 4);
  const int segs = K / seg;
  return seg * (segs < max_segs ? segs : max_segs);
}

struct Int8Args {
  const float* x;
  const int8_t* q;
  const float* s;
  float* y;
  int M, N, K;
};

template <int MT, int V, int R>
void launch_int8(const Int8Args& a, hipStream_t st) {
  const int KC = pick_chunk(a.K, kWave * V, MT);
  const int rows_per_block = kWaves * R;
  hipLaunchKernelGGL((int8_gemv_fast<MT, V, R, true>), dim3((a.N + rows_per_block - 1) / rows_per_block),
                     dim3(kWaves * kWave), MT * KC * sizeof(float), st, a.x, a.q, a.s, a.y, a.M,
                     a.N, a.K, KC);
}

template <int MT, int V>
void launch_int8_r(int R, const Int8Args& a, hipStream_t st) {
  if constexpr (MT >= 8) {  // 4 rows x 8+ activation rows would not fit the register file
    if (R >= 2)
      launch_int8<MT, V, 2>(a, st);
    else
      launch_int8<MT, V, 1>(a, st);
  } else {
    if (R == 4)
      launch_int8<MT, V, 4>(a, st);
    else if (R == 2)
      launch_int8<MT, V, 2>(a, st);
    else
      launch_int8<MT, V, 1>(a, st);
  }
}

template <int MT>
void dispatch_int8(bool fast_ok, const Int8Args& a, hipStream_t st) {
  const int V = fast_ok ? pick_vec(a.K, 1, MT) : 0;
  if (V == 0) {
    hipLaunchKernelGGL(int8_gemv_generic<MT>, dim3((a.N + kWaves - 1) / kWaves),
                       dim3(kWaves * kWave), 0, st, a.x, a.q, a.s, a.y, a.M, a.N, a.K);
    return;
  }
  const int R = pick_rows(a.N, MT);
  if (V == 16)
    launch_int8_r<MT, 16>(R, a, st);
  else if (V == 8)
    launch_int8_r<MT, 8>(R, a, st);
  else
    launch_int8_r<MT, 4>(R, a, st);
}

struct Int4Args {
  const float* x;
  const float* inv;
  const uint8_t* nib;
  const float* gs;
  const float* gz;
  float* y;
  int M, N, K, group;
};

template <int MT, int V, int R>
void launch_int4(const Int4Args& a, hipStream_t st) {
  const int KC = pick_chunk(a.K, 2 * kWave * V, MT);
  const int rows_per_block = kWaves * R;
  hipLaunchKernelGGL((int4_gemv_fast<MT, V, R, true>), dim3((a.N + rows_per_block - 1) / rows_per_block),
                     dim3(kWaves * kWave), MT * KC * sizeof(float), st, a.x, a.inv, a.nib, a.gs,
                     a.gz, a.y, a.M, a.N, a.K, a.group, KC);
}

template <int MT, int V>
void launch_int4_r(int R, const Int4Args& a, hipStream_t st) {
  if constexpr (MT >= 8) {  // 4 rows x 8+ activation rows would not fit the register file
    if (R >= 2)
      launch_int4<MT, V, 2>(a, st);
    else
      launch_int4<MT, V, 1>(a, st);
  } else {
    if (R == 4)
      launch_int4<MT, V, 4>(a, st);
    else if (R == 2)
      launch_int4<MT, V, 2>(a, st);
    else
      launch_int4<MT, V, 1>(a, st);
  }
}

template <int MT>
void dispatch_int4(bool fast_ok, const Int4Args& a, hipStream_t st) {
  int V = fast_ok ? pick_vec(a.K / 2, 2, MT) : 0;
  // a lane slice (2V channels) must stay inside one quantization group
  while (V && a.group % (2 * V) != 0) V = (V == 4) ? 0 : V / 2;
  if (V && (a.K / 2) % (kWave * V) != 0) V = 0;
  if (V == 0) {
    hipLaunchKernelGGL(int4_gemv_generic<MT>, dim3((a.N + kWaves - 1) / kWaves),
                       dim3(kWaves * kWave), 0, st, a.x, a.inv, a.nib, a.gs, a.gz, a.y, a.M, a.N,
                       a.K, a.group);
    return;
  }
  const int R = pick_rows(a.N, MT);
  if (V == 16)
    launch_int4_r<MT, 16>(R, a, st);
  else if (V == 8)
    launch_int4_r<MT, 8>(R, a, st);
  else
    launch_int4_r<MT, 4>(R, a, st);
}

}  // namespace

extern "C" int llmserve_int8_linear(const float* x, const int8_t* q, const float* scale, float* y,
                                    int64_t M, int64_t N, int64_t K, void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 1, "int8_linear: bad shape M=%lld N=%lld K=%lld",
            (long long)M, (long long)N, (long long)K);
  LSH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int8_linear: meant for small batches (M <= 64)");
  LSH_CHECK(N < (1LL << 31) && K < (1LL << 31) && N * K < (1LL << 40),
            "int8_linear: shape too large");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(x && q && scale && y, "int8_linear: null pointer");
  hipStream_t st = lsh::as_stream(stream);
  const bool fast_ok = lsh::aligned16(x) && lsh::aligned16(q) && K % 16 == 0;
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int mt = static_cast<int>(M - m0 < 16 ? M - m0 : 16);
    const Int8Args a{x + m0 * K, q, scale, y + m0 * N, mt, static_cast<int>(N), static_cast<int>(K)};
    switch (pick_mt(mt)) {
      case 1: dispatch_int8<1>(fast_ok, a, st); break;
      case 2: dispatch_int8<2>(fast_ok, a, st); break;
      case 4: dispatch_int8<4>(fast_ok, a, st); break;
      case 8: dispatch_int8<8>(fast_ok, a, st); break;
      default: dispatch_int8<16>(fast_ok, a, st); break;
    }
    const int rc = lsh::launch_status("int8_linear");
    if (rc) return rc;
  }
  return LLMSERVE_OK;
}

extern "C" int llmserve_int4_linear(const float* x, const float* inv_act_scale,
                                    const uint8_t* nibbles, const float* g_scale,
                                    const float* g_zero, float* y, int64_t M, int64_t N, int64_t K,
                                    int64_t group_size, void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 1 && group_size >= 2, "int4: shapes");
  LSH_CHECK(K % group_size == 0 && group_size % 2 == 0, "int4: shapes");
  LSH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int4_linear: meant for small batches (M <= 64)");
  LSH_CHECK(N < (1LL << 31) && K < (1LL << 31) && N * K < (1LL << 41),
            "int4_linear: shape too large");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(x && nibbles && g_scale && g_zero && y, "int4_linear: null pointer");
  hipStream_t st = lsh::as_stream(stream);
  const bool fast_ok = lsh::aligned16(x) && lsh::aligned16(nibbles) && K % 32 == 0 &&
                       (inv_act_scale == nullptr || lsh::aligned16(inv_act_scale));
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int mt = static_cast<int>(M - m0 < 16 ? M - m0 : 16);
    const Int4Args a{x + m0 * K, inv_act_scale, nibbles, g_scale, g_zero, y + m0 * N, mt,
                     static_cast<int>(N), static_cast<int>(K), static_cast<int>(group_size)};
    switch (pick_mt(mt)) {
      case 1: dispatch_int4<1>(fast_ok, a, st); break;
      case 2: dispatch_int4<2>(fast_ok, a, st); break;
      case 4: dispatch_int4<4>(fast_ok, a, st); break;
      case 8: dispatch_int4<8>(fast_ok, a, st); break;
      default: dispatch_int4<16>(fast_ok, a, st); break;
    }
    const int rc = lsh::launch_status("int4_linear");
    if (rc) return rc;
  }
  return LLMSERVE_OK;
}
