// Weight-only int8 / int4 GEMV for decode (M <= 16 activation rows per launch; the host
// loops over row tiles up to the 64-row limit).
//
// Decode is bound by HBM and, at the Qwen3-0.6B layer sizes (1-6 MB per matrix), by the
// latency of one kernel: a plain read of 4 MB takes ~2.3 us on MI355X (a null kernel ~1.6 us),
// and it is fastest with many small wavefronts that each issue one 16-byte load per lane.
// The kernels are laid out for that:
//  * every lane loads 16 weight bytes per load (global_load_dwordx4, non-temporal): 16 int8
//    or 32 int4 input channels;
//  * LPR lanes (16, 32 or 64) cover LPR*16 bytes of one output row; a wavefront holds
//    64/LPR row slots, so one wave-level load reads 64/LPR consecutive rows = 1 KB of
//    contiguous weights when a row is LPR*16 bytes long;
//  * a wavefront owns R such row groups; a 256-thread workgroup is 4 wavefronts;
//  * the activations x (M x K fp32, a few KB) are staged once per workgroup in LDS (the
//    int4 AWQ pre-scale x * inv_act_scale is applied while staging) or, for M <= 2, read
//    directly from L1/L2; every row slot of the wave reuses the same x slice;
//  * partial sums are finished with xor-shuffles over the LPR lanes of a row.
// The int4 path uses the reference's group decomposition
//   y = sum_g s * sum_{k in g} x q + (z - 8 s) * sum_{k in g} x     (int8_gemv.cpp:48-52)
// per 32-channel lane slice, which always lies inside one quantization group (group % 32 == 0).
// Shapes the fast path cannot tile go to a generic kernel with scalar loads.
#include "common.h"

namespace {

using lsh::kWave;
constexpr int kWaves = 4;
constexpr int kLdsBudget = 64 * 1024;  // bytes of staged x per workgroup

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GemvArgs {
  const float* x;      // [M, K]
  const float* inv;    // [K] int4 AWQ pre-scale, or null
  const uint8_t* w;    // int8 [N, K] or nibbles [N, K/2]
  const float* s;      // int8: scale [N]; int4: g_scale [N, G]
  const float* z;      // int4: g_zero [N, G]
  float* y;            // [M, N]
  int M, N, K, group, KC;
};

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Channels 2b (low nibble) and 2b+1 (high nibble) of byte b, for the 4 bytes of u.
__device__ __forceinline__ void unpack_nibbles(uint32_t u, float (&q)[8]) {
  const uint32_t lo = u & 0x0f0f0f0fu, hi = (u >> 4) & 0x0f0f0f0fu;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    q[2 * b] = static_cast<float>((lo >> (8 * b)) & 0xffu);
    q[2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xffu);
  }
}

__device__ __forceinline__ void unpack_int8(uint32_t u, float (&q)[4]) {
#pragma unroll
  for (int b = 0; b < 4; ++b) q[b] = static_cast<float>(static_cast<int8_t>((u >> (8 * b)) & 0xffu));
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

// NX consecutive activations of row m from channel k: from the staged chunk (XLDS; the
// chunk starts at channel c0, row stride KC) or from global memory.
template <int NX, bool XLDS>
__device__ __forceinline__ void read_x(float (&xv)[NX], const float* xs, const GemvArgs& a, int m,
                                       int k, int c0) {
  if (XLDS) {
    const float4* p = reinterpret_cast<const float4*>(xs + m * a.KC + (k - c0));
#pragma unroll
    for (int i = 0; i < NX / 4; ++i) {
      const float4 v = p[i];
      xv[4 * i] = v.x;
      xv[4 * i + 1] = v.y;
      xv[4 * i + 2] = v.z;
      xv[4 * i + 3] = v.w;
    }
  } else {
    if (m >= a.M) {
#pragma unroll
      for (int i = 0; i < NX; ++i) xv[i] = 0.f;
      return;
    }
    const float4* p = reinterpret_cast<const float4*>(a.x + static_cast<int64_t>(m) * a.K + k);
    const float4* s = a.inv ? reinterpret_cast<const float4*>(a.inv + k) : nullptr;
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

// The fast GEMV. INT4 selects the nibble format. Requires: K a multiple of the segment
// (LPR * CPL channels), 16-byte aligned rows, and for int4 group % 32 == 0.
template <int MT, int LPR, int R, bool XLDS, bool INT4>
__global__ __launch_bounds__(256) void gemv_fast(GemvArgs a) {
  extern __shared__ float xs[];
  constexpr int RPW = kWave / LPR;         // row slots per wavefront
  constexpr int CPL = INT4 ? 32 : 16;      // input channels per lane per 16-byte load
  constexpr int SEGK = LPR * CPL;          // input channels per row segment
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int rs = lane / LPR, li = lane % LPR;
  const int row0 = (blockIdx.x * kWaves + wave) * R * RPW + rs;  // row of group r: row0 + r*RPW
  const int RB = INT4 ? a.K / 2 : a.K;
  const int nseg = a.K / SEGK;
  const int spc = a.KC / SEGK;  // segments per staged chunk
  const int G = INT4 ? a.K / a.group : 1;

  auto load_seg = [&](int j, u32x4 (&w)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r * RPW;
      w[r] = row < a.N ? load16(a.w + static_cast<int64_t>(row) * RB + j * LPR * 16 + li * 16)
                       : u32x4{0u, 0u, 0u, 0u};
    }
  };

  u32x4 w[R];
  load_seg(0, w);
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  int c0 = 0;
  for (int j = 0; j < nseg; ++j) {
    u32x4 wn[R];
    if (j + 1 < nseg) load_seg(j + 1, wn);
    const int k0 = j * SEGK + li * CPL;
    float sc[R], zc[R];
    if constexpr (INT4) {
      const int g = k0 / a.group;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r * RPW, a.N - 1);
        sc[r] = a.s[static_cast<int64_t>(row) * G + g];
        zc[r] = a.z[static_cast<int64_t>(row) * G + g] - 8.f * sc[r];
      }
    }
    if (XLDS && j % spc == 0) {
      c0 = j * SEGK;
      if (j) __syncthreads();
      stage_x<MT>(xs, a.x, INT4 ? a.inv : nullptr, a.M, a.K, c0, min(a.KC, a.K - c0), a.KC);
      __syncthreads();
    }
    if constexpr (!INT4) {
      float wf[R][16];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float t[4];
          unpack_int8(w[r][i], t);
#pragma unroll
          for (int b = 0; b < 4; ++b) wf[r][4 * i + b] = t[b];
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[16];
        read_x<16, XLDS>(xv, xs, a, m, k0, c0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float t = acc[r][m];
#pragma unroll
          for (int i = 0; i < 16; ++i) t += xv[i] * wf[r][i];
          acc[r][m] = t;
        }
      }
    } else if constexpr (MT <= 2) {
      // x slice read once per m; nibbles unpacked per (m, row)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[32];
        read_x<32, XLDS>(xv, xs, a, m, k0, c0);
        float xsum = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) xsum += xv[i];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float qf[8];
            unpack_nibbles(w[r][i], qf);
#pragma unroll
            for (int e = 0; e < 8; ++e) d += xv[8 * i + e] * qf[e];
          }
          acc[r][m] += sc[r] * d + zc[r] * xsum;
        }
      }
    } else {
      // nibbles unpacked once per row; x slice re-read from LDS per row
      float xsum[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[32];
        read_x<32, XLDS>(xv, xs, a, m, k0, c0);
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) t += xv[i];
        xsum[m] = t;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float qf[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float t[8];
          unpack_nibbles(w[r][i], t);
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[8 * i + e] = t[e];
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float xv[32];
          read_x<32, XLDS>(xv, xs, a, m, k0, c0);
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 32; ++i) d += xv[i] * qf[i];
          acc[r][m] += sc[r] * d + zc[r] * xsum[m];
        }
      }
    }
    if (j + 1 < nseg) {
#pragma unroll
      for (int r = 0; r < R; ++r) w[r] = wn[r];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r * RPW;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = lsh::group_sum<LPR>(acc[r][m]);
      if (li == 0 && m < a.M && row < a.N)
        a.y[static_cast<int64_t>(m) * a.N + row] = INT4 ? v : v * a.s[row];
    }
  }
}

// Any shape / alignment: one wavefront per output row, lanes stride over k with byte loads.
template <int MT, bool INT4>
__global__ __launch_bounds__(256) void gemv_generic(GemvArgs a) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= a.N) return;  // whole wave; no barriers in this kernel
  const int G = INT4 ? a.K / a.group : 1;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;
  for (int k = lane; k < a.K; k += kWave) {
    float wv, s = 1.f, c = 0.f;
    if constexpr (INT4) {
      const uint8_t b = a.w[static_cast<int64_t>(row) * (a.K / 2) + k / 2];
      wv = static_cast<float>((k & 1) ? (b >> 4) : (b & 0xf));
      const int g = k / a.group;
      s = a.s[static_cast<int64_t>(row) * G + g];
      c = a.z[static_cast<int64_t>(row) * G + g] - 8.f * s;
    } else {
      wv = static_cast<float>(reinterpret_cast<const int8_t*>(a.w)[static_cast<int64_t>(row) * a.K + k]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m < a.M) {
        float xv = a.x[static_cast<int64_t>(m) * a.K + k];
        if (INT4 && a.inv) xv = __fmul_rn(xv, a.inv[k]);
        acc[m] += INT4 ? s * (xv * wv) + c * xv : xv * wv;
      }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float v = lsh::wave_sum_from<1>(acc[m]);
    if (lane == 0 && m < a.M) a.y[static_cast<int64_t>(m) * a.N + row] = INT4 ? v : v * a.s[row];
  }
}

// ---------------------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------------------
struct Config {
  int lpr;     // lanes per row: 16, 32, 64 (0 = generic kernel)
  int rows;    // R: row groups per wavefront
  bool xlds;   // stage x in LDS
};

int pick_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// Fast-path tiling for a (bits, MT, N, K, group) problem; lpr = 0 when it cannot tile.
Config choose(bool int4, int MT, int N, int K, int group, bool aligned) {
  Config c{0, 1, true};
  if (!aligned || (int4 && group % 32 != 0)) return c;
  const int cpl = int4 ? 32 : 16;
  const int row_bytes = int4 ? K / 2 : K;
  for (int lpr : {64, 32, 16}) {
    if (row_bytes % (lpr * 16) != 0) continue;
    if (MT * lpr * cpl * 4 > kLdsBudget) continue;  // one staged segment must fit
    c.lpr = lpr;
    break;
  }
  if (c.lpr == 0) return c;
  // R = 2 only when there are wavefronts to spare (~4 per SIMD)
  const int rpw = kWave / c.lpr;
  const int waves = (N + rpw - 1) / rpw;
  c.rows = (MT <= 2 && waves >= 2 * 4096) ? 2 : 1;
  c.xlds = MT > 2 || (static_cast<int64_t>(MT) * K * 4 <= kLdsBudget);
  return c;
}

int pick_chunk(int K, int segk, int MT) {
  const int max_segs = kLdsBudget / (MT * segk * 4);
  const int segs = K / segk;
  return segk * (segs < max_segs ? segs : max_segs);
}

template <int MT, int LPR, int R, bool XLDS, bool INT4>
void launch_fast(GemvArgs a, hipStream_t st, bool last) {
  constexpr int SEGK = LPR * (INT4 ? 32 : 16);
  constexpr int rows_per_block = kWaves * R * (kWave / LPR);
  a.KC = XLDS ? pick_chunk(a.K, SEGK, MT) : SEGK;
  const size_t lds = XLDS ? static_cast<size_t>(MT) * a.KC * sizeof(float) : 0;
  lsh::launch(gemv_fast<MT, LPR, R, XLDS, INT4>, dim3((a.N + rows_per_block - 1) / rows_per_block),
              dim3(kWaves * kWave), lds, st, last, a);
}

template <int MT, int LPR, bool INT4>
void launch_lpr(const Config& c, const GemvArgs& a, hipStream_t st, bool last) {
  if constexpr (MT > 2) {  // x always staged; one row group (register budget)
    launch_fast<MT, LPR, 1, true, INT4>(a, st, last);
  } else {
    if (c.rows == 2) {
      if (c.xlds)
        launch_fast<MT, LPR, 2, true, INT4>(a, st, last);
      else
        launch_fast<MT, LPR, 2, false, INT4>(a, st, last);
    } else {
      if (c.xlds)
        launch_fast<MT, LPR, 1, true, INT4>(a, st, last);
      else
        launch_fast<MT, LPR, 1, false, INT4>(a, st, last);
    }
  }
}

template <int MT, bool INT4>
void launch_mt(const Config& c, const GemvArgs& a, hipStream_t st, bool last) {
  switch (c.lpr) {
    case 64: launch_lpr<MT, 64, INT4>(c, a, st, last); break;
    case 32: launch_lpr<MT, 32, INT4>(c, a, st, last); break;
    case 16: launch_lpr<MT, 16, INT4>(c, a, st, last); break;
    default:
      lsh::launch(gemv_generic<MT, INT4>, dim3((a.N + kWaves - 1) / kWaves), dim3(kWaves * kWave),
                  0, st, last, a);
  }
}

template <bool INT4>
int run_gemv(GemvArgs a, bool aligned, hipStream_t st, const char* what) {
  const int M = a.M;
  for (int m0 = 0; m0 < M; m0 += 16) {
    GemvArgs t = a;
    t.M = M - m0 < 16 ? M - m0 : 16;
    t.x = a.x + static_cast<int64_t>(m0) * a.K;
    t.y = a.y + static_cast<int64_t>(m0) * a.N;
    const int MT = pick_mt(t.M);
    const Config c = choose(INT4, MT, a.N, a.K, a.group, aligned);
    const bool last = m0 + 16 >= M;
    switch (MT) {
      case 1: launch_mt<1, INT4>(c, t, st, last); break;
      case 2: launch_mt<2, INT4>(c, t, st, last); break;
      case 4: launch_mt<4, INT4>(c, t, st, last); break;
      case 8: launch_mt<8, INT4>(c, t, st, last); break;
      default: launch_mt<16, INT4>(c, t, st, last); break;
    }
    const int rc = lsh::launch_status(what);
    if (rc) return rc;
  }
  return LLMSERVE_OK;
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
  GemvArgs a{x, nullptr, reinterpret_cast<const uint8_t*>(q), scale, nullptr, y,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), 1, 0};
  const bool aligned = lsh::aligned16(x) && lsh::aligned16(q) && K % 16 == 0;
  return run_gemv<false>(a, aligned, lsh::as_stream(stream), "int8_linear");
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
  GemvArgs a{x, inv_act_scale, nibbles, g_scale, g_zero, y, static_cast<int>(M),
             static_cast<int>(N), static_cast<int>(K), static_cast<int>(group_size), 0};
  const bool aligned = lsh::aligned16(x) && lsh::aligned16(nibbles) && K % 32 == 0 &&
                       (inv_act_scale == nullptr || lsh::aligned16(inv_act_scale));
  return run_gemv<true>(a, aligned, lsh::as_stream(stream), "int4_linear");
}
