// Fused elementwise kernels of the decoder layer (the reference's fused_ops.cpp:39-125:
// rmsnorm, add_rmsnorm_, silu_mul, rope_qk_) and the decode-step glue around them:
//  * the post-qkv decode kernel: per-head RMSNorm of q and k (Qwen3), rotate-half RoPE at each
//    sequence's position, q written contiguous for the attention kernel, k and v quantized
//    straight into the int8 KV cache (QuantizedKV.write, attention.py:153-162, with the
//    key-smoothing division) at the slot of the new token: one launch where the reference runs
//    rope_qk_, two index_copy_ writes and a copy of q;
//  * greedy next-token selection (argmax over the logits row, sampling.py:151-170 at
//    temperature 0) that also advances each sequence's context length by the new token.
// The reference's sum-of-squares loops are OpenMP simd reductions (any order); here they are
// trees over the wavefront / workgroup in a fixed order.
#include <initializer_list>

#include "common.h"
#include "kv_quant.h"
#include "rope.h"
#include "xfrag.h"

namespace {

using lsh::kWave;
constexpr int kRowThreads = 256;

// Sum over the 256 threads of the workgroup, in a fixed order; every thread gets it.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = lsh::wave_sum_from<1>(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// out = w * (x * inv), inv = 1 / sqrt(mean(x^2) + eps) (fused_ops.cpp:23-30). One workgroup
// per row. kNormAdd first does x += r in place (add_rmsnorm_, fused_ops.cpp:60-81);
// kNormGather first copies the embedding row r[ids[t]] into x (the embedding lookup of
// transformer.py:151 followed by its first rmsnorm, :155); an id outside [0, V) gives a NaN
// row, so that a bad token shows in the logits instead of reading out of bounds.
enum NormMode { kNormPlain = 0, kNormAdd = 1, kNormGather = 2 };

template <int MODE>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(float* __restrict__ x,
                                                              const float* __restrict__ r,
                                                              const int64_t* __restrict__ ids,
                                                              int64_t V,
                                                              const float* __restrict__ w,
                                                              float* __restrict__ out, int64_t H,
                                                              float eps) {
  __shared__ float red[kRowThreads / kWave];
  const int64_t t = blockIdx.x;
  float* xr = x + t * H;
  float* orow = out + t * H;
  const float* src = xr;
  bool bad = false;
  if (MODE == kNormGather) {
    const int64_t id = ids[t];
    bad = id < 0 || id >= V;
    src = r + (bad ? 0 : id) * H;
  }
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += kRowThreads) {
    float v = src[i];
    if (MODE == kNormAdd) v += r[t * H + i];
    if (MODE == kNormGather && bad) v = __builtin_nanf("");
    if (MODE != kNormPlain) xr[i] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(H) + eps);
  for (int64_t i = threadIdx.x; i < H; i += kRowThreads) orow[i] = w[i] * (xr[i] * inv);
}

// The norms above, vectorized (rows of H % 4 == 0 channels, 16-byte aligned, H <= 4 * 256 * NC):
// thread i holds channels 4 (i + 256 j) .. + 4, j < NC, in registers from the loads to the
// output, and every load of the row (x or the embedding row, the residual's PL planes, w and
// act_inv) is issued before the first use, so the row costs one memory round trip instead of
// one per channel group and plane. The arithmetic per channel is rmsnorm_kernel's (planes
// added in order, then to x); the sum of squares runs over the thread's channels in index
// order, then block_sum.
constexpr int kNormChunk = 4 * kRowThreads;  // channels per round of the threads (1024)
constexpr int kNormMaxH = 4 * kNormChunk;     // rows the vectorized norms take (NC <= 4)

constexpr int kPlaneGroup = 4;  // residual planes loaded together

template <int MODE, int NC>
__device__ __forceinline__ float norm_vec_pass(float* xr, const float* src, const float* rrow,
                                               int64_t pstride, int planes, bool bad,
                                               const float* w, const float* act, int H,
                                               float4 (&v)[NC], float4 (&wv)[NC],
                                               float4 (&av)[NC], bool (&on)[NC]) {
  const int n4 = H / 4;
  int cc[NC];
  float4 rp[NC][kPlaneGroup];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = static_cast<int>(threadIdx.x) + kRowThreads * j;
    on[j] = c < n4;
    cc[j] = on[j] ? c : n4 - 1;  // clamped: the loads stay unconditional
    v[j] = reinterpret_cast<const float4*>(src)[cc[j]];
    wv[j] = reinterpret_cast<const float4*>(w)[cc[j]];
    av[j] = reinterpret_cast<const float4*>(act ? act : w)[cc[j]];  // act null: unused
    if constexpr (MODE == kNormAdd) {
#pragma unroll
      for (int q = 0; q < kPlaneGroup; ++q)  // planes past the last repeat it (not added)
        rp[j][q] = reinterpret_cast<const float4*>(
            rrow + static_cast<int64_t>(q < planes ? q : planes - 1) * pstride)[cc[j]];
    }
  }
  float4 rs[NC];
  if constexpr (MODE == kNormAdd) {
    auto add4 = [](float4& a, const float4& b) {
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    };
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      rs[j] = rp[j][0];
#pragma unroll
      for (int q = 1; q < kPlaneGroup; ++q)
        if (q < planes) add4(rs[j], rp[j][q]);
    }
    for (int p0 = kPlaneGroup; p0 < planes; p0 += kPlaneGroup) {  // more than 4 planes
#pragma unroll
      for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int q = 0; q < kPlaneGroup; ++q)
          rp[j][q] = reinterpret_cast<const float4*>(
              rrow + static_cast<int64_t>(p0 + q < planes ? p0 + q : planes - 1) * pstride)[cc[j]];
#pragma unroll
      for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int q = 0; q < kPlaneGroup; ++q)
          if (p0 + q < planes) add4(rs[j], rp[j][q]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    float4 x = v[j];
    if constexpr (MODE == kNormAdd) {
      x.x += rs[j].x;
      x.y += rs[j].y;
      x.z += rs[j].z;
      x.w += rs[j].w;
    }
    if (MODE == kNormGather && bad) {
      const float nan = __builtin_nanf("");
      x = make_float4(nan, nan, nan, nan);
    }
    v[j] = x;
    if (on[j]) {
      if constexpr (MODE != kNormPlain)
        reinterpret_cast<float4*>(xr)[threadIdx.x + kRowThreads * j] = x;
      ss = __builtin_fmaf(x.x, x.x, ss);  // explicit fmas: the order cannot be contracted
      ss = __builtin_fmaf(x.y, x.y, ss);  // differently in the kernels that share this pass
      ss = __builtin_fmaf(x.z, x.z, ss);
      ss = __builtin_fmaf(x.w, x.w, ss);
    }
  }
  return ss;
}

template <int MODE, int NC>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_vec_kernel(float* __restrict__ x,
                                                                  const float* __restrict__ r,
                                                                  const int64_t* __restrict__ ids,
                                                                  int64_t V,
                                                                  const float* __restrict__ w,
                                                                  float* __restrict__ out, int H,
                                                                  float eps) {
  __shared__ float red[kRowThreads / kWave];
  const int64_t t = blockIdx.x;
  float* xr = x + t * H;
  const float* src = xr;
  const float* rrow = r ? r + t * H : nullptr;
  bool bad = false;
  if (MODE == kNormGather) {
    const int64_t id = ids[t];
    bad = id < 0 || id >= V;
    src = r + (bad ? 0 : id) * H;
  }
  float4 v[NC], wv[NC], av[NC];
  bool on[NC];
  float ss = norm_vec_pass<MODE, NC>(xr, src, rrow, 0, 1, bad, w, nullptr, H, v, wv, av, on);
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(H) + eps);
  float4* orow = reinterpret_cast<float4*>(out + t * H);
#pragma unroll
  for (int j = 0; j < NC; ++j)
    if (on[j])
      orow[threadIdx.x + kRowThreads * j] =
          make_float4(wv[j].x * (v[j].x * inv), wv[j].y * (v[j].y * inv), wv[j].z * (v[j].z * inv),
                      wv[j].w * (v[j].w * inv));
}

// out[t, i] = silu(gate) * up = gate / (1 + exp(-gate)) * up for a fused [T, 2I] gate|up row
// (fused_ops.cpp:83-99).
__global__ __launch_bounds__(kRowThreads) void silu_mul_kernel(const float* __restrict__ gu,
                                                               float* __restrict__ out, int64_t T,
                                                               int64_t I) {
  const int64_t n = T * I;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowThreads;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x; e < n; e += stride) {
    const int64_t t = e / I, i = e - t * I;
    const float g = gu[t * 2 * I + i], u = gu[t * 2 * I + I + i];
    out[e] = g / (1.f + expf(-g)) * u;
  }
}

// rmsnorm_kernel's arithmetic with the fragments as output, one channel per thread and
// round: the form for rows that rmsnorm_frag_kernel does not take (H above kNormMaxH or
// unaligned rows). Same x update, same sum of squares and inv as rmsnorm_kernel.
template <int MODE>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_frag_scalar_kernel(
    float* __restrict__ x, const float* __restrict__ r, const int64_t* __restrict__ ids, int64_t V,
    const float* __restrict__ w, const float* __restrict__ act_inv, __bf16* __restrict__ xf,
    float* __restrict__ xsum, int T, int H, int mp, float eps, int planes) {
  __shared__ float red[kRowThreads / kWave];
  const int t = blockIdx.x;
  const int nblk = H / lsh::kFragBlk;
  if (t >= T) {  // padding row of the last 16-row tile
    for (int c0 = 4 * threadIdx.x; c0 < H; c0 += 4 * kRowThreads) {
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
      lsh::frag_store<4>(xf, t, c0, nblk, z);
      if (threadIdx.x % 32 == 0) xsum[static_cast<int64_t>(c0 / lsh::kFragBlk) * mp + t] = 0.f;
    }
    return;
  }
  float* xr = x + static_cast<int64_t>(t) * H;
  const float* src = xr;
  bool bad = false;
  if (MODE == kNormGather) {
    const int64_t id = ids[t];
    bad = id < 0 || id >= V;
    src = r + (bad ? 0 : id) * H;
  }
  float ss = 0.f;
  const int64_t pstride = static_cast<int64_t>(T) * H;
  for (int i = threadIdx.x; i < H; i += kRowThreads) {
    float v = src[i];
    if (MODE == kNormAdd) {
      float rs = r[static_cast<int64_t>(t) * H + i];
      for (int p = 1; p < planes; ++p) rs += r[p * pstride + static_cast<int64_t>(t) * H + i];
      v += rs;
    }
    if (MODE == kNormGather && bad) v = __builtin_nanf("");
    if (MODE != kNormPlain) xr[i] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum(ss, red);  // its barriers also order the x writes above before the reads below
  const float inv = 1.f / sqrtf(ss / static_cast<float>(H) + eps);
  for (int c0 = 4 * threadIdx.x; c0 < H; c0 += 4 * kRowThreads) {
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h = w[c0 + e] * (xr[c0 + e] * inv);
      v[e] = act_inv ? __fmul_rn(h, act_inv[c0 + e]) : h;
    }
    lsh::frag_store<4>(xf, t, c0, nblk, v);
    const float sblk = lsh::group_sum<32>(lsh::tree_sum<4>(v));
    if (threadIdx.x % 32 == 0) xsum[static_cast<int64_t>(c0 / lsh::kFragBlk) * mp + t] = sblk;
  }
}

// The norms above with the int4 linear's activation fragments as output (xfrag.h): the
// first pass is rmsnorm_vec_kernel's (norm_vec_pass: same x update, same sum of squares, same
// inv); the second computes h = w * (x * inv) as it does, x' = h * act_inv (the next linear's
// AWQ pre-scale, or h) and writes x' as bf16 hi / mid / lo fragments and block sums, with 4
// consecutive channels per thread (32 threads per 128-channel block). One workgroup per
// fragment row: rows past T write zeros. H is a multiple of 128, at most 1024 NC. The residual
// r may come as `planes` partial sums [planes, T, H] (a K-split linear's output planes): they
// are added in plane order, then to x.
template <int MODE, int NC>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_frag_kernel(
    float* __restrict__ x, const float* __restrict__ r, const int64_t* __restrict__ ids, int64_t V,
    const float* __restrict__ w, const float* __restrict__ act_inv, __bf16* __restrict__ xf,
    float* __restrict__ xsum, int T, int H, int mp, float eps, int planes) {
  __shared__ float red[kRowThreads / kWave];
  const int t = blockIdx.x;
  const int nblk = H / lsh::kFragBlk;
  if (t >= T) {  // padding row of the last 16-row tile
    for (int c0 = 4 * threadIdx.x; c0 < H; c0 += 4 * kRowThreads) {
      const float z[4] = {0.f, 0.f, 0.f, 0.f};
      lsh::frag_store<4>(xf, t, c0, nblk, z);
      if (threadIdx.x % 32 == 0) xsum[static_cast<int64_t>(c0 / lsh::kFragBlk) * mp + t] = 0.f;
    }
    return;
  }
  float* xr = x + static_cast<int64_t>(t) * H;
  const float* src = xr;
  const float* rrow = r ? r + static_cast<int64_t>(t) * H : nullptr;
  bool bad = false;
  if (MODE == kNormGather) {
    const int64_t id = ids[t];
    bad = id < 0 || id >= V;
    src = r + (bad ? 0 : id) * H;
  }
  float4 v[NC], wv[NC], av[NC];
  bool on[NC];
  float ss = norm_vec_pass<MODE, NC>(xr, src, rrow, static_cast<int64_t>(T) * H, planes, bad, w,
                                      act_inv, H, v, wv, av, on);
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(H) + eps);
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (!on[j]) continue;  // H % 128 == 0: whole 32-lane groups agree
    const int c0 = 4 * (static_cast<int>(threadIdx.x) + kRowThreads * j);
    const float hx[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    const float wx[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
    const float ax[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h = wx[e] * (hx[e] * inv);
      o[e] = act_inv ? __fmul_rn(h, ax[e]) : h;
    }
    lsh::frag_store<4>(xf, t, c0, nblk, o);
    const float sblk = lsh::group_sum<32>(lsh::tree_sum<4>(o));
    if (threadIdx.x % 32 == 0) xsum[static_cast<int64_t>(c0 / lsh::kFragBlk) * mp + t] = sblk;
  }
}

// silu(gate) * up (silu_mul_kernel's arithmetic) times the next linear's AWQ pre-scale, as
// fragments and block sums. One wavefront per (fragment row, block), two channels per lane;
// rows past T write zeros.
__global__ __launch_bounds__(kRowThreads) void silu_mul_frag_kernel(
    const float* __restrict__ gu, const float* __restrict__ act_inv, __bf16* __restrict__ xf,
    float* __restrict__ xsum, int T, int I, int mp) {
  const int nblk = I / lsh::kFragBlk;
  const int item = blockIdx.x * (kRowThreads / kWave) + threadIdx.x / kWave;
  if (item >= mp * nblk) return;  // whole wavefront
  const int t = item / nblk, b = item % nblk;
  const int lane = threadIdx.x % kWave;
  const int c = lsh::kFragBlk * b + 2 * lane;
  float v[2] = {0.f, 0.f};
  if (t < T) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float g = gu[static_cast<int64_t>(t) * 2 * I + c + e];
      const float u = gu[static_cast<int64_t>(t) * 2 * I + I + c + e];
      const float a = g / (1.f + expf(-g)) * u;
      v[e] = act_inv ? __fmul_rn(a, act_inv[c + e]) : a;
    }
  }
  lsh::frag_store<2>(xf, t, c, nblk, v);
  const float sblk = lsh::group_sum<64>(lsh::tree_sum<2>(v));
  if (lane == 0) xsum[static_cast<int64_t>(b) * mp + t] = sblk;
}

struct RopeArgs {
  float* qkv;                 // [T, row_stride] floats: n_q q heads, n_k k heads, n_k v heads
  int64_t row_stride;
  const float* cos;           // rows of D: per token (rope_qk_) or per position (decode)
  const float* sin;
  const float* q_w;           // [D] per-head RMSNorm weights, or null
  const float* k_w;
  float eps;
  int T, n_q, n_k, D;
  // decode: position of token t = context_lens[t] - 1 (its cos/sin row and cache slot)
  const int64_t* ctx;
  const int64_t* bt;          // [T, max_blocks]
  int64_t max_blocks, bs, num_slots, max_pos;
  const float* smooth;        // [n_k, D] key smoothing, or null
  float* q_out;               // [T, n_q, D]
  int8_t* kc;                 // [num_slots, n_k, D]
  int8_t* vc;
  float* ks;                  // [num_slots, n_k]
  float* vs;
};

template <int N, bool DECODE>
__global__ __launch_bounds__(kRowThreads) void rope_kernel(RopeArgs a) {
  const int lane = threadIdx.x % kWave;
  const int heads = DECODE ? a.n_q + 2 * a.n_k : a.n_q + a.n_k;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * (kRowThreads / kWave) + threadIdx.x / kWave;
  if (gid >= static_cast<int64_t>(a.T) * heads) return;  // whole wavefront
  const int t = static_cast<int>(gid / heads), hh = static_cast<int>(gid % heads);
  float* row = a.qkv + t * a.row_stride + static_cast<int64_t>(hh) * a.D;
  float v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int d = lane + i * kWave;
    v[i] = d < a.D ? row[d] : 0.f;
  }
  int64_t cs_row = t, slot = -1;
  if constexpr (DECODE) {
    const int64_t pos = a.ctx[t] - 1;
    if (pos < 0 || pos >= a.max_pos || pos / a.bs >= a.max_blocks) return;
    cs_row = pos;
    const int64_t blk = a.bt[t * a.max_blocks + pos / a.bs];
    slot = blk * a.bs + pos % a.bs;
    if (blk < 0 || slot >= a.num_slots) slot = -1;
  }
  const bool is_q = hh < a.n_q, is_k = !is_q && hh < a.n_q + a.n_k;
  if (is_q || is_k)
    lsh::norm_rope(v, is_q ? a.q_w : a.k_w, a.cos + cs_row * a.D, a.sin + cs_row * a.D, a.D, a.eps);
  if constexpr (!DECODE) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int d = lane + i * kWave;
      if (d < a.D) row[d] = v[i];
    }
  } else {
    if (is_q) {
      float* o = a.q_out + (static_cast<int64_t>(t) * a.n_q + hh) * a.D;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int d = lane + i * kWave;
        if (d < a.D) o[d] = v[i];
      }
    } else if (slot >= 0) {
      const int h = is_k ? hh - a.n_q : hh - a.n_q - a.n_k;
      const int64_t at = slot * a.n_k + h;
      if (is_k)
        lsh::kv_quant_row(v, a.smooth ? a.smooth + static_cast<int64_t>(h) * a.D : nullptr, a.D,
                          a.kc + at * a.D, a.ks + at);
      else
        lsh::kv_quant_row(v, nullptr, a.D, a.vc + at * a.D, a.vs + at);
    }
  }
}

// Greedy selection in two launches: argmax_parts splits each logits row into kArgParts
// ranges (kArgParts workgroups per row, so the 64-row batch covers the GPU) and writes each
// range's (max, first index of the max); argmax_finish picks the best range per row (larger
// value, then smaller index: the first index among equal maxima), writes next_ids[t] and
// advances context_lens[t] by the new token. NaN orders above every number, as in
// torch.argmax (the reference's greedy path), so the first NaN of a row is selected.

constexpr int kArgParts = 32;

// x ranks above y: NaN above every number, else the larger value
__device__ __forceinline__ bool arg_above(float x, float y) {
  return x > y || (__builtin_isnan(x) && !__builtin_isnan(y));
}

// the higher-ranked value wins, then the smaller index
__device__ __forceinline__ void arg_better(float& best, int64_t& idx, float ob, int64_t oi) {
  const bool same = ob == best || (__builtin_isnan(ob) && __builtin_isnan(best));
  if (arg_above(ob, best) || (same && oi < idx)) {
    best = ob;
    idx = oi;
  }
}

__global__ __launch_bounds__(kRowThreads) void argmax_parts_kernel(const float* __restrict__ logits,
                                                                   int64_t V,
                                                                   float* __restrict__ part_v,
                                                                   int64_t* __restrict__ part_i) {
  __shared__ float bv[kRowThreads / kWave];
  __shared__ int64_t bi[kRowThreads / kWave];
  const int64_t t = blockIdx.x / kArgParts;
  const int part = blockIdx.x % kArgParts;
  const int64_t per = (V + kArgParts - 1) / kArgParts;
  const int64_t lo = part * per, hi = lo + per < V ? lo + per : V;
  const float* row = logits + t * V;
  float best = -__builtin_inff();
  int64_t idx = V;  // none
  // kArgUnroll loads (clamped into the range, so that all of them go out before the first
  // compare) per round: one memory round trip per round rather than one per element
  constexpr int kArgUnroll = 16;
  for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += kArgUnroll * kRowThreads) {
    float x[kArgUnroll];
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kRowThreads;
      x[u] = row[i < hi ? i : hi - 1];
    }
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kRowThreads;
      if (i < hi && arg_above(x[u], best)) {  // strictly above: the first index of equal values stays
        best = x[u];
        idx = i;
      }
    }
  }
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) arg_better(best, idx, __shfl_xor(best, d, kWave), __shfl_xor(idx, d, kWave));
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kRowThreads / kWave; ++k) arg_better(best, idx, bv[k], bi[k]);
    part_v[blockIdx.x] = best;
    part_i[blockIdx.x] = idx;
  }
}

__global__ __launch_bounds__(kWave) void argmax_finish_kernel(const float* __restrict__ part_v,
                                                              const int64_t* __restrict__ part_i,
                                                              int64_t V, int64_t* __restrict__ next_ids,
                                                              int64_t* __restrict__ ctx) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  float best = -__builtin_inff();
  int64_t idx = V;
  if (lane < kArgParts) {
    best = part_v[t * kArgParts + lane];
    idx = part_i[t * kArgParts + lane];
  }
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) arg_better(best, idx, __shfl_xor(best, d, kWave), __shfl_xor(idx, d, kWave));
  if (lane == 0) {
    next_ids[t] = idx < V ? idx : 0;
    ctx[t] += 1;
  }
}

int rope_slots(int64_t D) { return D <= kWave ? 1 : static_cast<int>((D + kWave - 1) / kWave); }

template <bool DECODE>
int launch_rope(const RopeArgs& a, hipStream_t st) {
  const int heads = DECODE ? a.n_q + 2 * a.n_k : a.n_q + a.n_k;
  const int64_t waves = static_cast<int64_t>(a.T) * heads;
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4)), block(kRowThreads);
  switch (rope_slots(a.D)) {
    case 1: lsh::launch(rope_kernel<1, DECODE>, grid, block, 0, st, true, a); break;
    case 2: lsh::launch(rope_kernel<2, DECODE>, grid, block, 0, st, true, a); break;
    default: lsh::launch(rope_kernel<4, DECODE>, grid, block, 0, st, true, a); break;
  }
  return LLMSERVE_OK;
}

// The vectorized norms take rows of H % 4 == 0 channels up to kNormMaxH with 16-byte aligned
// pointers (thread chunks of 4 channels); anything else runs the one-channel-per-thread form.
// Both forms of a norm with fragments and without agree bit for bit for the same rows.
bool norm_vec_ok(int64_t H, std::initializer_list<const void*> ptrs) {
  if (H % 4 != 0 || H > kNormMaxH) return false;
  for (const void* p : ptrs)
    if (p != nullptr && !lsh::aligned16(p)) return false;
  return true;
}

// the chunk count (template NC) of the vectorized norms for H <= kNormMaxH
int norm_chunks(int64_t H) { return H <= kNormChunk ? 1 : (H <= 2 * kNormChunk ? 2 : 4); }

template <int MODE>
void launch_norm(float* x, const float* r, const int64_t* ids, int64_t V, const float* w,
                 float* out, int64_t T, int64_t H, float eps, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(T)), block(kRowThreads);
  if (!norm_vec_ok(H, {x, r, w, out})) {
    lsh::launch(rmsnorm_kernel<MODE>, grid, block, 0, st, true, x, r, ids, V, w, out, H, eps);
    return;
  }
  const int Hi = static_cast<int>(H);
  switch (norm_chunks(H)) {
    case 1: lsh::launch(rmsnorm_vec_kernel<MODE, 1>, grid, block, 0, st, true, x, r, ids, V, w, out, Hi, eps); break;
    case 2: lsh::launch(rmsnorm_vec_kernel<MODE, 2>, grid, block, 0, st, true, x, r, ids, V, w, out, Hi, eps); break;
    default: lsh::launch(rmsnorm_vec_kernel<MODE, 4>, grid, block, 0, st, true, x, r, ids, V, w, out, Hi, eps); break;
  }
}

bool head_dim_ok(int64_t D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

}  // namespace

extern "C" int llmserve_rmsnorm(const float* x, const float* w, float* out, int64_t T, int64_t H,
                                float eps, void* stream) {
  LSH_CHECK(T >= 0 && H >= 1 && T < (1LL << 31), "rmsnorm: bad shape T=%lld H=%lld", (long long)T,
            (long long)H);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(x && w && out, "rmsnorm: null pointer");
  launch_norm<kNormPlain>(const_cast<float*>(x), nullptr, nullptr, 0, w, out, T, H, eps,
                          lsh::as_stream(stream));
  return lsh::launch_status("rmsnorm");
}

extern "C" int llmserve_add_rmsnorm(float* x, const float* r, const float* w, float* out,
                                    int64_t T, int64_t H, float eps, void* stream) {
  LSH_CHECK(T >= 0 && H >= 1 && T < (1LL << 31), "add_rmsnorm: bad shape T=%lld H=%lld",
            (long long)T, (long long)H);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(x && r && w && out, "add_rmsnorm: null pointer");
  launch_norm<kNormAdd>(x, r, nullptr, 0, w, out, T, H, eps, lsh::as_stream(stream));
  return lsh::launch_status("add_rmsnorm");
}

extern "C" int llmserve_embed_rmsnorm(const int64_t* ids, const float* embed, int64_t V,
                                      const float* w, float* x, float* out, int64_t T, int64_t H,
                                      float eps, void* stream) {
  LSH_CHECK(T >= 0 && H >= 1 && V >= 1 && T < (1LL << 31),
            "embed_rmsnorm: bad shape T=%lld H=%lld V=%lld", (long long)T, (long long)H,
            (long long)V);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(ids && embed && w && x && out, "embed_rmsnorm: null pointer");
  launch_norm<kNormGather>(x, embed, ids, V, w, out, T, H, eps, lsh::as_stream(stream));
  return lsh::launch_status("embed_rmsnorm");
}

extern "C" int llmserve_silu_mul(const float* gate_up, float* out, int64_t T, int64_t I,
                                 void* stream) {
  LSH_CHECK(T >= 0 && I >= 1, "silu_mul: bad shape T=%lld I=%lld", (long long)T, (long long)I);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(gate_up && out, "silu_mul: null pointer");
  const int64_t n = T * I;
  const int64_t blocks = (n + kRowThreads - 1) / kRowThreads;
  lsh::launch(silu_mul_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
              dim3(kRowThreads), 0, lsh::as_stream(stream), true, gate_up, out, T, I);
  return lsh::launch_status("silu_mul");
}

extern "C" int llmserve_rope_qk(float* qkv, const float* cos, const float* sin, int64_t T,
                                int64_t row_stride, int64_t n_q, int64_t n_k, int64_t D,
                                const float* q_w, const float* k_w, float eps, void* stream) {
  LSH_CHECK(T >= 0 && n_q >= 0 && n_k >= 0 && head_dim_ok(D),
            "rope_qk_: bad shape (head_dim %lld not in {16, 32, 64, 128, 256})", (long long)D);
  LSH_CHECK(row_stride >= (n_q + n_k) * D, "rope_qk_: bad shapes");
  LSH_CHECK(T < (1LL << 31) && n_q + n_k < 65536, "rope_qk_: too large");
  if (T == 0 || n_q + n_k == 0) return LLMSERVE_OK;
  LSH_CHECK(qkv && cos && sin, "rope_qk_: null pointer");
  RopeArgs a{};
  a.qkv = qkv;
  a.row_stride = row_stride;
  a.cos = cos;
  a.sin = sin;
  a.q_w = q_w;
  a.k_w = k_w;
  a.eps = eps;
  a.T = static_cast<int>(T);
  a.n_q = static_cast<int>(n_q);
  a.n_k = static_cast<int>(n_k);
  a.D = static_cast<int>(D);
  launch_rope<false>(a, lsh::as_stream(stream));
  return lsh::launch_status("rope_qk_");
}

extern "C" int llmserve_decode_qkv_kv(
    const float* qkv, int64_t row_stride, const float* cos_table, const float* sin_table,
    int64_t max_pos, const int64_t* context_lens, const int64_t* block_tables, int64_t max_blocks,
    int64_t block_size, const float* q_w, const float* k_w, float eps, const float* k_smooth,
    float* q_out, int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
    int64_t num_slots, int64_t T, int64_t n_q, int64_t n_k, int64_t D, void* stream) {
  LSH_CHECK(T >= 0 && n_q >= 1 && n_k >= 1 && head_dim_ok(D),
            "decode_qkv_kv: bad shape (head_dim %lld not in {16, 32, 64, 128, 256})",
            (long long)D);
  LSH_CHECK(row_stride >= (n_q + 2 * n_k) * D, "decode_qkv_kv: qkv rows too short");
  LSH_CHECK(block_size >= 1 && max_blocks >= 1 && num_slots >= 0 && max_pos >= 1,
            "decode_qkv_kv: bad cache shape");
  LSH_CHECK(T < (1LL << 31) && n_q + 2 * n_k < 65536, "decode_qkv_kv: too large");
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(qkv && cos_table && sin_table && context_lens && block_tables && q_out && k_cache &&
                v_cache && k_scale && v_scale,
            "decode_qkv_kv: null pointer");
  RopeArgs a{};
  a.qkv = const_cast<float*>(qkv);
  a.row_stride = row_stride;
  a.cos = cos_table;
  a.sin = sin_table;
  a.q_w = q_w;
  a.k_w = k_w;
  a.eps = eps;
  a.T = static_cast<int>(T);
  a.n_q = static_cast<int>(n_q);
  a.n_k = static_cast<int>(n_k);
  a.D = static_cast<int>(D);
  a.ctx = context_lens;
  a.bt = block_tables;
  a.max_blocks = max_blocks;
  a.bs = block_size;
  a.num_slots = num_slots;
  a.max_pos = max_pos;
  a.smooth = k_smooth;
  a.q_out = q_out;
  a.kc = k_cache;
  a.vc = v_cache;
  a.ks = k_scale;
  a.vs = v_scale;
  launch_rope<true>(a, lsh::as_stream(stream));
  return lsh::launch_status("decode_qkv_kv");
}

extern "C" int64_t llmserve_argmax_advance_workspace_bytes(int64_t T) {
  return T > 0 ? T * kArgParts * static_cast<int64_t>(sizeof(float) + sizeof(int64_t)) : 0;
}

extern "C" int llmserve_argmax_advance(const float* logits, int64_t T, int64_t V,
                                       int64_t* next_ids, int64_t* context_lens, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  LSH_CHECK(T >= 0 && V >= 1 && T < (1LL << 24), "argmax_advance: bad shape");
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(logits && next_ids && context_lens, "argmax_advance: null pointer");
  LSH_CHECK(workspace != nullptr && workspace_bytes >= llmserve_argmax_advance_workspace_bytes(T) &&
                lsh::aligned16(workspace),
            "argmax_advance: a 16-byte aligned workspace of %lld bytes is needed",
            (long long)llmserve_argmax_advance_workspace_bytes(T));
  int64_t* part_i = static_cast<int64_t*>(workspace);
  float* part_v = reinterpret_cast<float*>(part_i + T * kArgParts);
  hipStream_t st = lsh::as_stream(stream);
  lsh::launch(argmax_parts_kernel, dim3(static_cast<unsigned>(T * kArgParts)), dim3(kRowThreads), 0,
              st, false, logits, V, part_v, part_i);
  lsh::launch(argmax_finish_kernel, dim3(static_cast<unsigned>(T)), dim3(kWave), 0, st, true,
              part_v, part_i, V, next_ids, context_lens);
  return lsh::launch_status("argmax_advance");
}

// ---- producers of the int4 linear's activation fragments -------------------------------------

namespace {

int launch_norm_frag(int mode, float* x, const float* r, const int64_t* ids, int64_t V,
                     const float* w, const float* act_inv, void* xfrag, int64_t T, int64_t H,
                     float eps, void* stream, const char* what, int planes = 1) {
  LSH_CHECK(T >= 0 && H >= lsh::kFragBlk && H % lsh::kFragBlk == 0 && T < (1LL << 24) &&
                H < (1LL << 24),
            "%s: T=%lld, H=%lld (H a multiple of 128)", what, (long long)T, (long long)H);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(x && w && xfrag && (mode != kNormAdd || r) && (mode != kNormGather || (ids && r)),
            "%s: null pointer", what);
  LSH_CHECK(lsh::aligned16(xfrag), "%s: the fragment buffer must be 16-byte aligned", what);
  const int mp = static_cast<int>(lsh::frag_rows(T));
  __bf16* xf = static_cast<__bf16*>(xfrag);
  float* xsum = lsh::frag_sums(xf, mp, H);
  const dim3 grid(static_cast<unsigned>(mp)), block(kRowThreads);
  hipStream_t st = lsh::as_stream(stream);
  const int Ti = static_cast<int>(T), Hi = static_cast<int>(H);
  const int pl = mode == kNormAdd ? planes : 1;
  if (!norm_vec_ok(H, {x, r, w, act_inv})) {
    switch (mode) {
      case kNormAdd:
        lsh::launch(rmsnorm_frag_scalar_kernel<kNormAdd>, grid, block, 0, st, true, x, r, ids, V, w,
                    act_inv, xf, xsum, Ti, Hi, mp, eps, pl);
        break;
      case kNormGather:
        lsh::launch(rmsnorm_frag_scalar_kernel<kNormGather>, grid, block, 0, st, true, x, r, ids, V,
                    w, act_inv, xf, xsum, Ti, Hi, mp, eps, pl);
        break;
      default:
        lsh::launch(rmsnorm_frag_scalar_kernel<kNormPlain>, grid, block, 0, st, true, x, r, ids, V,
                    w, act_inv, xf, xsum, Ti, Hi, mp, eps, pl);
        break;
    }
    return lsh::launch_status(what);
  }
#define LSH_NF(m, nc)                                                                          \
  lsh::launch(rmsnorm_frag_kernel<m, nc>, grid, block, 0, st, true, x, r, ids, V, w, act_inv, xf, \
              xsum, Ti, Hi, mp, eps, pl)
#define LSH_NF_MODE(m)                  \
  switch (norm_chunks(H)) {             \
    case 1: LSH_NF(m, 1); break;        \
    case 2: LSH_NF(m, 2); break;        \
    default: LSH_NF(m, 4); break;       \
  }
  switch (mode) {
    case kNormAdd: LSH_NF_MODE(kNormAdd) break;
    case kNormGather: LSH_NF_MODE(kNormGather) break;
    default: LSH_NF_MODE(kNormPlain) break;
  }
#undef LSH_NF_MODE
#undef LSH_NF
  return lsh::launch_status(what);
}

}  // namespace

extern "C" int llmserve_rmsnorm_xfrag(const float* x, const float* w, const float* act_inv,
                                      void* xfrag, int64_t T, int64_t H, float eps,
                                      void* stream) {
  return launch_norm_frag(kNormPlain, const_cast<float*>(x), nullptr, nullptr, 0, w, act_inv, xfrag,
                          T, H, eps, stream, "rmsnorm_xfrag");
}

extern "C" int llmserve_add_rmsnorm_xfrag(float* x, const float* r, const float* w,
                                          const float* act_inv, void* xfrag, int64_t T, int64_t H,
                                          float eps, void* stream) {
  return launch_norm_frag(kNormAdd, x, r, nullptr, 0, w, act_inv, xfrag, T, H, eps, stream,
                          "add_rmsnorm_xfrag");
}

extern "C" int llmserve_add_rmsnorm_split_xfrag(float* x, const float* r, int64_t planes,
                                                const float* w, const float* act_inv, void* xfrag,
                                                int64_t T, int64_t H, float eps, void* stream) {
  LSH_CHECK(planes >= 1 && planes <= 64, "add_rmsnorm_split_xfrag: planes %lld not in [1, 64]",
            (long long)planes);
  return launch_norm_frag(kNormAdd, x, r, nullptr, 0, w, act_inv, xfrag, T, H, eps, stream,
                          "add_rmsnorm_split_xfrag", static_cast<int>(planes));
}

extern "C" int llmserve_embed_rmsnorm_xfrag(const int64_t* ids, const float* embed, int64_t V,
                                            const float* w, const float* act_inv, float* x,
                                            void* xfrag, int64_t T, int64_t H, float eps,
                                            void* stream) {
  LSH_CHECK(V >= 1, "embed_rmsnorm_xfrag: empty embedding");
  return launch_norm_frag(kNormGather, x, embed, ids, V, w, act_inv, xfrag, T, H, eps, stream,
                          "embed_rmsnorm_xfrag");
}

extern "C" int llmserve_silu_mul_xfrag(const float* gate_up, const float* act_inv, void* xfrag,
                                       int64_t T, int64_t I, void* stream) {
  LSH_CHECK(T >= 0 && I >= lsh::kFragBlk && I % lsh::kFragBlk == 0 && T < (1LL << 24) &&
                I < (1LL << 24),
            "silu_mul_xfrag: T=%lld, I=%lld (I a multiple of 128)", (long long)T, (long long)I);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(gate_up && xfrag, "silu_mul_xfrag: null pointer");
  LSH_CHECK(lsh::aligned16(xfrag), "silu_mul_xfrag: the fragment buffer must be 16-byte aligned");
  const int mp = static_cast<int>(lsh::frag_rows(T));
  __bf16* xf = static_cast<__bf16*>(xfrag);
  float* xsum = lsh::frag_sums(xf, mp, I);
  const int64_t items = static_cast<int64_t>(mp) * (I / lsh::kFragBlk);
  const int wpb = kRowThreads / kWave;
  lsh::launch(silu_mul_frag_kernel, dim3(static_cast<unsigned>((items + wpb - 1) / wpb)),
              dim3(kRowThreads), 0, lsh::as_stream(stream), true, gate_up, act_inv, xf, xsum,
              static_cast<int>(T), static_cast<int>(I), mp);
  return lsh::launch_status("silu_mul_xfrag");
}
