// Int4 (group-wise, AWQ-scaled) weight-only linear for more than 16 activation rows, on the
// bf16 matrix cores. This is Int4Linear.forward's large-M branch (reference quant.py:141-142:
// x * inv_act_scale, then x @ dequantize().T), computed with the same group decomposition as
// the reference's kernel (int8_gemv.cpp:48-52):
//   y[m, n] = sum_g s[n, g] * sum_{k in g} x'[m, k] q[n, k] + (z[n, g] - 8 s[n, g]) * sum_{k in g} x'[m, k]
// so the matrix cores multiply only exact operands:
//  * q in [0, 15] is exact in bf16;
//  * x' = x * inv (fp32, rounded as the reference's separate multiply) is split by a pre-pass
//    into bf16 xh = bf16(x') and xl = bf16(x' - xh): xh + xl equals x' to 2^-17 relative
//    (the decode-batch kernel int4_gemm_lat below reads three pieces, xfrag.h: fp32-faithful);
//  * every product of two bf16 values is exact in fp32, and v_mfma_f32_16x16x32_bf16 adds
//    them in fp32. The result is within a few 1e-6 (relative) of fp32 arithmetic.
// The pre-pass also writes the channel sums of x' over every 128-channel block (the
// (z - 8 s) factor). Requires K % 128 == 0 and group % 128 == 0 (the scale is constant over
// a 128-channel block), N % 16 == 0.
//
// Work: a wavefront computes a 16 x 64 output slab (4 tiles of 16 x 16: 16 activation rows,
// 64 output channels) over its share of the K blocks; the x fragments it loads for a block
// feed all four channel tiles (x is re-read from L2 once per 64 output channels). ~150
// registers, so 3 wavefronts per SIMD hide each other's load latency.
// Lane l (fr = l % 16, fc = l / 16) of a k-step j (32 channels) of block b supplies the
// channels 128 b + 32 fc + 8 j .. + 8, for
// both operands: its 16-byte nibble load (row n0 + fr, bytes 64 b + 16 fc .. + 16) holds
// exactly its 32 channels of the block, word j feeding step j; its x fragments are the 64
// contiguous bytes of xh (and of xl) at the same channels. The mapping is a permutation of
// the k index that both operands share, so the dot products are unchanged.
// Blocks are software-pipelined: the loads of block b + 1 are in flight while block b runs.
// When the output has few slabs, S = 2 or 4 wavefronts of a workgroup split the K blocks
// of one slab and add their sums in LDS in a fixed order (deterministic).
#include <algorithm>

#include "common.h"
#include "xfrag.h"

namespace {

using lsh::kWave;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlk = 128;              // channels per k block
constexpr int kMT = 1;                 // 16-row tiles per wavefront
constexpr int kNT = 4;                 // 16-channel tiles per wavefront
constexpr int kRows = 16 * kMT;        // activation rows per wavefront
constexpr int kCols = 16 * kNT;        // output channels per wavefront
constexpr int kWaves = 4;              // wavefronts of the x-split workgroups
constexpr int kSplitWaves = 4;         // largest K split
constexpr int kMaxPlanes = 8;          // largest K split across workgroups (output planes)
constexpr int64_t kWideTiles = 4096;   // slab x row tiles from which int4_gemm_wide runs

// x' = x * inv -> xh, xl (bf16, round to nearest even) and xsum[b, m] = sum of x' over block
// b. One wavefront per (m, b): lane i holds channels 2i, 2i + 1 of the block. xsum rows are
// `mp` floats apart (mp >= M, a multiple of 4: a lane of the GEMM reads 4 consecutive rows).
__global__ __launch_bounds__(kWaves * kWave) void x_split_kernel(
    const float* __restrict__ x, const float* __restrict__ inv, __bf16* __restrict__ xh,
    __bf16* __restrict__ xl, float* __restrict__ xsum, int M, int K, int mp) {
  const int nb = K / kBlk;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
  if (item >= static_cast<int64_t>(M) * nb) return;  // whole wavefront
  const int m = static_cast<int>(item / nb), b = static_cast<int>(item % nb);
  const int lane = threadIdx.x % kWave;
  const int64_t off = static_cast<int64_t>(m) * K + b * kBlk + 2 * lane;
  float2 v = *reinterpret_cast<const float2*>(x + off);
  if (inv) {
    const float2 t = *reinterpret_cast<const float2*>(inv + b * kBlk + 2 * lane);
    v.x = __fmul_rn(v.x, t.x);
    v.y = __fmul_rn(v.y, t.y);
  }
  const __bf16 h0 = static_cast<__bf16>(v.x), h1 = static_cast<__bf16>(v.y);
  const __bf16 l0 = static_cast<__bf16>(v.x - static_cast<float>(h0));
  const __bf16 l1 = static_cast<__bf16>(v.y - static_cast<float>(h1));
  const __bf16 hp[2] = {h0, h1}, lp[2] = {l0, l1};
  *reinterpret_cast<uint32_t*>(xh + off) = *reinterpret_cast<const uint32_t*>(hp);
  *reinterpret_cast<uint32_t*>(xl + off) = *reinterpret_cast<const uint32_t*>(lp);
  const float s = lsh::wave_sum_from<1>(v.x + v.y);
  if (lane == 0) xsum[static_cast<int64_t>(b) * mp + m] = s;
}

struct Int4GemmArgs {
  const __bf16* xh;    // [M, K]
  const __bf16* xl;    // [M, K]
  const float* xsum;   // [K / 128, mp]
  const uint8_t* w;    // nibbles [N, K / 2]
  const float* s;      // g_scale [N, G]
  const float* z;      // g_zero [N, G]
  float* y;            // [M, N]
  int M, N, K, G, bpg, mp;  // bpg: 128-channel blocks per quantization group
};

// 8 nibbles (channels 2e low, 2e + 1 high of byte e) -> 8 bf16, exact: each value one
// byte-select conversion (v_cvt_f32_ubyteN) of the two masked words, then two per packed
// conversion. The empty asm hides the masks from the compiler, which would otherwise
// extract each nibble with a bit-field extract first; it emits nothing.
__device__ __forceinline__ bf16x8 nibbles_bf16(uint32_t wd) {
  uint32_t lo = wd & 0x0f0f0f0fu, hi = (wd >> 4) & 0x0f0f0f0fu;
  asm("" : "+v"(lo), "+v"(hi));
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[2 * e] = static_cast<__bf16>(static_cast<float>((lo >> (8 * e)) & 0xffu));
    r[2 * e + 1] = static_cast<__bf16>(static_cast<float>((hi >> (8 * e)) & 0xffu));
  }
  return r;
}

// Workgroups of 4 wavefronts: R = 4 / S slabs side by side, S wavefronts splitting each
// slab's K blocks.
template <int S>
__global__ __launch_bounds__(256) void int4_gemm_mfma(Int4GemmArgs a) {
  extern __shared__ f32x4 red[];  // S > 1: [wave][kNT * kMT][64] sums of each wavefront
  constexpr int R = 4 / S;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int ks = wave % S;                             // K split
  const int slab = blockIdx.x * R + wave / S;          // 64-channel output slab
  const int n0 = slab * kCols, m0 = blockIdx.y * kRows;
  const int fr = lane % 16, fc = lane / 16;
  const int nblk = a.K / kBlk;
  const int per = (nblk + S - 1) / S;
  const int kb0 = min(nblk, ks * per), kb1 = min(nblk, kb0 + per);

  // Operand bases (rows clamped into the matrices; clamped rows are never stored).
  int nrow[kNT];
  const uint8_t* wp[kNT];
#pragma unroll
  for (int u = 0; u < kNT; ++u) {
    nrow[u] = min(n0 + 16 * u + fr, a.N - 1);
    wp[u] = a.w + static_cast<int64_t>(nrow[u]) * (a.K / 2) + 16 * fc;
  }
  const __bf16* hp[kMT];
  const __bf16* lp[kMT];
#pragma unroll
  for (int t = 0; t < kMT; ++t) {
    const int64_t m = min(m0 + 16 * t + fr, a.M - 1);
    hp[t] = a.xh + m * a.K + 32 * fc;
    lp[t] = a.xl + m * a.K + 32 * fc;
  }

  // one block's operands: nibbles of the 4 channel tiles (4 words each: steps 0..3), x
  // fragments (4 steps x 16 bytes per tile and term), channel sums of the lane's 4 output rows
  auto load = [&](int b, u32x4 (&w)[kNT], u32x4 (&xh)[kMT][4], u32x4 (&xl)[kMT][4],
                  f32x4 (&xs)[kMT]) {
#pragma unroll
    for (int u = 0; u < kNT; ++u)
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp[u] + 64 * b));
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xh[t][j] = *reinterpret_cast<const u32x4*>(hp[t] + kBlk * b + 8 * j);
        xl[t][j] = *reinterpret_cast<const u32x4*>(lp[t] + kBlk * b + 8 * j);
      }
      xs[t] = *reinterpret_cast<const f32x4*>(a.xsum + static_cast<int64_t>(b) * a.mp + m0 +
                                              16 * t + 4 * fc);
    }
  };

  f32x4 acc[kNT][kMT];
#pragma unroll
  for (int u = 0; u < kNT; ++u)
#pragma unroll
    for (int t = 0; t < kMT; ++t) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 w[kNT], xh[kMT][4], xl[kMT][4];
  f32x4 xs[kMT];
  if (kb0 < kb1) load(kb0, w, xh, xl, xs);
  for (int b = kb0; b < kb1; ++b) {
    u32x4 wn[kNT], xhn[kMT][4], xln[kMT][4];
    f32x4 xsn[kMT];
    if (b + 1 < kb1) load(b + 1, wn, xhn, xln, xsn);
    const int g = b / a.bpg;
#pragma unroll
    for (int u = 0; u < kNT; ++u) {
      const float sc = a.s[static_cast<int64_t>(nrow[u]) * a.G + g];
      const float zc = a.z[static_cast<int64_t>(nrow[u]) * a.G + g] - 8.f * sc;
      bf16x8 bq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[j] = nibbles_bf16(w[u][j]);
#pragma unroll
      for (int t = 0; t < kMT; ++t) {
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xh[t][j]), bq[j],
                                                     d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xl[t][j]), bq[j],
                                                     d, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[u][t][r] += sc * d[r] + zc * xs[t][r];
      }
    }
    if (b + 1 < kb1) {
#pragma unroll
      for (int u = 0; u < kNT; ++u) w[u] = wn[u];
#pragma unroll
      for (int t = 0; t < kMT; ++t) {
        xs[t] = xsn[t];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xh[t][j] = xhn[t][j];
          xl[t][j] = xln[t][j];
        }
      }
    }
  }

  if constexpr (S > 1) {
#pragma unroll
    for (int u = 0; u < kNT; ++u)
#pragma unroll
      for (int t = 0; t < kMT; ++t) red[(wave * kNT * kMT + u * kMT + t) * kWave + lane] = acc[u][t];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int k = 1; k < S; ++k)
#pragma unroll
      for (int u = 0; u < kNT; ++u)
#pragma unroll
        for (int t = 0; t < kMT; ++t)
          acc[u][t] += red[((wave + k) * kNT * kMT + u * kMT + t) * kWave + lane];
  }
  // lane holds rows 4 fc + r, column fr of each 16 x 16 tile
#pragma unroll
  for (int u = 0; u < kNT; ++u) {
    const int n = n0 + 16 * u + fr;
    if (n >= a.N) continue;
#pragma unroll
    for (int t = 0; t < kMT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * t + 4 * fc + r;
        if (m < a.M) a.y[static_cast<int64_t>(m) * a.N + n] = acc[u][t][r];
      }
  }
}

// Packed operands of the decode-sized kernel (written once per weight by
// llmserve_int4_gemm_pack, and per call by x_split_frag). Each is laid out in the order the
// wavefronts read it, so that every load instruction of int4_gemm_lat reads contiguous bytes
// (1 KB for a nibble tile or an x fragment) instead of 16 rows x 64 bytes:
//  * nibbles: [slab][block][tile u][lane][16 bytes]; lane l of tile u holds row
//    64 slab + 16 u + l % 16 (zero past N), bytes 64 b + 16 (l / 16) .. + 16 of that row;
//  * scales:  [group][slab][fr][8 floats]: s of the rows 64 slab + 16 u + fr (u = 0..3), then
//    z - 8 s of the same rows (the constant term of the group decomposition, rounded as the
//    kernel would round it);
//  * x:       [row tile][block][step q][hi, mid, lo][lane][8 bf16] (xfrag.h): lane (fr, fc)
//    holds row 16 t + fr (zero past M), channels 128 b + 32 fc + 8 q .. + 8, of each piece.
constexpr int kPkTile = kWave * 16;           // bytes of one nibble tile (4 per slab and block)
constexpr int kPkFrag = kWave * 8;            // bf16 of one x fragment

__host__ __device__ inline int64_t pk_slabs(int64_t N) { return (N + kCols - 1) / kCols; }
inline int64_t pk_weight_bytes(int64_t N, int64_t K) { return pk_slabs(N) * (K / kBlk) * kNT * kPkTile; }
inline int64_t pk_scale_floats(int64_t N, int64_t G) { return G * pk_slabs(N) * 16 * 8; }

__global__ __launch_bounds__(256) void pack_nibbles_kernel(const uint8_t* __restrict__ nib,
                                                           uint8_t* __restrict__ out, int N, int K,
                                                           int64_t pieces) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= pieces) return;
  const int nblk = K / kBlk;
  const int lane = static_cast<int>(i % kWave);
  const int u = static_cast<int>((i / kWave) % kNT);
  const int64_t sb = i / (kWave * kNT);  // slab * nblk + b
  const int b = static_cast<int>(sb % nblk);
  const int64_t slab = sb / nblk;
  const int64_t n = slab * kCols + 16 * u + lane % 16;
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (n < N)
    v = *reinterpret_cast<const u32x4*>(nib + n * (K / 2) + 64 * b + 16 * (lane / 16));
  *reinterpret_cast<u32x4*>(out + i * 16) = v;
}

__global__ __launch_bounds__(256) void pack_scales_kernel(const float* __restrict__ gs,
                                                          const float* __restrict__ gz,
                                                          float* __restrict__ out, int N, int G,
                                                          int64_t items) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (g, slab, fr, u)
  if (i >= items) return;
  const int u = static_cast<int>(i % kNT);
  const int fr = static_cast<int>((i / kNT) % 16);
  const int64_t gslab = i / (kNT * 16);
  const int64_t slabs = pk_slabs(N);
  const int64_t slab = gslab % slabs, g = gslab / slabs;
  const int64_t n = slab * kCols + 16 * u + fr;
  float sc = 0.f, zz = 0.f;
  if (n < N) {
    sc = gs[n * G + g];
    zz = gz[n * G + g] - 8.f * sc;
  }
  float* o = out + (gslab * 16 + fr) * 8;
  o[u] = sc;
  o[4 + u] = zz;
}

// x' = x * inv split into bf16 hi / mid / lo fragments (xfrag.h) and xsum[b, m]. One workgroup
// per (row tile, block): thread (row fr, segment s) handles channels 8 s .. + 8 of row
// 16 t + fr; rows past M are zeros. xsum is the pairwise tree of the block's 128 channels.
__global__ __launch_bounds__(256) void x_split_frag_kernel(
    const float* __restrict__ x, const float* __restrict__ inv, __bf16* __restrict__ xf,
    float* __restrict__ xsum, int M, int K, int mp) {
  const int nblk = K / kBlk;
  const int t = blockIdx.x / nblk, b = blockIdx.x % nblk;
  const int fr = threadIdx.x / 16, seg = threadIdx.x % 16;
  const int m = 16 * t + fr;
  const int c = kBlk * b + 8 * seg;
  float v[8];
  if (m < M) {
    const f32x4 a0 = *reinterpret_cast<const f32x4*>(x + static_cast<int64_t>(m) * K + c);
    const f32x4 a1 = *reinterpret_cast<const f32x4*>(x + static_cast<int64_t>(m) * K + c + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a0[e];
      v[4 + e] = a1[e];
    }
    if (inv) {
      const f32x4 i0 = *reinterpret_cast<const f32x4*>(inv + c);
      const f32x4 i1 = *reinterpret_cast<const f32x4*>(inv + c + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = __fmul_rn(v[e], i0[e]);
        v[4 + e] = __fmul_rn(v[4 + e], i1[e]);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
  }
  lsh::frag_store<8>(xf, m, c, nblk, v);
  const float s = lsh::group_sum<16>(lsh::tree_sum<8>(v));
  if (seg == 0) xsum[static_cast<int64_t>(b) * mp + m] = s;
}

// Decode-sized batches (up to a few 16-row tiles). The time goes to each CU's memory
// requests, not to bandwidth or matrix-core throughput: int4_gemm_lat gives a wavefront
// only KB <= 2 blocks of K per round (one round up to K = 2048), issues every load of them
// (nibbles, x fragments, channel sums, group scales and zeros) before the first use, and
// lets S wavefronts of a workgroup split the K blocks of one 16 x 64 slab; their partial sums meet in LDS and each output tile is
// finished by one wavefront adding the S partials in a fixed order (deterministic).
// Workgroups are numbered so that the row tiles of one slab run on the same XCD: the slab's
// nibbles come from HBM into that XCD's L2 once. Operands are the packed ones (a.w, a.s and
// a.xh as above; a.z and a.xl are unused).
// K split across workgroups (narrow outputs, whose slabs alone leave most CUs idle): plane p
// of the grid takes the blocks [p bpp, (p + 1) bpp) and writes its sums to y + p M N; the
// consumer adds the planes in order (llmserve_add_rmsnorm_split_xfrag). bpp = nblk: one plane.
template <int KB, int S>
__global__ __launch_bounds__(S * kWave) void int4_gemm_lat(Int4GemmArgs a, int slabs_pad, int mtiles,
                                                           int bpp) {
  extern __shared__ f32x4 red[];  // S > 1: [S][kNT][64]
  const int lane = threadIdx.x % kWave, ks = threadIdx.x / kWave;
  const int per_plane = slabs_pad * mtiles;
  const int plane = blockIdx.x / per_plane, wg = blockIdx.x % per_plane;
  const int xcd = wg % 8, j = wg / 8;
  const int t = j % mtiles;
  const int slab = (j / mtiles) * 8 + xcd;
  const int n0 = slab * kCols, m0 = t * kRows;
  if (n0 >= a.N) return;  // padding workgroup (whole workgroup: no barrier is reached)
  const int fr = lane % 16, fc = lane / 16;
  const int nblk = a.K / kBlk;
  const int slabs = (a.N + kCols - 1) / kCols;
  const int b0 = plane * bpp, b1 = min(b0 + bpp, nblk);  // this plane's blocks
  float* y = a.y + static_cast<int64_t>(plane) * a.M * a.N;

  f32x4 acc[kNT];
#pragma unroll
  for (int u = 0; u < kNT; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Rounds of S x KB blocks (one round up to K = 2048 at S = 8, KB = 2).
  for (int base = b0; base < b1; base += S * KB) {
    u32x4 w[KB][kNT], xh[KB][4], xm[KB][4], xl[KB][4];
    f32x4 xs[KB];
    float sc[KB][kNT], zc[KB][kNT];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int b = min(base + ks * KB + kb, b1 - 1);  // clamped: loads stay unconditional
      const int g = b / a.bpg;
      const uint8_t* wt = a.w + ((static_cast<int64_t>(slab) * nblk + b) * kNT) * kPkTile + 16 * lane;
#pragma unroll
      for (int u = 0; u < kNT; ++u)
        w[kb][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + u * kPkTile));
      constexpr int P = lsh::kFragPieces;
      const __bf16* xt = a.xh + ((static_cast<int64_t>(t) * nblk + b) * 4 * P) * kPkFrag + 8 * lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xh[kb][q] = *reinterpret_cast<const u32x4*>(xt + (P * q) * kPkFrag);
        xm[kb][q] = *reinterpret_cast<const u32x4*>(xt + (P * q + 1) * kPkFrag);
        xl[kb][q] = *reinterpret_cast<const u32x4*>(xt + (P * q + 2) * kPkFrag);
      }
      const float* st = a.s + ((static_cast<int64_t>(g) * slabs + slab) * 16 + fr) * 8;
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(st);
      const f32x4 z4 = *reinterpret_cast<const f32x4*>(st + 4);  // z - 8 s
#pragma unroll
      for (int u = 0; u < kNT; ++u) {
        sc[kb][u] = s4[u];
        zc[kb][u] = z4[u];
      }
      xs[kb] = *reinterpret_cast<const f32x4*>(a.xsum + static_cast<int64_t>(b) * a.mp + m0 + 4 * fc);
    }
    // all loads above are issued before any of the products below (the scheduler would
    // otherwise interleave them, turning one memory round trip into several)
    __builtin_amdgcn_sched_barrier(0);
    // Blocks past the end (when S x KB does not divide nblk) were loaded clamped and are
    // weighted by 0: no branch, so that the compiler keeps every load ahead of the first use.
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const float on = base + ks * KB + kb < b1 ? 1.f : 0.f;
#pragma unroll
      for (int u = 0; u < kNT; ++u) {
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bf16x8 bq = nibbles_bf16(w[kb][u][q]);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xh[kb][q]), bq, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xm[kb][q]), bq, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xl[kb][q]), bq, d, 0, 0, 0);
        }
        const float s1 = on * sc[kb][u];
        const float zz = on * zc[kb][u];
        // one explicit form (s1 d + (zz xs rounded), then the sum), so that every kernel
        // computing a block's term rounds it the same way
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[u][r] += __builtin_fmaf(s1, d[r], zz * xs[kb][r]);
      }
    }
  }

  if constexpr (S > 1) {
#pragma unroll
    for (int u = 0; u < kNT; ++u) red[(ks * kNT + u) * kWave + lane] = acc[u];
    __syncthreads();
  }
  // wavefront ks finishes the tiles u = ks, ks + S, ...
#pragma unroll
  for (int u = 0; u < kNT; ++u) {
    const bool mine = S == 1 || (S <= kNT ? u % S == ks : u == ks);
    if (!mine) continue;
    f32x4 v = acc[u];
    if constexpr (S > 1) {
      v = red[u * kWave + lane];
#pragma unroll
      for (int k = 1; k < S; ++k) v += red[(k * kNT + u) * kWave + lane];
    }
    const int n = n0 + 16 * u + fr;
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 4 * fc + r;
      if (m < a.M) y[static_cast<int64_t>(m) * a.N + n] = v[r];
    }
  }
}

// Very wide outputs (an LM head: thousands of slabs). int4_gemm_lat re-reads a row tile's x
// fragments for every slab it computes (96 KB per 64 output channels at K = 1024: ten times
// the nibble bytes). Here the S = K / 128 wavefronts of a workgroup each keep one K block's x
// fragments and channel sums in registers, and the workgroup runs a range of slabs for one
// row tile, loading each slab's nibbles and scales one slab ahead. The per-block arithmetic
// and the fixed-order sum of the S partials in LDS are int4_gemm_lat<1, S>'s. Workgroups of
// the mtiles row tiles of one slab range are numbered onto one XCD, so that a slab's nibbles
// come from HBM into that XCD's L2 once.
template <int S>
__global__ __launch_bounds__(S * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void int4_gemm_wide(Int4GemmArgs a, int mtiles, int groups) {
  __shared__ f32x4 red[S * kNT * kWave];
  const int lane = threadIdx.x % kWave, ks = threadIdx.x / kWave;
  const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
  const int t = j % mtiles;
  const int grp = (j / mtiles) * 8 + xcd;  // slab range of this workgroup
  const int slabs = (a.N + kCols - 1) / kCols;
  const int s0 = static_cast<int>(static_cast<int64_t>(grp) * slabs / groups);
  const int s1 = static_cast<int>(static_cast<int64_t>(grp + 1) * slabs / groups);
  if (grp >= groups || s0 >= s1) return;  // whole workgroup: no barrier is reached
  const int fr = lane % 16, fc = lane / 16;
  const int b = ks, g = b / a.bpg;  // this wavefront's K block (S == K / 128)
  const int m0 = t * kRows;

  u32x4 xh[4], xm[4], xl[4];
  constexpr int P = lsh::kFragPieces;
  const __bf16* xt = a.xh + ((static_cast<int64_t>(t) * S + b) * 4 * P) * kPkFrag + 8 * lane;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    xh[q] = *reinterpret_cast<const u32x4*>(xt + (P * q) * kPkFrag);
    xm[q] = *reinterpret_cast<const u32x4*>(xt + (P * q + 1) * kPkFrag);
    xl[q] = *reinterpret_cast<const u32x4*>(xt + (P * q + 2) * kPkFrag);
  }
  const f32x4 xs = *reinterpret_cast<const f32x4*>(a.xsum + static_cast<int64_t>(b) * a.mp + m0 + 4 * fc);

  auto load_w = [&](int slab, u32x4 (&w)[kNT], f32x4& s4, f32x4& z4) {
    const uint8_t* wt = a.w + ((static_cast<int64_t>(slab) * S + b) * kNT) * kPkTile + 16 * lane;
#pragma unroll
    for (int u = 0; u < kNT; ++u)
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + u * kPkTile));
    const float* st = a.s + ((static_cast<int64_t>(g) * slabs + slab) * 16 + fr) * 8;
    s4 = *reinterpret_cast<const f32x4*>(st);
    z4 = *reinterpret_cast<const f32x4*>(st + 4);  // z - 8 s
  };
  auto run = [&](int slab, const u32x4 (&w)[kNT], const f32x4& s4, const f32x4& z4) {
#pragma unroll
    for (int u = 0; u < kNT; ++u) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x8 bq = nibbles_bf16(w[u][q]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xh[q]), bq, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xm[q]), bq, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xl[q]), bq, d, 0, 0, 0);
      }
      const float s1 = s4[u], zz = z4[u];
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += __builtin_fmaf(s1, d[r], zz * xs[r]);  // as int4_gemm_lat
      red[(ks * kNT + u) * kWave + lane] = acc;
    }
    __syncthreads();
    if (ks < kNT) {  // wavefront ks finishes channel tile u = ks
      const int u = ks;
      f32x4 v = red[u * kWave + lane];
#pragma unroll
      for (int k = 1; k < S; ++k) v += red[(k * kNT + u) * kWave + lane];
      const int n = slab * kCols + 16 * u + fr;
      if (n < a.N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 4 * fc + r;
          if (m < a.M) a.y[static_cast<int64_t>(m) * a.N + n] = v[r];
        }
      }
    }
    __syncthreads();  // red is rewritten by the next slab
  };

  // two register sets, each slab's loads issued before the previous slab's products; past the
  // range the last slab is loaded again (unused), so the loads stay unconditional
  u32x4 wa[kNT], wb[kNT];
  f32x4 sa, za, sb, zb;
  load_w(s0, wa, sa, za);
  for (int sl = s0; sl < s1; sl += 2) {
    load_w(sl + 1 < s1 ? sl + 1 : s1 - 1, wb, sb, zb);
    run(sl, wa, sa, za);
    if (sl + 1 >= s1) break;
    load_w(sl + 2 < s1 ? sl + 2 : s1 - 1, wa, sa, za);
    run(sl + 1, wb, sb, zb);
  }
}

// One 16-row tile of activations (M <= 16: a decode batch through Int4Linear.forward) in ONE
// launch: each wavefront builds its K block's three-piece fragments and block sums from the
// fp32 x rows itself, in registers, instead of reading those of a separate split pass. The
// values are the split pass's bit for bit: x' = x * inv (rounded multiply), hi / mid / lo as
// split3_bf16 (two channels per packed conversion), and each row's block sum as the same pairwise tree (lane (fr, fc) holds the
// channels 32 fc .. + 32 of row fr, i.e. the split pass's segments 4 fc .. 4 fc + 3: its
// 8-channel trees and their first two butterfly levels are in-lane, the last two are lane
// swaps 16 and 32 apart; the MFMA layout then wants the sums of rows 4 fc + r, fetched with
// four lane shuffles). The products and their accumulation are int4_gemm_lat's.
// Work: S wavefronts split the K blocks of NT 16-column tiles (one block per wavefront and
// round); NT = 1 gives each workgroup one tile of a slab, so a narrow output (N = 1024:
// 16 slabs) spreads over 64 workgroups instead of 16; NT = 2 where the tiles outnumber the
// CUs (one x conversion per block serves both tiles). With bpp < K / 128 the K blocks are
// split across workgroups as well: plane p (blocks [p bpp, (p + 1) bpp)) goes to y (p = 0)
// or ys + (p - 1) M N, with int4_gemm_lat's per-plane order (the fragment path's K-split
// planes, bit for bit), and plane_sum_kernel adds the planes in order.
// v_permlane32_swap: the upper 32 lanes of a trade places with the lower 32 of b.
__device__ __forceinline__ void swap_halves32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a),
                                                  __builtin_bit_cast(uint32_t, b), false, false);
  a = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  b = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// v_permlane16_swap: the odd 16-lane rows of a trade places with the even rows of b.
__device__ __forceinline__ void swap_rows16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a),
                                                  __builtin_bit_cast(uint32_t, b), false, false);
  a = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  b = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

struct Int4GemmXArgs {
  const float* x;    // [M, K] fp32
  const float* inv;  // [K] AWQ pre-scale (INV only)
  const uint8_t* w;  // packed nibbles
  const float* s;    // packed scales
  float* y;          // [M, N]: the output, or plane 0 when bpp < K / 128
  float* ys;         // planes 1, 2, ... [planes - 1, M, N] (bpp < K / 128)
  int M, N, K, bpg;
  int bpp;           // K blocks per plane
};

template <int S, int NT, bool INV, bool CO>
__global__ __launch_bounds__(S * kWave) void int4_gemm_x(Int4GemmXArgs a) {
  extern __shared__ f32x4 red[];  // S > 1: [S][NT][64]
  constexpr int kUnits = kNT / NT;  // workgroups per slab
  const int lane = threadIdx.x % kWave, ks = threadIdx.x / kWave;
  const int slabs = (a.N + kCols - 1) / kCols;
  const int per_plane = slabs * kUnits;
  const int plane = blockIdx.x / per_plane, wg = blockIdx.x % per_plane;
  const int slab = wg / kUnits, u0 = (wg % kUnits) * NT;
  const int n0 = slab * kCols + 16 * u0;
  if (n0 >= a.N) return;  // whole workgroup: no barrier is reached
  const int fr = lane % 16, fc = lane / 16;
  const int nblk = a.K / kBlk;
  const int b0 = plane * a.bpp, b1 = min(b0 + a.bpp, nblk);  // this plane's blocks
  float* y = plane == 0 ? a.y : a.ys + static_cast<int64_t>(plane - 1) * a.M * a.N;
  // rows past M repeat row M - 1 (in bounds): each output row depends on its own x row
  // only, and theirs are not stored
  const float* xrow =
      a.x + static_cast<int64_t>(fr < a.M ? fr : a.M - 1) * a.K + (CO ? 4 * fc : 32 * fc);

  f32x4 acc[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int base = b0; base < b1; base += S) {
    const int b = min(base + ks, b1 - 1);  // clamped: loads stay unconditional
    const int g = b / a.bpg;
    u32x4 w[NT];
    const uint8_t* wt = a.w + ((static_cast<int64_t>(slab) * nblk + b) * kNT + u0) * kPkTile + 16 * lane;
#pragma unroll
    for (int u = 0; u < NT; ++u)
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + u * kPkTile));
    const float* st = a.s + ((static_cast<int64_t>(g) * slabs + slab) * 16 + fr) * 8;
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(st);
    const f32x4 z4 = *reinterpret_cast<const f32x4*>(st + 4);  // z - 8 s
    // CO: load i gives lane (fr, fc) the channels 16 i + 4 fc .. + 4 of row fr: the four
    // lanes of a row read 64 contiguous bytes, so each instruction touches 16 cache lines.
    // Otherwise the MFMA layout is read directly (lane (fr, fc): channels 32 fc + 4 i .. + 4):
    // 4 lines per distinct row, 64 at 16 rows, but no transpose (fewer instructions when few
    // rows are distinct).
    f32x4 xv[8], iv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      xv[i] = *reinterpret_cast<const f32x4*>(xrow + b * kBlk + (CO ? 16 : 4) * i);
    if constexpr (INV) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        iv[i] = *reinterpret_cast<const f32x4*>(a.inv + b * kBlk +
                                                (CO ? 16 * i + 4 * fc : 32 * fc + 4 * i));
    }
    // every load above goes out before the arithmetic below
    __builtin_amdgcn_sched_barrier(0);
    float t[8][4];  // x' in the load layout
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) t[i][c] = INV ? __fmul_rn(xv[i][c], iv[i][c]) : xv[i][c];
    // CO, to the MFMA layout (lane (fr, fc): channels 32 fc .. + 32 of row fr, in order): the
    // loads 2 p, 2 p + 1 of lane group fc' belong to lane group p, as its channel quads fc'
    // and 4 + fc'. A 4 x 4 transpose of (lane group, load pair) over the four 16-lane rows:
    // swap the 32-lane halves of pairs (0, 2) and (1, 3), then the odd / even rows of pairs
    // (0, 1) and (2, 3). Afterwards quad j of the lane's channels is t[2 (j % 4) + j / 4].
    if constexpr (CO) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) swap_halves32(t[i][c], t[i + 4][c]);
#pragma unroll
      for (int i : {0, 1, 4, 5})
#pragma unroll
        for (int c = 0; c < 4; ++c) swap_rows16(t[i][c], t[i + 2][c]);
    }
    u32x4 xh[4], xm[4], xl[4];
    float tq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 2 * q + e / 4;  // channel quad of the lane's 32
        v[e] = t[CO ? 2 * (j % 4) + j / 4 : j][e % 4];
      }
      tq[q] = lsh::tree_sum<8>(v);
      uint32_t h[4], md[4], l[4];
      lsh::split3_words<8>(v, h, md, l);
      xh[q] = u32x4{h[0], h[1], h[2], h[3]};
      xm[q] = u32x4{md[0], md[1], md[2], md[3]};
      xl[q] = u32x4{l[0], l[1], l[2], l[3]};
    }
    float rs = (tq[0] + tq[1]) + (tq[2] + tq[3]);  // row fr: this lane's 32 channels
    rs += __shfl_xor(rs, 16, kWave);               // + the neighbouring 32
    rs += __shfl_xor(rs, 32, kWave);               // + the other 64: the block sum of row fr
    f32x4 xs;
#pragma unroll
    for (int r = 0; r < 4; ++r) xs[r] = __shfl(rs, 4 * fc + r, kWave);  // rows 4 fc + r
    const float on = base + ks < b1 ? 1.f : 0.f;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x8 bq = nibbles_bf16(w[u][q]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xh[q]), bq, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xm[q]), bq, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xl[q]), bq, d, 0, 0, 0);
      }
      const float s1 = on * s4[u0 + u];
      const float zz = on * z4[u0 + u];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[u][r] += __builtin_fmaf(s1, d[r], zz * xs[r]);  // as int4_gemm_lat
    }
  }

  if constexpr (S > 1) {
#pragma unroll
    for (int u = 0; u < NT; ++u) red[(ks * NT + u) * kWave + lane] = acc[u];
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const bool mine = S == 1 || (S <= NT ? u % S == ks : u == ks);
    if (!mine) continue;
    f32x4 v = acc[u];
    if constexpr (S > 1) {
      v = red[u * kWave + lane];
#pragma unroll
      for (int k = 1; k < S; ++k) v += red[(k * NT + u) * kWave + lane];
    }
    const int n = n0 + 16 * u + fr;
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * fc + r;
      if (m < a.M) y[static_cast<int64_t>(m) * a.N + n] = v[r];
    }
  }
}

// y = y + ys[0] + ... + ys[P - 2] over n elements (plane 0 is y itself), added in plane
// order (the fragment path's plane consumers add them in the same order); the planes' loads
// go out together (P <= 4).
__global__ __launch_bounds__(256) void plane_sum_kernel(float* __restrict__ y,
                                                        const float* __restrict__ ys, int64_t n,
                                                        int P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float t[4];
  t[0] = y[i];
#pragma unroll
  for (int p = 1; p < 4; ++p) t[p] = p < P ? ys[(p - 1) * n + i] : 0.f;
  float v = t[0];
#pragma unroll
  for (int p = 1; p < 4; ++p)
    if (p < P) v += t[p];
  y[i] = v;
}

// Wavefronts of a workgroup whose wavefronts take one K block per round: the fewest rounds of
// up to 16 wavefronts, then the smallest of 4, 8, 12, 16 that covers the nb blocks in that
// many rounds.
int one_block_waves(int nb) {
  const int rounds = (nb + 15) / 16;
  int S = 16;
  for (int s : {12, 8, 4})
    if (s * rounds >= nb) S = s;
  return S;
}

template <int S, int NT, bool CO>
void launch_x(const Int4GemmXArgs& a, int64_t slabs, int planes, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(slabs * (kNT / NT) * planes)), block(S * kWave);
  const size_t lds = S > 1 ? static_cast<size_t>(S) * NT * kWave * sizeof(f32x4) : 0;
  if (a.inv)
    lsh::launch(int4_gemm_x<S, NT, true, CO>, grid, block, lds, st, true, a);
  else
    lsh::launch(int4_gemm_x<S, NT, false, CO>, grid, block, lds, st, true, a);
}

int device_cus();

// Tiles per workgroup of the one-tile GEMM: one while the output's 16-column tiles fit the
// CUs, two beyond (a workgroup converts its x blocks once for both tiles; with one tile per
// workgroup config 2's gate_up, 384 tiles, puts two workgroups on half the CUs).
int x_tile_nt(int64_t slabs) { return slabs * kNT > device_cus() ? 2 : 1; }

// S: wavefronts to cover the K blocks in one round (up to 16: K = 2048; K = 3072 takes two
// rounds); NT: tiles per workgroup (x_tile_nt). More workgroups beat less redundant conversion
// while they fit the CUs: config 2 at 16 rows (the four Qwen3-0.6B shapes, 112 launches) 273
// GB/s with one tile per workgroup for all shapes, 276 with two, 219 with a whole slab (four);
// 5 rows 324 / 307 / 221. Two tiles only where one would put two workgroups on some CUs
// (gate_up, 384 tiles: 8.88 -> 6.52 us per call, 348 -> 375 GB/s).
// CO (coalesced x loads and the lane transpose) above 8 rows: 16 rows 279 -> 292 GB/s;
// at 1-8 rows the direct loads touch no more lines and skip the transpose (8 rows 330
// against 319).
// S = one_block_waves(nb) (idle wavefronts of a last round would still convert x): K = 3072
// (24 blocks) takes two rounds of 12, 16 rows 292 -> 302 GB/s.
// planes > 1: the K blocks split across workgroups (a.bpp blocks each), S from a.bpp.
// Returns false (nothing launched) for a configuration without an instance.
bool launch_x_tile(const Int4GemmXArgs& a, int64_t slabs, int planes, hipStream_t st) {
  const int S = one_block_waves(a.bpp);
  const int NT = x_tile_nt(slabs);
  const bool co = a.M > 8;
#define LSH_X(s, nt)                                                                        \
  if (S == s && NT == nt) {                                                                 \
    co ? launch_x<s, nt, true>(a, slabs, planes, st)                                        \
       : launch_x<s, nt, false>(a, slabs, planes, st);                                      \
    return true;                                                                            \
  }
  LSH_X(4, 1) LSH_X(4, 2) LSH_X(8, 1) LSH_X(8, 2) LSH_X(12, 1) LSH_X(12, 2) LSH_X(16, 1)
  LSH_X(16, 2)
#undef LSH_X
  return false;
}

int64_t xsum_rows(int64_t M) { return (M + kRows - 1) / kRows * kRows; }

// CUs of the current device (cached per device: the linears ask on every call).
int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int c = 0;
    cached[dev] = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) ==
                              hipSuccess && c > 0
                      ? c
                      : 256;
  }
  return cached[dev];
}

// K planes of the one-launch GEMM (one 16-row tile): a narrow output, whose tiles alone leave
// most CUs idle and whose every workgroup converts x for all its K blocks, splits the blocks
// across workgroups: the largest P <= 4 with tiles x P <= CUs, at least 4 blocks in every
// plane, and planes 1 .. P - 1 (M x N floats each; plane 0 is the output) inside the fragment
// workspace the call takes anyway. Config 2's o_proj (16 K blocks) and down_proj (24) at 16
// rows: 4 planes each.
int packed_planes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > kRows || K % kBlk != 0) return 1;
  const int64_t nb = K / kBlk, slabs = pk_slabs(N);
  const int64_t tiles = slabs * (kNT / x_tile_nt(slabs));
  const int64_t cus = device_cus(), room = lsh::frag_bytes(M, K);
  for (int P = 4; P >= 2; --P) {  // plane_sum_kernel adds at most 4
    const int64_t bpp = (nb + P - 1) / P;
    if (tiles * P <= cus && bpp >= 4 && (nb + bpp - 1) / bpp == P &&
        (P - 1) * M * N * static_cast<int64_t>(sizeof(float)) <= room)
      return P;
  }
  return 1;
}

template <int KB, int S>
void launch_lat_ks(const Int4GemmArgs& a, int64_t slabs, int64_t mtiles, int planes, int bpp,
                   hipStream_t st) {
  const int64_t slabs_pad = (slabs + 7) / 8 * 8;
  const dim3 grid(static_cast<unsigned>(slabs_pad * mtiles * planes)), block(S * kWave);
  const size_t lds = S > 1 ? static_cast<size_t>(S) * kNT * kWave * sizeof(f32x4) : 0;
  lsh::launch(int4_gemm_lat<KB, S>, grid, block, lds, st, true, a,
              static_cast<int>(slabs_pad), static_cast<int>(mtiles), bpp);
}

// Blocks per wavefront and round KB = ceil(nb / 8) (at most 2: three blocks of three-piece x
// fragments take more than the 256 registers a wavefront of an 8-wavefront workgroup has, and
// the spills cost more than a second round: down 3072->1024 at 64 rows 15.5 against 14.3 us),
// then the fewest of 1, 2, 4, 8
// wavefronts that cover the nb blocks (8 when more than one round is needed); the exceptions
// below.
// Returns false (nothing launched) for a configuration without an instance.
bool launch_lat(const Int4GemmArgs& a, int64_t slabs, int64_t mtiles, int nb_all, hipStream_t st,
                int planes = 1) {
  // very wide outputs (at least 256 slabs) with K = 512 or 1024: int4_gemm_wide, about two
  // workgroups per CU
  if (planes == 1 && (nb_all == 4 || nb_all == 8) && slabs >= 256 && slabs * mtiles >= kWideTiles) {
    const int cus = device_cus();
    int64_t groups = (2 * cus + mtiles - 1) / mtiles;
    groups = std::min<int64_t>(groups, slabs / 2);
    groups = std::max<int64_t>(8, (groups + 7) / 8 * 8);
    const dim3 grid(static_cast<unsigned>(mtiles * groups));
    if (nb_all == 8)
      lsh::launch(int4_gemm_wide<8>, grid, dim3(8 * kWave), 0, st, true, a, static_cast<int>(mtiles),
                  static_cast<int>(groups));
    else
      lsh::launch(int4_gemm_wide<4>, grid, dim3(4 * kWave), 0, st, true, a, static_cast<int>(mtiles),
                  static_cast<int>(groups));
    return true;
  }
  const int bpp = (nb_all + planes - 1) / planes;  // blocks per plane
  const int nb = bpp;
  int KB = std::min(2, (nb + 7) / 8);
  int S = 1;
  while (S < 8 && S * KB < nb) S *= 2;
  // more than 8 blocks on a narrow output: up to 16 wavefronts of one block each (4 per SIMD)
  // keep more loads in flight per CU than 8 of two blocks (o_proj at M = 64: 6.3 against
  // 6.7 us); the fewest rounds, then the smallest of 8, 12, 16 wavefronts covering the blocks
  // in them (down, 24 blocks: two rounds of 12), as int4_gemm_x chooses
  if (KB == 2 && S == 8 && slabs * mtiles * planes < 256) {
    KB = 1;
    S = one_block_waves(nb);
  }
  // very large outputs (an LM head) fill the GPU anyway: fewer, longer wavefronts
  if (KB == 1 && S == 8 && slabs * mtiles * planes * S > 16384) {
    KB = 2;
    S = 4;
  }
#define LSH_LAT(kb, s)                                              \
  if (KB == kb && S == s) {                                         \
    launch_lat_ks<kb, s>(a, slabs, mtiles, planes, bpp, st);        \
    return true;                                                    \
  }
  LSH_LAT(1, 1) LSH_LAT(1, 2) LSH_LAT(1, 4) LSH_LAT(1, 8)
  LSH_LAT(2, 4) LSH_LAT(2, 8) LSH_LAT(1, 12) LSH_LAT(1, 16)
#undef LSH_LAT
  return false;
}

}  // namespace

extern "C" int64_t llmserve_int4_linear_gemm_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return M * K * 4 + (K / kBlk) * xsum_rows(M) * 4;
}

extern "C" int llmserve_int4_linear_gemm(const float* x, const float* inv_act_scale,
                                         const uint8_t* nibbles, const float* g_scale,
                                         const float* g_zero, float* y, int64_t M, int64_t N,
                                         int64_t K, int64_t group_size, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 1 && group_size >= 2, "int4_linear_gemm: bad shape");
  LSH_CHECK(K % kBlk == 0 && group_size % kBlk == 0 && K % group_size == 0,
            "int4_linear_gemm: K and group_size must be multiples of 128 (K %% group == 0)");
  LSH_CHECK(N % 16 == 0, "int4_linear_gemm: out_features must be a multiple of 16");
  LSH_CHECK(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && M * K < (1LL << 40) &&
                N * K < (1LL << 41),
            "int4_linear_gemm: shape too large");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(x && nibbles && g_scale && g_zero && y, "int4_linear_gemm: null pointer");
  LSH_CHECK(lsh::aligned16(nibbles) && (reinterpret_cast<uintptr_t>(x) & 7) == 0 &&
                (inv_act_scale == nullptr || (reinterpret_cast<uintptr_t>(inv_act_scale) & 7) == 0),
            "int4_linear_gemm: nibbles must be 16-byte and x / inv_act_scale 8-byte aligned");
  const int64_t need = llmserve_int4_linear_gemm_workspace_bytes(M, K);
  LSH_CHECK(workspace != nullptr && workspace_bytes >= need && lsh::aligned16(workspace),
            "int4_linear_gemm: a 16-byte aligned workspace of %lld bytes is needed (%lld given)",
            (long long)need, (long long)workspace_bytes);
  hipStream_t st = lsh::as_stream(stream);
  const int nb = static_cast<int>(K / kBlk);
  const int mp = static_cast<int>(xsum_rows(M));
  __bf16* xh = static_cast<__bf16*>(workspace);
  __bf16* xl = xh + M * K;
  float* xsum = reinterpret_cast<float*>(xl + M * K);
  const int64_t items = M * nb;
  lsh::launch(x_split_kernel, dim3(static_cast<unsigned>((items + kWaves - 1) / kWaves)),
              dim3(kWaves * kWave), 0, st, false, x, inv_act_scale, xh, xl, xsum,
              static_cast<int>(M), static_cast<int>(K), mp);

  Int4GemmArgs a{xh, xl, xsum, nibbles, g_scale, g_zero, y, static_cast<int>(M),
                 static_cast<int>(N), static_cast<int>(K), static_cast<int>(K / group_size),
                 static_cast<int>(group_size / kBlk), mp};
  const int64_t slabs = (N + kCols - 1) / kCols, mtiles = (M + kRows - 1) / kRows;
  // K split: the smallest S (1, 2, 4) that gives >= 768 wavefronts, with >= 2 blocks each
  int S = 1;
  while (S < kSplitWaves && slabs * mtiles * S < 768 && nb >= 2 * (2 * S)) S *= 2;
  const int R = 4 / S;  // slabs per workgroup
  const dim3 grid(static_cast<unsigned>((slabs + R - 1) / R), static_cast<unsigned>(mtiles));
  const dim3 block(static_cast<unsigned>(R * S * kWave));
  const size_t lds = S > 1 ? static_cast<size_t>(R * S) * kNT * kMT * kWave * sizeof(f32x4) : 0;
  switch (S) {
    case 4: lsh::launch(int4_gemm_mfma<4>, grid, block, lds, st, true, a); break;
    case 2: lsh::launch(int4_gemm_mfma<2>, grid, block, lds, st, true, a); break;
    default: lsh::launch(int4_gemm_mfma<1>, grid, block, lds, st, true, a); break;
  }
  return lsh::launch_status("int4_linear_gemm");
}

extern "C" int64_t llmserve_int4_gemm_pack_bytes(int64_t N, int64_t K, int64_t group_size) {
  if (N <= 0 || K <= 0 || group_size <= 0 || K % kBlk || K % group_size) return 0;
  const int64_t w = (pk_weight_bytes(N, K) + 255) / 256 * 256;
  return w + pk_scale_floats(N, K / group_size) * 4;
}

extern "C" int llmserve_int4_gemm_pack(const uint8_t* nibbles, const float* g_scale,
                                       const float* g_zero, int64_t N, int64_t K,
                                       int64_t group_size, void* packed, int64_t packed_bytes,
                                       void* stream) {
  LSH_CHECK(N >= 1 && K >= 1 && group_size >= 2 && N < (1LL << 31) && K < (1LL << 31),
            "int4_gemm_pack: bad shape");
  LSH_CHECK(K % kBlk == 0 && group_size % kBlk == 0 && K % group_size == 0,
            "int4_gemm_pack: K and group_size must be multiples of 128 (K %% group == 0)");
  LSH_CHECK(nibbles && g_scale && g_zero && packed, "int4_gemm_pack: null pointer");
  LSH_CHECK(lsh::aligned16(nibbles) && lsh::aligned16(packed),
            "int4_gemm_pack: nibbles and the packed buffer must be 16-byte aligned");
  const int64_t need = llmserve_int4_gemm_pack_bytes(N, K, group_size);
  LSH_CHECK(packed_bytes >= need, "int4_gemm_pack: %lld bytes needed, %lld given",
            (long long)need, (long long)packed_bytes);
  hipStream_t st = lsh::as_stream(stream);
  uint8_t* wpk = static_cast<uint8_t*>(packed);
  float* spk = reinterpret_cast<float*>(wpk + (pk_weight_bytes(N, K) + 255) / 256 * 256);
  const int64_t pieces = pk_weight_bytes(N, K) / 16;
  lsh::launch(pack_nibbles_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0,
              st, false, nibbles, wpk, static_cast<int>(N), static_cast<int>(K), pieces);
  const int64_t G = K / group_size;
  const int64_t items = pk_scale_floats(N, G) / 2;
  lsh::launch(pack_scales_kernel, dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0,
              st, true, g_scale, g_zero, spk, static_cast<int>(N), static_cast<int>(G), items);
  return lsh::launch_status("int4_gemm_pack");
}

extern "C" int64_t llmserve_int4_linear_gemm_packed_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return lsh::frag_bytes(M, K);
}

extern "C" int64_t llmserve_int4_packed_splits(int64_t M, int64_t N, int64_t K) {
  return packed_planes(M, N, K);
}

extern "C" int64_t llmserve_int4_xfrag_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % kBlk) return 0;
  return lsh::frag_bytes(M, K);
}

extern "C" int llmserve_int4_linear_gemm_packed(const float* x, const float* inv_act_scale,
                                                const void* packed, float* y, int64_t M,
                                                int64_t N, int64_t K, int64_t group_size,
                                                void* workspace, int64_t workspace_bytes,
                                                void* stream) {
  LSH_CHECK(M >= 0 && N >= 1 && K >= 1 && group_size >= 2, "int4_linear_gemm_packed: bad shape");
  LSH_CHECK(K % kBlk == 0 && group_size % kBlk == 0 && K % group_size == 0,
            "int4_linear_gemm_packed: K and group_size must be multiples of 128 (K %% group == 0)");
  LSH_CHECK(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && M * K < (1LL << 40) &&
                N * K < (1LL << 41),
            "int4_linear_gemm_packed: shape too large");
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(x && packed && y, "int4_linear_gemm_packed: null pointer");
  LSH_CHECK(lsh::aligned16(x) && lsh::aligned16(packed) &&
                (inv_act_scale == nullptr || lsh::aligned16(inv_act_scale)),
            "int4_linear_gemm_packed: x, inv_act_scale and the packed weight must be 16-byte "
            "aligned");
  const int64_t need = llmserve_int4_linear_gemm_packed_workspace_bytes(M, K);
  LSH_CHECK(workspace != nullptr && workspace_bytes >= need && lsh::aligned16(workspace),
            "int4_linear_gemm_packed: a 16-byte aligned workspace of %lld bytes is needed "
            "(%lld given)",
            (long long)need, (long long)workspace_bytes);
  hipStream_t st = lsh::as_stream(stream);
  const int nb = static_cast<int>(K / kBlk);
  const int64_t mtiles = (M + kRows - 1) / kRows;
  const int mp = static_cast<int>(xsum_rows(M));
  const uint8_t* wpk0 = static_cast<const uint8_t*>(packed);
  if (mtiles == 1) {  // one row tile: fragments built inside the GEMM
    // narrow outputs: K planes in the workspace (unused by this path otherwise), then their sum
    const int planes = packed_planes(M, N, K);
    float* ys = static_cast<float*>(workspace);  // planes 1 ..
    Int4GemmXArgs xa{x, inv_act_scale, wpk0,
                     reinterpret_cast<const float*>(wpk0 + (pk_weight_bytes(N, K) + 255) / 256 * 256),
                     y, ys, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                     static_cast<int>(group_size / kBlk), (nb + planes - 1) / planes};
    LSH_CHECK(launch_x_tile(xa, pk_slabs(N), planes, st),
              "int4_linear_gemm_packed: no kernel instance for K=%lld", (long long)K);
    if (planes > 1)
      lsh::launch(plane_sum_kernel, dim3(static_cast<unsigned>((M * N + 255) / 256)), dim3(256),
                  0, st, true, y, static_cast<const float*>(ys), M * N, planes);
    return lsh::launch_status("int4_linear_gemm_packed");
  }
  __bf16* xf = static_cast<__bf16*>(workspace);
  float* xsum = lsh::frag_sums(xf, mp, K);
  lsh::launch(x_split_frag_kernel, dim3(static_cast<unsigned>(mtiles * nb)), dim3(256), 0, st, false,
              x, inv_act_scale, xf, xsum, static_cast<int>(M), static_cast<int>(K), mp);
  const uint8_t* wpk = static_cast<const uint8_t*>(packed);
  const float* spk = reinterpret_cast<const float*>(wpk + (pk_weight_bytes(N, K) + 255) / 256 * 256);
  Int4GemmArgs a{xf, nullptr, xsum, wpk, spk, nullptr, y, static_cast<int>(M),
                 static_cast<int>(N), static_cast<int>(K), static_cast<int>(K / group_size),
                 static_cast<int>(group_size / kBlk), mp};
  LSH_CHECK(launch_lat(a, pk_slabs(N), mtiles, nb, st),
            "int4_linear_gemm_packed: no kernel instance for M=%lld K=%lld", (long long)M,
            (long long)K);
  return lsh::launch_status("int4_linear_gemm_packed");
}

extern "C" int llmserve_int4_xfrag_split(const float* x, const float* inv_act_scale, void* xfrag,
                                         int64_t M, int64_t K, int64_t xfrag_bytes, void* stream) {
  LSH_CHECK(M >= 0 && K >= kBlk && K % kBlk == 0, "int4_xfrag_split: K must be a multiple of 128");
  LSH_CHECK(M < (1LL << 31) && K < (1LL << 31) && M * K < (1LL << 40), "int4_xfrag_split: shape too large");
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(x && xfrag, "int4_xfrag_split: null pointer");
  LSH_CHECK(lsh::aligned16(x) && lsh::aligned16(xfrag) &&
                (inv_act_scale == nullptr || lsh::aligned16(inv_act_scale)),
            "int4_xfrag_split: x, inv_act_scale and xfrag must be 16-byte aligned");
  LSH_CHECK(xfrag_bytes >= lsh::frag_bytes(M, K), "int4_xfrag_split: %lld bytes of fragments needed",
            (long long)lsh::frag_bytes(M, K));
  const int nb = static_cast<int>(K / kBlk);
  const int64_t mtiles = (M + kRows - 1) / kRows;
  const int mp = static_cast<int>(xsum_rows(M));
  __bf16* xf = static_cast<__bf16*>(xfrag);
  lsh::launch(x_split_frag_kernel, dim3(static_cast<unsigned>(mtiles * nb)), dim3(256), 0,
              lsh::as_stream(stream), true, x, inv_act_scale, xf, lsh::frag_sums(xf, mp, K),
              static_cast<int>(M), static_cast<int>(K), mp);
  return lsh::launch_status("int4_xfrag_split");
}

extern "C" int llmserve_int4_linear_gemm_xfrag(const void* xfrag, const void* packed, float* y,
                                               int64_t M, int64_t N, int64_t K,
                                               int64_t group_size, void* stream) {
  LSH_CHECK(M >= 0 && N >= 1 && K >= 1 && group_size >= 2, "int4_linear_gemm_xfrag: bad shape");
  LSH_CHECK(K % kBlk == 0 && group_size % kBlk == 0 && K % group_size == 0,
            "int4_linear_gemm_xfrag: K and group_size must be multiples of 128 (K %% group == 0)");
  LSH_CHECK(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && M * K < (1LL << 40) &&
                N * K < (1LL << 41),
            "int4_linear_gemm_xfrag: shape too large");
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(xfrag && packed && y, "int4_linear_gemm_xfrag: null pointer");
  LSH_CHECK(lsh::aligned16(xfrag) && lsh::aligned16(packed),
            "int4_linear_gemm_xfrag: the fragments and the packed weight must be 16-byte aligned");
  const int nb = static_cast<int>(K / kBlk);
  const int64_t mtiles = (M + kRows - 1) / kRows;
  const int mp = static_cast<int>(lsh::frag_rows(M));
  const __bf16* xf = static_cast<const __bf16*>(xfrag);
  const float* xsum = lsh::frag_sums(xf, mp, K);
  const uint8_t* wpk = static_cast<const uint8_t*>(packed);
  const float* spk = reinterpret_cast<const float*>(wpk + (pk_weight_bytes(N, K) + 255) / 256 * 256);
  Int4GemmArgs a{xf, nullptr, xsum, wpk, spk, nullptr, y, static_cast<int>(M),
                 static_cast<int>(N), static_cast<int>(K), static_cast<int>(K / group_size),
                 static_cast<int>(group_size / kBlk), mp};
  LSH_CHECK(launch_lat(a, pk_slabs(N), mtiles, nb, lsh::as_stream(stream)),
            "int4_linear_gemm_xfrag: no kernel instance for M=%lld K=%lld", (long long)M,
            (long long)K);
  return lsh::launch_status("int4_linear_gemm_xfrag");
}

// K planes for a decode-batch linear on fragments: P doubles while the slab tiles of all
// planes still fit the CUs and every plane keeps at least 4 blocks of K; 1 when the slabs
// alone fill the GPU (qkv, gate_up at Qwen3-0.6B shapes). o_proj and down_proj at 64 rows
// (N = 1024: 64 slab tiles) take 4. The residual norm that adds the planes loads them all in
// one round: the config-5 step runs 18.84 k tok/s with 4 planes against 18.64 k with 2 and
// 18.72 k with 3 (with a norm that read the planes one after another, 2 beat 4: 17.99 k
// against 17.6 k).
extern "C" int64_t llmserve_int4_xfrag_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < kBlk) return 1;
  const int64_t tiles = pk_slabs(N) * ((M + kRows - 1) / kRows), nb = K / kBlk;
  const int64_t cus = device_cus();
  int64_t P = 1;
  while (P < kMaxPlanes && tiles * 2 * P <= cus && nb >= 4 * 2 * P) P *= 2;
  return P;
}

extern "C" int llmserve_int4_linear_gemm_xfrag_split(const void* xfrag, const void* packed,
                                                     float* y, int64_t M, int64_t N, int64_t K,
                                                     int64_t group_size, int64_t splits,
                                                     void* stream) {
  LSH_CHECK(splits >= 1 && splits <= kMaxPlanes,
            "int4_linear_gemm_xfrag_split: splits %lld not in [1, %d]", (long long)splits,
            kMaxPlanes);
  LSH_CHECK(M >= 0 && N >= 1 && K >= 1 && group_size >= 2,
            "int4_linear_gemm_xfrag_split: bad shape");
  LSH_CHECK(K % kBlk == 0 && group_size % kBlk == 0 && K % group_size == 0,
            "int4_linear_gemm_xfrag_split: K and group_size must be multiples of 128 (K %% group == 0)");
  LSH_CHECK(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && M * K < (1LL << 40) &&
                N * K < (1LL << 41) && splits * M * N < (1LL << 40),
            "int4_linear_gemm_xfrag_split: shape too large");
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(xfrag && packed && y, "int4_linear_gemm_xfrag_split: null pointer");
  LSH_CHECK(lsh::aligned16(xfrag) && lsh::aligned16(packed),
            "int4_linear_gemm_xfrag_split: the fragments and the packed weight must be 16-byte aligned");
  const int nb = static_cast<int>(K / kBlk);
  const int64_t mtiles = (M + kRows - 1) / kRows;
  const int mp = static_cast<int>(lsh::frag_rows(M));
  const __bf16* xf = static_cast<const __bf16*>(xfrag);
  const float* xsum = lsh::frag_sums(xf, mp, K);
  const uint8_t* wpk = static_cast<const uint8_t*>(packed);
  const float* spk = reinterpret_cast<const float*>(wpk + (pk_weight_bytes(N, K) + 255) / 256 * 256);
  Int4GemmArgs a{xf, nullptr, xsum, wpk, spk, nullptr, y, static_cast<int>(M),
                 static_cast<int>(N), static_cast<int>(K), static_cast<int>(K / group_size),
                 static_cast<int>(group_size / kBlk), mp};
  LSH_CHECK(launch_lat(a, pk_slabs(N), mtiles, nb, lsh::as_stream(stream), static_cast<int>(splits)),
            "int4_linear_gemm_xfrag_split: no kernel instance for M=%lld K=%lld", (long long)M,
            (long long)K);
  return lsh::launch_status("int4_linear_gemm_xfrag_split");
}
