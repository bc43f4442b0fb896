// Activation fragments of the batched int4 linear (int4_gemm_lat): x' = x * inv_act_scale
// split into three bf16 pieces hi = bf16(x'), mid = bf16(x' - hi), lo = bf16(x' - hi - mid),
// laid out in the order the matrix-core wavefronts read them, plus the channel sums of x' over
// every 128-channel block. Each difference is exact in fp32 and each piece takes the next 8
// significant bits, so hi + mid + lo equals x' to ~2^-26 relative: below fp32's own rounding,
// so that the products on the matrix cores are those of fp32 arithmetic (two pieces keep only
// ~2^-17, an error that 28 decoder layers amplify into the logits' third digit).
//
//   fragments: [row tile t][block b][step q][hi, mid, lo][lane][8 bf16]; lane = fr + 16 fc
//              holds row 16 t + fr, channels 128 b + 32 fc + 8 q .. + 8 (rows past M are
//              zero);
//   xsum:      [block][mp] fp32 after the fragments, mp = M rounded up to 16.
//
// Every producer (the split pass of llmserve_int4_linear_gemm_packed, the fused norms and
// silu * up) sums a block as the same pairwise tree over the 128 channels in index order, so
// their outputs are bit-identical for the same x'.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lsh {

constexpr int kFragBlk = 128;       // channels of a block
constexpr int kFragPieces = 3;      // hi, mid, lo
constexpr int kFragElems = 64 * 8;  // bf16 of one (step, piece) fragment

__host__ __device__ inline int64_t frag_rows(int64_t M) { return (M + 15) / 16 * 16; }

// Bytes of fragments + channel sums for M rows and K channels (K a multiple of 128).
inline int64_t frag_bytes(int64_t M, int64_t K) {
  return frag_rows(M) * K * 2 * kFragPieces + (K / kFragBlk) * frag_rows(M) * 4;
}

// The channel sums after the fragments of mp (padded) rows and K channels.
__host__ __device__ inline float* frag_sums(void* xf, int64_t mp, int64_t K) {
  return reinterpret_cast<float*>(static_cast<__bf16*>(xf) + kFragPieces * mp * K);
}
__host__ __device__ inline const float* frag_sums(const void* xf, int64_t mp, int64_t K) {
  return reinterpret_cast<const float*>(static_cast<const __bf16*>(xf) + kFragPieces * mp * K);
}

// Element offset of the hi value of x'[m, c] (mid and lo follow, kFragElems apart).
__device__ __forceinline__ int64_t frag_offset(int m, int c, int nblk) {
  const int t = m / 16, fr = m % 16, b = c / kFragBlk, cc = c % kFragBlk;
  const int fc = cc / 32, q = (cc % 32) / 8, e = cc % 8;
  return ((((static_cast<int64_t>(t) * nblk + b) * 4 + q) * kFragPieces) * 64 + fr + 16 * fc) * 8 + e;
}

// hi / mid / lo bf16 split (each difference exact in fp32; the sum equals v to ~2^-26).
// The differences and sums below must stay separately rounded: fused with the multiply that
// made v (x * inv), a difference would round differently in each producer. Every helper here
// turns floating-point contraction off.
__device__ __forceinline__ void split3_bf16(float v, __bf16& hi, __bf16& mid, __bf16& lo) {
#pragma clang fp contract(off)
  hi = static_cast<__bf16>(v);
  const float r = v - static_cast<float>(hi);
  mid = static_cast<__bf16>(r);
  lo = static_cast<__bf16>(r - static_cast<float>(mid));
}

// split3_bf16 of two values at once, each piece of the pair as one 32-bit word (a in the low
// half): one packed conversion per piece, whose halves are widened back to fp32 by shifting
// and masking the packed word (converting each value alone as well would double the
// conversions). Bit-identical to split3_bf16 of a and of b.
__device__ __forceinline__ void split3_bf16x2(float a, float b, uint32_t& hi, uint32_t& mid,
                                              uint32_t& lo) {
#pragma clang fp contract(off)
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  auto pk = [](float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x, y}, bf16x2));
  };
  auto lo_f = [](uint32_t w) { return __builtin_bit_cast(float, w << 16); };
  auto hi_f = [](uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); };
  hi = pk(a, b);
  const float ra = a - lo_f(hi), rb = b - hi_f(hi);
  mid = pk(ra, rb);
  lo = pk(ra - lo_f(mid), rb - hi_f(mid));
}

// The three pieces of N consecutive values as packed words (N / 2 words each).
template <int N>
__device__ __forceinline__ void split3_words(const float (&v)[N], uint32_t (&hi)[N / 2],
                                             uint32_t (&mid)[N / 2], uint32_t (&lo)[N / 2]) {
#pragma unroll
  for (int e = 0; e < N / 2; ++e) split3_bf16x2(v[2 * e], v[2 * e + 1], hi[e], mid[e], lo[e]);
}

// Writes N consecutive channels c .. c + N - 1 (within one 8-channel group) of row m.
template <int N>
__device__ __forceinline__ void frag_store(__bf16* xf, int m, int c, int nblk, const float (&v)[N]) {
  static_assert(N == 2 || N == 4 || N == 8, "frag_store: 2, 4 or 8 channels");
  uint32_t h[N / 2], md[N / 2], l[N / 2];
  split3_words<N>(v, h, md, l);
  __bf16* p = xf + frag_offset(m, c, nblk);
  if constexpr (N == 2) {
    *reinterpret_cast<uint32_t*>(p) = h[0];
    *reinterpret_cast<uint32_t*>(p + kFragElems) = md[0];
    *reinterpret_cast<uint32_t*>(p + 2 * kFragElems) = l[0];
  } else {
    typedef uint32_t uN __attribute__((ext_vector_type(N / 2)));
    uN hv, mv, lv;
#pragma unroll
    for (int e = 0; e < N / 2; ++e) {
      hv[e] = h[e];
      mv[e] = md[e];
      lv[e] = l[e];
    }
    *reinterpret_cast<uN*>(p) = hv;
    *reinterpret_cast<uN*>(p + kFragElems) = mv;
    *reinterpret_cast<uN*>(p + 2 * kFragElems) = lv;
  }
}

// Pairwise tree of N consecutive values in index order (the first levels of a block sum).
template <int N>
__device__ __forceinline__ float tree_sum(const float (&v)[N]) {
#pragma clang fp contract(off)
  if constexpr (N == 2) {
    return v[0] + v[1];
  } else if constexpr (N == 4) {
    return (v[0] + v[1]) + (v[2] + v[3]);
  } else {
    static_assert(N == 8, "tree_sum: 2, 4 or 8");
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
}

}  // namespace lsh
