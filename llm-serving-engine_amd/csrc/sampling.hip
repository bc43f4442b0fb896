// Batched token sampler on the device: the body of the reference's sampling.sample
// (sampling.py:151-189) for a logits batch already in HBM, one workgroup per row, in the
// reference's order:
//  1. presence / frequency penalties over the row's generated tokens, then the repetition
//     penalty over its prompt and generated tokens (apply_penalties, sampling.py:100-120),
//     written into the logits in place as the reference does;
//  2. the allowed set (every other token to -inf) and the banned tokens (-inf)
//     (sampling.py:165-170), also in place;
//  3. greedy rows (temperature < 1e-5): the first index of the row maximum, NaN above every
//     number (torch.argmax, sampling.py:169-174);
//  4. sampled rows: s = logits / temperature. When the batch uses top-k or top-p, the kept
//     tokens are the first L of the row in descending order of s (equal values by ascending
//     index), L the smaller of k and the number of tokens whose preceding mass under
//     softmax(s) over the whole row is below top_p (_top_k_top_p_min_p, sampling.py:123-143:
//     a token is dropped once the mass before it reaches top_p). When the batch uses min-p,
//     kept tokens whose probability under the softmax of the kept set is below min_p times
//     its largest are dropped. Then token = argmax p / E over the row, p the softmax of the
//     kept s and E the row's Exp(1) noise (the exponential race, sampling.py:183-187).
//
// The top-k / top-p cut is found without sorting: a radix select over the 32-bit
// order-preserving key of s, four passes of 8 bits from the top, each building a 256-bucket
// histogram of counts and of probability mass (fixed point, 2^-40 units, integer atomics, so
// the sums do not depend on the order the atomics land in) over the tokens whose key matches
// the digits chosen so far; the walk down the buckets stops at the first bucket where the
// count reaches k or the mass reaches top_p. The last level leaves a group of equal keys, of
// which the first n (by index, three more 8-bit passes over the index when the group is cut
// inside) are kept. The masses are summed in another order than the reference's sorted
// float32 cumsum, so a token whose preceding mass lies within rounding of top_p can fall on the
// other side of the cut; with top_p = 1 every token is kept (the reference's float cumsum can
// reach 1.0 before the last tokens and drop a few of the smallest).
#include "common.h"

namespace {

using lsh::kWave;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr double kFix = 1099511627776.0;  // 2^40: fixed-point unit of probability mass

struct SampleArgs {
  float* logits;  // [B, V], penalties and masks applied in place
  int64_t B, V;
  const float *temperature, *top_p, *min_p;  // [B]
  const int* top_k;                          // [B], -1: off
  const float *presence, *frequency, *repetition;  // [B]
  // CSR lists per row (offsets [B + 1]): generated tokens (distinct) with their counts, the
  // distinct prompt + generated tokens, the allowed set (row used only when has_allow[b]),
  // the banned tokens
  const int64_t *out_ptr, *out_ids;
  const int* out_cnt;
  const int64_t *seen_ptr, *seen_ids;
  const int64_t *allow_ptr, *allow_ids;
  const uint8_t* has_allow;
  const int64_t *ban_ptr, *ban_ids;
  const float* noise;         // [n, V] Exp(1) noise of the sampled rows
  const int64_t* noise_row;   // [B] row of `noise` for row b (sampled rows)
  int use_topkp, use_minp;    // the batch-wide switches of _top_k_top_p_min_p
  int64_t* tokens;            // [B]
};

// float -> uint32 with the same order (larger value, larger key)
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// x ranks above y for argmax: NaN above every number, else the larger value
__device__ __forceinline__ bool arg_above(float x, float y) {
  return x > y || (__builtin_isnan(x) && !__builtin_isnan(y));
}

__device__ __forceinline__ void arg_better(float& best, int64_t& idx, float ob, int64_t oi) {
  const bool same = ob == best || (__builtin_isnan(ob) && __builtin_isnan(best));
  if (arg_above(ob, best) || (same && oi < idx)) {
    best = ob;
    idx = oi;
  }
}

// Block argmax (first index among equal maxima); every thread gets the index.
__device__ int64_t block_argmax(float best, int64_t idx, float* fv, int64_t* iv) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1)
    arg_better(best, idx, __shfl_xor(best, d, kWave), __shfl_xor(idx, d, kWave));
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) {
    fv[wave] = best;
    iv[wave] = idx;
  }
  __syncthreads();
  best = fv[0];
  idx = iv[0];
  for (int w = 1; w < kWaves; ++w) arg_better(best, idx, fv[w], iv[w]);
  return idx;
}

// Block max / sum of one value per thread, the same bits in every thread (fixed order).
__device__ float block_max(float v, float* red) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) v = fmaxf(v, __shfl_xor(v, d, kWave));
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ float block_sum(float v, float* red) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) v += __shfl_xor(v, d, kWave);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kWaves; ++w) r += red[w];
  return r;
}

__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a) {
  extern __shared__ uint32_t allow_bits[];  // [V / 32] when a row has an allowed set
  __shared__ uint32_t hcount[256];
  __shared__ unsigned long long hmass[256];
  __shared__ float red[kWaves];
  __shared__ float fv[kWaves];
  __shared__ int64_t iv[kWaves];
  __shared__ uint32_t sel[4];
  __shared__ unsigned long long selm[2];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t V = a.V;
  float* row = a.logits + b * V;

  // 1. penalties (the reference's row skip: all three at their neutral values)
  const float pres = a.presence[b], freq = a.frequency[b], rep = a.repetition[b];
  if (pres != 0.f || freq != 0.f) {
    for (int64_t i = a.out_ptr[b] + tid; i < a.out_ptr[b + 1]; i += kThreads) {
      const int64_t t = a.out_ids[i];
      const float c = static_cast<float>(a.out_cnt[i]);
      if (t >= 0 && t < V)  // x - (f * count + p * (count > 0)), each operation rounded
        row[t] = __fsub_rn(row[t], __fadd_rn(__fmul_rn(freq, c), __fmul_rn(pres, c > 0.f ? 1.f : 0.f)));
    }
    __syncthreads();
  }
  if (rep != 1.f) {
    for (int64_t i = a.seen_ptr[b] + tid; i < a.seen_ptr[b + 1]; i += kThreads) {
      const int64_t t = a.seen_ids[i];
      if (t >= 0 && t < V) {
        const float v = row[t];
        row[t] = v > 0.f ? __fdiv_rn(v, rep) : __fmul_rn(v, rep);
      }
    }
    __syncthreads();
  }
  // 2. allowed set and banned tokens
  if (a.has_allow[b]) {
    const int64_t words = (V + 31) / 32;
    for (int64_t w = tid; w < words; w += kThreads) allow_bits[w] = 0u;
    __syncthreads();
    for (int64_t i = a.allow_ptr[b] + tid; i < a.allow_ptr[b + 1]; i += kThreads) {
      const int64_t t = a.allow_ids[i];
      if (t >= 0 && t < V) atomicOr(&allow_bits[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    for (int64_t j = tid; j < V; j += kThreads)
      if (!((allow_bits[j >> 5] >> (j & 31)) & 1u)) row[j] = -__builtin_inff();
    __syncthreads();
  }
  for (int64_t i = a.ban_ptr[b] + tid; i < a.ban_ptr[b + 1]; i += kThreads) {
    const int64_t t = a.ban_ids[i];
    if (t >= 0 && t < V) row[t] = -__builtin_inff();
  }
  __syncthreads();

  const float temp = a.temperature[b];
  if (temp < 1e-5f) {  // 3. greedy
    float best = -__builtin_inff();
    int64_t idx = V;
    for (int64_t j = tid; j < V; j += kThreads) {
      const float x = row[j];
      if (arg_above(x, best)) {
        best = x;
        idx = j;
      }
    }
    idx = block_argmax(best, idx, fv, iv);
    if (tid == 0) a.tokens[b] = idx < V ? idx : 0;
    return;
  }

  // 4. sampled rows
  auto sv = [&](int64_t j) { return __fdiv_rn(row[j], temp); };
  float m = -__builtin_inff();
  for (int64_t j = tid; j < V; j += kThreads) m = fmaxf(m, sv(j));
  m = block_max(m, red);

  // kept(j): key above kkey, or equal to it with index below kidx
  uint32_t kkey = 0u;
  int64_t kidx = V;  // every token kept
  if (a.use_topkp) {
    float z = 0.f;
    for (int64_t j = tid; j < V; j += kThreads) z += expf(sv(j) - m);
    z = block_sum(z, red);
    const int64_t klim = a.top_k[b] > 0 && a.top_k[b] < V ? a.top_k[b] : V;
    const float tp = a.top_p[b];
    const unsigned long long plim =
        tp >= 1.f ? ~0ull : static_cast<unsigned long long>(static_cast<double>(tp) * kFix);
    auto pfix = [&](int64_t j) {
      return static_cast<unsigned long long>(static_cast<double>(expf(sv(j) - m) / z) * kFix);
    };
    uint32_t prefix = 0u, pmask = 0u;
    uint32_t cnt_above = 0u;
    unsigned long long mass_above = 0ull;
    uint32_t tie_cnt = 0u;
    unsigned long long tie_mass = 0ull;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += kThreads) {
        hcount[i] = 0u;
        hmass[i] = 0ull;
      }
      __syncthreads();
      for (int64_t j = tid; j < V; j += kThreads) {
        const uint32_t key = order_key(sv(j));
        if ((key & pmask) == prefix) {
          const int bk = (key >> shift) & 255;
          atomicAdd(&hcount[bk], 1u);
          atomicAdd(&hmass[bk], pfix(j));
        }
      }
      __syncthreads();
      if (tid == 0) {
        // the first bucket (from the top) where the count reaches k or the mass reaches
        // top_p; the matching tokens always reach one of the two (their count reaches k at
        // the first level, and a bucket picked below holds all of the count or mass that
        // made its parent the pick), so the walk ends inside the loop
        int pick = -1, last = 0;
        for (int bk = 255; bk >= 0; --bk) {
          const uint32_t c = hcount[bk];
          const unsigned long long ms = hmass[bk];
          if (c == 0u) continue;
          last = bk;
          if (cnt_above + c >= klim || mass_above + ms >= plim) {
            pick = bk;
            break;
          }
          cnt_above += c;
          mass_above += ms;
        }
        if (pick < 0) {  // not reached (see above); keep the smallest bucket whole
          pick = last;
          cnt_above -= hcount[last];
          mass_above -= hmass[last];
        }
        sel[0] = static_cast<uint32_t>(pick);
        sel[1] = cnt_above;
        sel[2] = hcount[pick];
        selm[0] = mass_above;
        selm[1] = hmass[pick];
      }
      __syncthreads();
      prefix |= sel[0] << shift;
      pmask |= 255u << shift;
      cnt_above = sel[1];
      mass_above = selm[0];
      tie_cnt = sel[2];
      tie_mass = selm[1];
      __syncthreads();
    }
    // the group of equal keys `prefix`: n of its tie_cnt tokens are kept
    uint32_t n = tie_cnt;
    if (cnt_above + n > klim) n = static_cast<uint32_t>(klim - cnt_above);
    const unsigned long long pv = tie_cnt ? tie_mass / tie_cnt : 0ull;  // equal keys, equal p
    if (plim != ~0ull && pv > 0ull && mass_above + tie_mass >= plim) {
      // token i of the group (0-based) is kept while mass_above + i pv < plim
      const unsigned long long need = (plim - mass_above + pv - 1) / pv;
      if (need < n) n = static_cast<uint32_t>(need < 1 ? 1 : need);
    }
    kkey = prefix;
    kidx = V;
    if (n < tie_cnt) {  // cut inside the group: the n-th smallest index among its tokens
      uint32_t iprefix = 0u, imask = 0u, before = 0u;
      for (int shift = 16; shift >= 0; shift -= 8) {  // V < 2^24
        for (int i = tid; i < 256; i += kThreads) hcount[i] = 0u;
        __syncthreads();
        for (int64_t j = tid; j < V; j += kThreads) {
          const uint32_t jj = static_cast<uint32_t>(j);
          if (order_key(sv(j)) == prefix && (jj & imask) == iprefix)
            atomicAdd(&hcount[(jj >> shift) & 255], 1u);
        }
        __syncthreads();
        if (tid == 0) {
          int pick = 255;
          for (int bk = 0; bk < 256; ++bk) {
            if (before + hcount[bk] >= n) {
              pick = bk;
              break;
            }
            before += hcount[bk];
          }
          sel[0] = static_cast<uint32_t>(pick);
          sel[1] = before;
        }
        __syncthreads();
        iprefix |= sel[0] << shift;
        imask |= 255u << shift;
        before = sel[1];
        __syncthreads();
      }
      kidx = static_cast<int64_t>(iprefix) + 1;  // the n-th tie token is index iprefix
    }
  }
  auto kept = [&](int64_t j, float s) {
    if (!a.use_topkp) return true;
    const uint32_t key = order_key(s);
    return key > kkey || (key == kkey && j < kidx);
  };
  // min-p over the softmax of the kept set: p_j < max p * min_p is dropped
  const float mp = a.use_minp ? a.min_p[b] : 0.f;
  float pthr = -1.f, zk = 1.f;
  if (mp > 0.f) {
    float z = 0.f;
    for (int64_t j = tid; j < V; j += kThreads) {
      const float s = sv(j);
      if (kept(j, s)) z += expf(s - m);
    }
    zk = block_sum(z, red);
    pthr = __fmul_rn(1.f / zk, mp);  // the largest probability is exp(0) / zk
  }
  auto kept2 = [&](int64_t j, float s) {
    if (!kept(j, s)) return false;
    return pthr < 0.f || expf(s - m) / zk >= pthr;
  };
  float z = 0.f;
  for (int64_t j = tid; j < V; j += kThreads) {
    const float s = sv(j);
    if (kept2(j, s)) z += expf(s - m);
  }
  z = block_sum(z, red);
  const float* e = a.noise + a.noise_row[b] * V;
  float best = -__builtin_inff();
  int64_t idx = V;
  for (int64_t j = tid; j < V; j += kThreads) {
    const float s = sv(j);
    const float p = kept2(j, s) ? expf(s - m) / z : 0.f;
    const float q = p / e[j];
    if (arg_above(q, best)) {
      best = q;
      idx = j;
    }
  }
  idx = block_argmax(best, idx, fv, iv);
  if (tid == 0) a.tokens[b] = idx < V ? idx : 0;
}

}  // namespace

extern "C" int llmserve_sample(
    float* logits, int64_t B, int64_t V, const float* temperature, const int* top_k,
    const float* top_p, const float* min_p, const float* presence, const float* frequency,
    const float* repetition, const int64_t* out_ptr, const int64_t* out_ids, const int* out_cnt,
    const int64_t* seen_ptr, const int64_t* seen_ids, const int64_t* allow_ptr,
    const int64_t* allow_ids, const uint8_t* has_allow, const int64_t* ban_ptr,
    const int64_t* ban_ids, const float* noise, const int64_t* noise_row, int use_topkp,
    int use_minp, int64_t* tokens, void* stream) {
  LSH_CHECK(B >= 0 && V >= 1 && V < (1LL << 24), "sample: 1 <= V < 2^24 (got %lld)", (long long)V);
  if (B == 0) return LLMSERVE_OK;
  LSH_CHECK(logits && temperature && top_k && top_p && min_p && presence && frequency &&
                repetition && out_ptr && seen_ptr && allow_ptr && has_allow && ban_ptr &&
                noise_row && tokens,
            "sample: null pointer");
  LSH_CHECK(noise != nullptr, "sample: null noise (pass any [1, V] buffer when every row is greedy)");
  const size_t lds = static_cast<size_t>((V + 31) / 32) * sizeof(uint32_t);
  LSH_CHECK(lds <= 64 * 1024, "sample: V = %lld needs more LDS for the allowed-set mask",
            (long long)V);
  SampleArgs a{logits, B, V, temperature, top_p, min_p, top_k, presence, frequency, repetition,
               out_ptr, out_ids, out_cnt, seen_ptr, seen_ids, allow_ptr, allow_ids, has_allow,
               ban_ptr, ban_ids, noise, noise_row, use_topkp, use_minp, tokens};
  lsh::launch(sample_kernel, dim3(static_cast<unsigned>(B)), dim3(kThreads), lds,
              lsh::as_stream(stream), true, a);
  return lsh::launch_status("sample");
}
