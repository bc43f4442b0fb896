// int8-KV paged decode attention: the context split evenly over the GPU's wavefronts, an
// online softmax per wavefront, and a merge of the sequences that were split.
//
// Work split: the kv heads form NHG groups of HB heads (HB = the largest divisor of Hk up to
// 8). Each (sequence b, head group hg) unit is cut into ranges of at most Q tokens that never
// straddle two units; Q is chosen so that the ranges fit the W resident workgroups (the work
// plan below; or a caller-fixed range size). A workgroup holds HB wavefronts, one per kv head of
// the group, which run the same tokens: together they read whole HB * D-byte pieces of every
// slot row (all of it when HB = Hk), so the cache streams in long contiguous runs. A range that
// is its unit's only one writes the output rows; the others write a partial (running max, sum,
// acc) per head to slot (u * kcap + k) * HB + head-in-group (unit u, range k of the unit, kcap
// slots per unit), and the merge kernel combines the partials of every split unit.
//
// Lane layout inside a wavefront (D = head dim, LPR = D / 16 lanes per token row):
//   lane = r * LPR + seg : row slot r of the RPW = 64 / LPR tokens of one step, dims
//                          [16 seg, 16 seg + 16) of that token.
// Step k covers tokens [k RPW, (k + 1) RPW) of the sequence; each lane loads 16 bytes of its
// token's K row and 16 bytes of its V row (one dwordx4 each, non-temporal) and the row's two
// scales. When the block size is a multiple of RPW a step lies inside one cache block, its
// block id is wave-uniform (read from the lane holding it) and the slot arithmetic is
// scalar; otherwise each lane fetches its own block id with a lane shuffle.
// Every row slot runs its own online softmax over the tokens it sees, so a step needs no
// cross-row communication:
//   * q.k: 16-dim partial dot per query head, summed over the LPR lanes of the row with DPP;
//     q is pre-scaled by scale * log2(e), so scores are in log2 units and p = exp2(s - m);
//   * the running max is raised only when a score exceeds it by more than kLazy2 (p stays
//     <= e^8); the rescale of (sum, acc) then runs under a wave-uniform branch;
//   * acc += (p * v_scale) * v_int8 in the lane's 16 dims.
// Up to four steps of K/V loads are kept in flight (a ring of registers, refilled as each
// step is consumed). Block ids are read in windows of 64 (one per lane). At the end the RPW
// row-slot states are merged with DPP / lane shuffles.
// The scores are the reference's s = (scale * k_scale) * (q . k_int8) and the values
// acc += (p * v_scale) * v_int8 (paged_attention.cpp:301-355), up to the order of the
// float operations (scale folded into q; exp2 of log2-unit scores).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "paged_core.h"
#include "xfrag.h"

namespace {

using lsh::kWave;
constexpr int kMaxHeadsPerBlock = 8;  // wavefronts of a decode workgroup (HB <= 8)
constexpr int kMergeWaves = 4;        // wavefronts of a merge workgroup
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// ---- the work plan ------------------------------------------------------------------------------
// Ranges never straddle two (sequence b, head group hg) units: unit (b, hg) gets
// n_b = ceil(ctx_b / Q) ranges, numbered unit by unit in (b, hg) order. With a caller's fixed
// partition size P (the reference's partitions) Q = P and the ranges hold P tokens, the last
// one the rest. The balanced default chooses Q, a multiple of kMinRange, between
// max(ceil(T / W), kMinRange, ceil(max ctx / kcap)), T = NHG * sum_b ctx_b, kcap the partial
// slots per unit, and ceil(T / (W - units)) (which always fits: each unit rounds up by less
// than one range) so that the R = NHG * sum_b n_b ranges fit the W resident workgroups: the
// lower end if it fits, else the feasible end of kPlanSteps bisections; its ranges then hold Q
// tokens as a fixed partition's do. (Ranges equalised within each unit, ceil(ctx_b / n_b)
// tokens, with Q to the token, measured slower: config 4 57.3-58.9 against 55.7-56.0 us per
// decode + merge; 64 rows of U[1024, 4096] 73.9-74.7 against 72.1.) Every workgroup derives the same plan from
// the contexts, with DPP / readlane reductions (no LDS crossbar round trips: the plan is on
// every range's critical path). A range that started a second unit would pay that unit's
// start-up (its context, then q and block ids, then the first K/V loads) as dependent round
// trips in a saturated memory system, microseconds each: measured, ranges that crossed a
// sequence boundary ended ~10 us after the others.
constexpr uint32_t kMinRange = 64;
constexpr int kPlanSteps = 5;

template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {  // lanes without a source get 0
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROWS, 0xF, false));
}

// Inclusive prefix sum over the wavefront's lanes (row shifts, then row broadcasts).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += dpp_u32<0x111, 0xF>(v);  // row_shr:1
  v += dpp_u32<0x112, 0xF>(v);  // row_shr:2
  v += dpp_u32<0x114, 0xF>(v);  // row_shr:4
  v += dpp_u32<0x118, 0xF>(v);  // row_shr:8
  v += dpp_u32<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
  v += dpp_u32<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
  return v;
}

// Sum over the wavefront (wave-uniform).
__device__ __forceinline__ uint32_t wave_total_u32(uint32_t v) {
  return __builtin_amdgcn_readlane(wave_scan_u32(v), kWave - 1);
}

// Max over the wavefront (wave-uniform): row mirrors, then the four rows' lanes.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  v = mx(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, true)));
  v = mx(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4E, 0xF, 0xF, true)));
  v = mx(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x141, 0xF, 0xF, true)));
  v = mx(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x140, 0xF, 0xF, true)));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return mx(mx(r0, r1), mx(r2, r3));
}

// Context of row b0 + lane (0 past B); contexts are below 2^31 (checked on the host).
__device__ __forceinline__ uint32_t lane_ctx(const DecodeArgs& a, int b0) {
  const int b = b0 + static_cast<int>(threadIdx.x % kWave);
  return b < a.B ? static_cast<uint32_t>(seq_ctx(a, b)) : 0u;
}

__device__ __forceinline__ uint32_t ranges_of(uint32_t c, uint32_t Q) {
  return c == 0 ? 0u : (c - 1) / Q + 1;
}

struct Plan {
  uint32_t Q;   // range size bound (fixed partition: the range size)
  int64_t R;    // ranges
  bool fixed;
  uint32_t c0;  // context of row `lane` when B <= 64 (held for the range lookups)
};

// NHG * sum_b ceil(ctx_b / Q) (wave-uniform). One row per lane up to 64 rows: with Q >= 64 the
// 64 counts sum below 2^31.
__device__ int64_t count_ranges(const DecodeArgs& a, uint32_t Q, uint32_t c0) {
  if (a.B <= kWave && Q >= kMinRange)
    return static_cast<int64_t>(wave_total_u32(ranges_of(c0, Q))) * a.NHG;
  int64_t s = 0;
  for (int b0 = 0; b0 < a.B; b0 += kWave)
    s += uniform64(wave_sum_i64(ranges_of(a.B <= kWave ? c0 : lane_ctx(a, b0), Q)));
  return s * a.NHG;
}

__device__ Plan make_plan(const DecodeArgs& a) {
  Plan p;
  p.c0 = a.B <= kWave ? lane_ctx(a, 0) : 0u;
  if (a.range > 0) {
    p.Q = static_cast<uint32_t>(a.range < 0x7fffffff ? a.range : 0x7fffffff);
    p.R = count_ranges(a, p.Q, p.c0);
    p.fixed = true;
    return p;
  }
  p.fixed = false;
  int64_t tot = 0, nz = 0;
  uint32_t mx = 0;
  for (int b0 = 0; b0 < a.B; b0 += kWave) {
    const uint32_t c = a.B <= kWave ? p.c0 : lane_ctx(a, b0);
    tot += uniform64(wave_sum_i64(c));
    nz += wave_total_u32(c != 0 ? 1u : 0u);
    const uint32_t m = wave_max_u32(c);
    mx = m > mx ? m : mx;
  }
  const int64_t T = tot * a.NHG, units = nz * a.NHG;
  const int64_t even = (T + a.W - 1) / a.W;
  uint32_t lo = even > kMinRange ? static_cast<uint32_t>(even < 0x7fffffff ? even : 0x7fffffff)
                                 : kMinRange;
  const uint32_t fit = (mx + static_cast<uint32_t>(a.kcap) - 1) / static_cast<uint32_t>(a.kcap);
  if (fit > lo) lo = fit;  // the longest unit's ranges fit its kcap partial slots
  if (lo >= mx) {
    p.Q = lo;  // every unit is one range
  } else if (units >= a.W) {
    p.Q = mx;  // the units alone fill the workgroups: one range each, workgroups loop
  } else {
    const int64_t f = (T + (a.W - units) - 1) / (a.W - units);
    uint32_t hi = f < mx ? static_cast<uint32_t>(f) : mx;  // fits
    if (hi < lo) hi = lo;
    // Q in whole multiples of kMinRange (rounding up keeps a bound feasible: the range count
    // only falls as Q grows)
    lo = (lo + kMinRange - 1) / kMinRange * kMinRange;
    hi = (hi + kMinRange - 1) / kMinRange * kMinRange;
    if (count_ranges(a, lo, p.c0) <= a.W) {
      hi = lo;
    } else {
      for (int it = 0; it < kPlanSteps && lo + kMinRange < hi; ++it) {  // (lo infeasible, hi feasible)
        const uint32_t mid = lo + (hi - lo) / kMinRange / 2 * kMinRange;
        if (count_ranges(a, mid, p.c0) <= a.W)
          hi = mid;
        else
          lo = mid;
      }
    }
    p.Q = hi;
  }
  p.R = count_ranges(a, p.Q, p.c0);
  return p;
}

// Range j of the plan: unit (b, hg), its tokens [t0, t1) and its unit's number of ranges n.
struct RangePos {
  int b, hg;
  int t0, t1;
  uint32_t n, k;  // the unit's ranges, this range's index among them
};

__device__ RangePos find_range(const DecodeArgs& a, const Plan& p, int64_t j) {
  const int lane = threadIdx.x % kWave;
  int64_t base = 0;
  for (int b0 = 0; b0 < a.B; b0 += kWave) {
    const uint32_t c = a.B <= kWave ? p.c0 : lane_ctx(a, b0);
    const uint32_t n = ranges_of(c, p.Q);
    int64_t incl;
    if (a.B <= kWave && !p.fixed) {
      incl = static_cast<int64_t>(wave_scan_u32(n)) * a.NHG;  // below 2^31 (see count_ranges)
    } else {
      incl = static_cast<int64_t>(n) * a.NHG;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const int64_t u = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += u;
      }
    }
    const uint64_t hit = __ballot(b0 + lane < a.B && base + incl > j);
    if (hit != 0) {
      const int i = __builtin_ctzll(hit);
      RangePos r;
      r.b = b0 + i;
      const uint32_t cb = __builtin_amdgcn_readlane(c, i);
      r.n = __builtin_amdgcn_readlane(n, i);
      if (r.n == 0) break;  // unreachable: the first row whose prefix passes j has ranges
      const int64_t pre = base + uniform64(__shfl(incl, i, kWave)) - static_cast<int64_t>(r.n) * a.NHG;
      const int64_t rel = j - pre;
      if (rel < 0 || rel >= static_cast<int64_t>(r.n) * a.NHG) break;  // unreachable
      r.hg = static_cast<int>(rel / r.n);
      const uint32_t k = static_cast<uint32_t>(rel - static_cast<int64_t>(r.hg) * r.n);
      const uint32_t L = p.Q;  // ranges of Q tokens, the unit's last one the rest
      const uint32_t t0 = k * L, t1 = t0 + L < cb ? t0 + L : cb;
      r.t0 = static_cast<int>(t0);
      r.t1 = static_cast<int>(t1);
      r.k = k;
      return r;
    }
    base += uniform64(__shfl(incl, kWave - 1, kWave));
  }
  return RangePos{a.B, 0, 0, 0, 0, 0};  // unreachable for j < R
}

// Runs tokens [t0, t1) of (b, h) and writes the output rows (whole) or partial `slot`.
template <typename E, int D, int G, bool kScalarBlk, bool kOff32>
__device__ __forceinline__ void decode_segment(const DecodeArgs& a, int b, int h, int t0, int t1,
                                               bool whole, int64_t slot) {
  constexpr int LPR = D / 16;
  const int lane = threadIdx.x % kWave;
  const int r = lane / LPR, seg = lane % LPR;
  SegState<G> s;
  segment_state<E, D, G, kScalarBlk, kOff32>(a, b, h, t0, t1, s);
  const float(&m)[G] = s.m;
  const float(&lt)[G] = s.lt;
  const float(&acc)[G][16] = s.acc;
  if (whole) {
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float inv = 1.f / lt[g];
        float4* o = reinterpret_cast<float4*>(
            a.out + (static_cast<int64_t>(b) * a.Hq + h * G + g) * D + seg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = make_float4(acc[g][4 * i] * inv, acc[g][4 * i + 1] * inv, acc[g][4 * i + 2] * inv,
                             acc[g][4 * i + 3] * inv);
      }
    }
    return;
  }
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4* o = reinterpret_cast<float4*>(a.part_acc + (slot * G + g) * D + seg * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = make_float4(acc[g][4 * i], acc[g][4 * i + 1], acc[g][4 * i + 2], acc[g][4 * i + 3]);
    }
  }
  if (lane < G) {
    float mm = m[0], ll = lt[0];
#pragma unroll
    for (int g = 1; g < G; ++g)
      if (lane == g) {
        mm = m[g];
        ll = lt[g];
      }
    a.part_ml[(slot * G + lane) * 2] = mm;
    a.part_ml[(slot * G + lane) * 2 + 1] = ll;
  }
}

// Decode kernel: workgroup w runs work ranges w, w + W, ... (one range each with the
// balanced default unless the units outnumber the workgroups); its wavefront i takes kv head
// hg * HB + i. Waves proceed independently (no barriers). A range that is its unit's only one
// writes the output rows, the others their partial at slot (u * kcap + k) * HB + i (unit
// u = b * NHG + hg, k its range in the unit), and the unit's first range records n, so that
// the merge finds the partials without the plan.
template <typename E, int D, int G, bool kScalarBlk, bool kOff32>
__global__ __launch_bounds__(kMaxHeadsPerBlock * kWave) void paged_decode_kernel(DecodeArgs a) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const Plan p = make_plan(a);
  for (int64_t j = blockIdx.x; j < p.R; j += a.W) {
    const RangePos rp = find_range(a, p, j);
    if (rp.b >= a.B) continue;  // unreachable for j < R
    const int64_t u = static_cast<int64_t>(rp.b) * a.NHG + rp.hg;
    if (rp.k == 0 && threadIdx.x == 0) a.unit_n[u] = static_cast<int>(rp.n);
    decode_segment<E, D, G, kScalarBlk, kOff32>(a, rp.b, rp.hg * a.HB + wave, rp.t0, rp.t1,
                                                rp.n == 1, (u * a.kcap + rp.k) * a.HB + wave);
  }
}

// Merge of the split units (paged_attention.cpp:432-455): one wavefront per (b, q head).
//   M = max_j m_j;  w_j = exp2(m_j - M);  out = sum_j w_j acc_j / sum_j w_j l_j  (l_j = 0 skipped)
// A unit's partials sit at slots (u * kcap + k) * HB + head-in-group, k < n, and the decode
// kernel records n in unit_n[u], so one round of loads brings everything the merge needs: the
// row's context (a zero context gives NaN, the reference's 0 * (1 / 0)), n (1: the unit was
// written whole), the (m, l) of the first 64 slots and the accumulator rows of the first
// kMergeBatch, taken speculatively up to kcap and masked once n is known.
constexpr int kMergeBatch = 16;

// What a merge wavefront loaded: the row's context, the unit's n, and (for n >= 2) the merged
// accumulators of this lane's N elements in o with L = sum_j w_j l_j (the same bits in every
// lane). ml(p) points at (m, l) of partial p; row(p) at this lane's first accumulator element
// of partial p, its N elements STEP floats apart.
struct UnitMerge {
  int64_t ctx;
  int n;
  float L;
};

template <int N, int STEP, typename ML, typename ROW>
__device__ __forceinline__ UnitMerge merge_unit(const DecodeArgs& a, int b, int64_t u, ML ml,
                                                ROW row, float (&o)[N]) {
  const int lane = threadIdx.x % kWave;
  const int kcap = a.kcap;
  // one round: context, n, the first (m, l) pairs and accumulator rows (slots below kcap)
  const int64_t ctx = seq_ctx(a, b);
  const int n_raw = a.unit_n[u];
  float v0[kMergeBatch][N];
#pragma unroll
  for (int j = 0; j < kMergeBatch; ++j) {
    const float* src = row(j < kcap ? j : kcap - 1);
#pragma unroll
    for (int e = 0; e < N; ++e) v0[j][e] = src[e * STEP];
  }
  float m0 = kNegBig, l0 = 0.f;
  if (lane < kcap) {
    m0 = ml(lane)[0];
    l0 = ml(lane)[1];
  }
  UnitMerge r;
  r.ctx = uniform64(ctx);
  r.n = __builtin_amdgcn_readfirstlane(n_raw);
  r.L = 0.f;
  if (r.ctx == 0 || r.n <= 1) return r;
  const int np = r.n < kcap ? r.n : kcap;
  if (lane >= np) {  // slots past the unit's ranges hold older partials
    m0 = kNegBig;
    l0 = 0.f;
  }
  float M = m0;
  for (int p = lane + kWave; p < np; p += kWave) M = fmaxf(M, ml(p)[0]);
  M = lsh::wave_max_from<1>(M);
  float L = 0.f;
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = 0.f;
  for (int p0 = 0; p0 < np; p0 += kWave) {
    float w = 0.f;
    if (p0 + lane < np) {
      const float mp = p0 == 0 ? m0 : ml(p0 + lane)[0];
      const float lp = p0 == 0 ? l0 : ml(p0 + lane)[1];
      w = lp == 0.f ? 0.f : __builtin_amdgcn_exp2f(mp - M);
      L += w * lp;
    }
    const int n = np - p0 < kWave ? np - p0 : kWave;
    for (int j0b = 0; j0b < n; j0b += kMergeBatch) {
      float v[kMergeBatch][N];
      if (p0 == 0 && j0b == 0) {
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
#pragma unroll
          for (int e = 0; e < N; ++e) v[j][e] = j < n ? v0[j][e] : 0.f;
      } else {
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          const float* src = row(p0 + (j0b + j < n ? j0b + j : n - 1));
#pragma unroll
          for (int e = 0; e < N; ++e) v[j][e] = src[e * STEP];
        }
      }
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        const float wj = j0b + j < n ? __shfl(w, j0b + j, kWave) : 0.f;
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] += wj * v[j][e];
      }
    }
  }
  r.L = lsh::group_sum<kWave>(L);  // the same bits in every lane (xor / mirror steps)
  return r;
}

template <int D>
__global__ __launch_bounds__(kMergeWaves * kWave) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int PER = (D + kWave - 1) / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kMergeWaves +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if (item >= static_cast<int64_t>(a.B) * a.Hq) return;
  const int b = static_cast<int>(item / a.Hq), hq = static_cast<int>(item % a.Hq);
  const int G = a.Hq / a.Hk;
  const int h = hq / G, g = hq % G;
  float* out = a.out + item * D;
  // partial k of unit u: slot (u * kcap + k) * HB + h % HB; lane holds dims lane + 64 i
  const int64_t u = static_cast<int64_t>(b) * a.NHG + h / a.HB;
  const int64_t base = u * a.kcap * a.HB + h % a.HB;
  const int dl = lane < D ? lane : 0;  // D < 64: lanes past D read dim 0 and write nothing
  float o[PER];
  const UnitMerge r = merge_unit<PER, kWave>(
      a, b, u, [&](int p) { return a.part_ml + ((base + static_cast<int64_t>(p) * a.HB) * G + g) * 2; },
      [&](int p) { return a.part_acc + ((base + static_cast<int64_t>(p) * a.HB) * G + g) * D + dl; },
      o);
  if (r.ctx == 0) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + i * kWave < D) out[lane + i * kWave] = __builtin_nanf("");
    return;
  }
  if (r.n <= 1) return;  // written whole by the decode kernel
  const float inv = 1.f / r.L;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + i * kWave;
    if (d < D) out[d] = o[i] * inv;
  }
}
template <int D>
__global__ __launch_bounds__(kMergeWaves * kWave) void paged_decode_merge_frag_kernel(
    DecodeArgs a, const float* __restrict__ act_inv, __bf16* __restrict__ xf,
    float* __restrict__ xsum, int mp) {
  static_assert(D == 128 || D == 256, "fragment merge: D = 128 or 256");
  constexpr int CPL = D / kWave;              // channels per lane: 2 or 4
  constexpr int LPB = lsh::kFragBlk / CPL;    // lanes per 128-channel block: 64 or 32
  const int lane = threadIdx.x % kWave;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kMergeWaves +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if (item >= static_cast<int64_t>(mp) * a.Hq) return;
  const int b = static_cast<int>(item / a.Hq), hq = static_cast<int>(item % a.Hq);
  const int nblk = a.Hq * D / lsh::kFragBlk;
  const int c0 = hq * D + lane * CPL;  // first channel of this lane in the [B, Hq * D] row
  float x[CPL];
  if (b >= a.B) {
#pragma unroll
    for (int e = 0; e < CPL; ++e) x[e] = 0.f;
  } else {
    const int G = a.Hq / a.Hk;
    const int h = hq / G, g = hq % G;
    float* out = a.out + item * D + lane * CPL;
    const int64_t u = static_cast<int64_t>(b) * a.NHG + h / a.HB;
    const int64_t base = u * a.kcap * a.HB + h % a.HB;
    float whole[CPL];  // the row as the decode kernel wrote it when the unit had one range
#pragma unroll
    for (int e = 0; e < CPL; ++e) whole[e] = out[e];
    float o[CPL];
    const UnitMerge r = merge_unit<CPL, 1>(
        a, b, u, [&](int p) { return a.part_ml + ((base + static_cast<int64_t>(p) * a.HB) * G + g) * 2; },
        [&](int p) {
          return a.part_acc + ((base + static_cast<int64_t>(p) * a.HB) * G + g) * D + lane * CPL;
        },
        o);
    if (r.ctx == 0) {
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        x[e] = __builtin_nanf("");
        out[e] = x[e];
      }
    } else if (r.n <= 1) {  // written whole by the decode kernel
#pragma unroll
      for (int e = 0; e < CPL; ++e) x[e] = whole[e];
    } else {
      const float inv = 1.f / r.L;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        x[e] = o[e] * inv;
        out[e] = x[e];
      }
    }
    if (act_inv) {
#pragma unroll
      for (int e = 0; e < CPL; ++e) x[e] = __fmul_rn(x[e], act_inv[c0 + e]);
    }
  }
  lsh::frag_store<CPL>(xf, b, c0, nblk, x);
  const float sum = lsh::group_sum<LPB>(lsh::tree_sum<CPL>(x));
  if (lane % LPB == 0) xsum[static_cast<int64_t>(c0 / lsh::kFragBlk) * mp + b] = sum;
}

// Resident workgroups of `waves` wavefronts of `Kernel` on the current device: CUs x blocks
// per CU (cached per kernel -- one instantiation each --, device and workgroup size).
template <auto Kernel>
int resident_blocks(int waves) {
  static int cached[64][kMaxHeadsPerBlock + 1] = {};  // [device][waves]
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev][waves] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, Kernel, waves * kWave, 0) != hipSuccess ||
        per < 1)
      per = 1;
    cached[dev][waves] = cus * per;
  }
  return cached[dev][waves];
}

// kv heads per decode workgroup: the largest divisor of Hk up to kMaxHeadsPerBlock.
int heads_per_block(int64_t Hk) {
  for (int hb = kMaxHeadsPerBlock; hb > 1; --hb)
    if (Hk % hb == 0) return hb;
  return 1;
}

// A step's block id is wave-uniform when each step lies inside one cache block (block size a
// power of two and a multiple of the rows per step).
bool scalar_blocks(int64_t D, int64_t block_size) {
  return (block_size & (block_size - 1)) == 0 && block_size % (kWave / (D / 16)) == 0;
}

// Workgroups of the decode grid (all resident at once) of the variant that runs; off32 < 0:
// the larger of the two scalar-block variants (the workspace bound, which does not know the
// cache size).
template <typename E, int D, int G>
int decode_blocks(bool scalar, int off32, int hb) {
  if (!scalar) return resident_blocks<paged_decode_kernel<E, D, G, false, false>>(hb);
  const int w32 = resident_blocks<paged_decode_kernel<E, D, G, true, true>>(hb);
  const int w64 = resident_blocks<paged_decode_kernel<E, D, G, true, false>>(hb);
  return off32 > 0 ? w32 : (off32 == 0 ? w64 : (w32 > w64 ? w32 : w64));
}

// Fragment output of the merge (nullptr: the plain merge writes out only).
struct FragOut {
  const float* act_inv;
  void* xfrag;
};

template <typename E, int D, int G>
void launch_decode(const DecodeArgs& a, bool scalar, bool off32, const FragOut& fo, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.W)), block(a.HB * kWave);
  if (scalar && off32)
    lsh::launch(paged_decode_kernel<E, D, G, true, true>, grid, block, 0, st, false, a);
  else if (scalar)
    lsh::launch(paged_decode_kernel<E, D, G, true, false>, grid, block, 0, st, false, a);
  else
    lsh::launch(paged_decode_kernel<E, D, G, false, false>, grid, block, 0, st, false, a);
  if constexpr (D == 128 || D == 256) {
    if (fo.xfrag != nullptr) {
      const int mp = static_cast<int>(lsh::frag_rows(a.B));
      const int64_t K = static_cast<int64_t>(a.Hq) * D;
      __bf16* xf = static_cast<__bf16*>(fo.xfrag);
      float* xsum = lsh::frag_sums(xf, mp, K);
      const int64_t items = static_cast<int64_t>(mp) * a.Hq;
      lsh::launch(paged_decode_merge_frag_kernel<D>,
                  dim3(static_cast<unsigned>((items + kMergeWaves - 1) / kMergeWaves)),
                  dim3(kMergeWaves * kWave), 0, st, true, a, fo.act_inv, xf, xsum, mp);
      return;
    }
  }
  const int64_t items = static_cast<int64_t>(a.B) * a.Hq;
  lsh::launch(paged_decode_merge_kernel<D>,
              dim3(static_cast<unsigned>((items + kMergeWaves - 1) / kMergeWaves)),
              dim3(kMergeWaves * kWave), 0, st, true, a);
}

// Calls f.template operator()<D, G>() for the runtime (D, G); false when unsupported.
template <typename F>
bool with_shape(int64_t D, int64_t G, F&& f) {
  auto g_switch = [&](auto dtag) {
    constexpr int Dv = decltype(dtag)::value;
    switch (G) {
      case 1: f.template operator()<Dv, 1>(); return true;
      case 2: f.template operator()<Dv, 2>(); return true;
      case 3: f.template operator()<Dv, 3>(); return true;
      case 4: f.template operator()<Dv, 4>(); return true;
      case 5: f.template operator()<Dv, 5>(); return true;
      case 6: f.template operator()<Dv, 6>(); return true;
      case 7: f.template operator()<Dv, 7>(); return true;
      case 8: f.template operator()<Dv, 8>(); return true;
      default: return false;
    }
  };
  switch (D) {
    case 16: return g_switch(std::integral_constant<int, 16>{});
    case 32: return g_switch(std::integral_constant<int, 32>{});
    case 64: return g_switch(std::integral_constant<int, 64>{});
    case 128: return g_switch(std::integral_constant<int, 128>{});
    case 256: return g_switch(std::integral_constant<int, 256>{});
    default: return false;
  }
}

// Decode workgroups for a cache of `elem_bytes`-byte elements (1: int8, 4: fp32; 0: the
// larger of the two, for workspace bounds that do not know the cache type).
int grid_blocks(int64_t D, int64_t G, int64_t Hk, int64_t block_size, int off32 = -1,
                int elem_bytes = 0) {
  int w8 = 0, w32 = 0;
  const bool scalar = scalar_blocks(D, block_size);
  const int hb = heads_per_block(Hk);
  with_shape(D, G, [&]<int Dv, int Gv>() {
    if (elem_bytes != 4) w8 = decode_blocks<int8_t, Dv, Gv>(scalar, off32, hb);
    if (elem_bytes != 1) w32 = decode_blocks<float, Dv, Gv>(scalar, off32, hb);
  });
  return w8 > w32 ? w8 : w32;
}

// Partial slots per (b, head group) unit: a bound on its ranges. A fixed range size P gives
// at most ceil(max context / P). The balanced plan's ranges hold at least kMinRange tokens,
// number at most the resident workgroups W, and the plan raises its range size until the
// longest unit fits kBalanceSlack x (its fair share W / units) + 1 slots: a unit up to
// kBalanceSlack x the mean context splits as the balance asks, and the workspace stays near
// kBalanceSlack x W slots for any batch.
constexpr int64_t kBalanceSlack = 4;

int64_t unit_slots(int64_t B, int64_t D, int64_t G, int64_t Hk, int64_t max_blocks,
                   int64_t block_size, int64_t partition_size) {
  const int64_t cap = max_blocks * block_size;
  if (partition_size > 0) return std::max<int64_t>(1, (cap + partition_size - 1) / partition_size);
  const int64_t w = grid_blocks(D, G, Hk, block_size);
  const int64_t units = B * (Hk / heads_per_block(Hk));
  const int64_t fair = (kBalanceSlack * w + units - 1) / units + 1;
  return std::max<int64_t>(1, std::min({w, (cap + kMinRange - 1) / kMinRange, fair}));
}

// Partial slots the workspace holds: HB per (unit, range in unit).
int64_t partial_slots(int64_t B, int64_t Hk, int64_t D, int64_t G, int64_t max_blocks,
                      int64_t block_size, int64_t partition_size) {
  const int64_t hb = heads_per_block(Hk), nhg = Hk / hb;
  return B * nhg * unit_slots(B, D, G, Hk, max_blocks, block_size, partition_size) * hb;
}

}  // namespace

extern "C" int64_t llmserve_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hk,
                                                            int64_t D, int64_t max_blocks,
                                                            int64_t block_size,
                                                            int64_t partition_size) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || D <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  if (Hq % Hk != 0 || Hq / Hk > 8) return 0;
  const int64_t G = Hq / Hk;
  const int64_t slots = partial_slots(B, Hk, D, G, max_blocks, block_size, partition_size);
  const int64_t units = B * (Hk / heads_per_block(Hk));
  return slots * G * (D + 2) * static_cast<int64_t>(sizeof(float)) + units * 4;
}

namespace {

// The cache a call attends over: int8 with per-(slot, head) scales, or fp32 (no scales).
struct CacheView {
  const void* k;
  const void* v;
  const float* k_scale;  // int8 only
  const float* v_scale;
  int elem_bytes;  // 1 or 4
};

// Query rows -> block-table rows (nullable: row b uses table row b).
struct RowMap {
  const int64_t* row_table;
  int64_t table_rows;
};

int decode_paged(const float* q, const CacheView& c, const int64_t* block_tables,
                 const RowMap& rows, const int64_t* context_lens, float* out, int64_t B,
                 int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
                 int64_t block_size, float scale, int64_t partition_size, const float* q_mult,
                 const FragOut& fo, void* workspace, int64_t workspace_bytes, void* stream) {
  LSH_CHECK(B >= 0 && Hq >= 1 && Hk >= 1 && D >= 1, "paged_attention: bad shape");
  LSH_CHECK(Hq % Hk == 0, "Hq must be a multiple of Hk");
  LSH_CHECK(block_size >= 1 && max_blocks >= 0 && num_slots >= 0, "paged_attention: bad cache shape");
  if (B == 0) return LLMSERVE_OK;
  LSH_CHECK(max_blocks >= 1 && num_slots >= block_size,
            "paged_attention: empty block table or cache");
  const int64_t G = Hq / Hk;
  LSH_CHECK(G <= 8, "paged_attention: at most 8 query heads per kv head (got %lld)", (long long)G);
  LSH_CHECK(D == 16 || D == 32 || D == 64 || D == 128 || D == 256,
            "paged_attention: head_dim %lld not in {16, 32, 64, 128, 256}", (long long)D);
  LSH_CHECK(B < (1LL << 24) && Hk <= 4096, "paged_attention: batch or kv heads too large");
  LSH_CHECK(max_blocks * block_size < (1LL << 31) && num_slots * Hk < (1LL << 31),
            "paged_attention: context or cache too long");
  const bool int8 = c.elem_bytes == 1;
  LSH_CHECK(c.elem_bytes == 1 || c.elem_bytes == 4, "paged_attention: cache of int8 or float32");
  LSH_CHECK(q && c.k && c.v && block_tables && context_lens && out &&
                (!int8 || (c.k_scale && c.v_scale)),
            "paged_attention: null pointer");
  LSH_CHECK(rows.row_table == nullptr || rows.table_rows >= 1,
            "paged_attention: a row map needs a non-empty block table");
  LSH_CHECK(lsh::aligned16(q) && lsh::aligned16(c.k) && lsh::aligned16(c.v) &&
                lsh::aligned16(out) && (q_mult == nullptr || lsh::aligned16(q_mult)),
            "paged_attention: q, caches, out and q_mult must be 16-byte aligned");
  const int64_t slots = partial_slots(B, Hk, D, G, max_blocks, block_size, partition_size);
  const int64_t units = B * (Hk / heads_per_block(Hk));
  const int64_t need = slots * G * (D + 2) * static_cast<int64_t>(sizeof(float)) + units * 4;
  LSH_CHECK(workspace != nullptr && workspace_bytes >= need,
            "paged_attention: workspace of %lld bytes needed, %lld given", (long long)need,
            (long long)workspace_bytes);
  LSH_CHECK(lsh::aligned16(workspace), "paged_attention: workspace must be 16-byte aligned");

  const bool scalar = scalar_blocks(D, block_size);
  DecodeArgs a{};
  a.q = q;
  a.kc = c.k;
  a.vc = c.v;
  a.ks = c.k_scale;
  a.vs = c.v_scale;
  a.bt = block_tables;
  a.row_tab = rows.row_table;
  a.tab_rows = rows.table_rows;
  a.cl = context_lens;
  a.q_mult = q_mult;
  a.out = out;
  float* ws = static_cast<float*>(workspace);
  a.part_ml = ws;
  a.part_acc = ws + slots * G * 2;
  a.unit_n = reinterpret_cast<int*>(ws + slots * G * (D + 2));
  a.kcap = static_cast<int>(unit_slots(B, D, G, Hk, max_blocks, block_size, partition_size));
  a.num_slots = num_slots;
  a.range = partition_size > 0 ? partition_size : 0;
  a.B = static_cast<int>(B);
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.max_blocks = static_cast<int>(max_blocks);
  a.bs = static_cast<int>(block_size);
  a.bs_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1LL << sh) == block_size) a.bs_shift = sh;
  a.HB = heads_per_block(Hk);
  a.NHG = static_cast<int>(Hk / a.HB);
  // one buffer resource per cache tensor when each is addressable with 32-bit offsets
  const bool off32 = num_slots * Hk * D * c.elem_bytes <= static_cast<int64_t>(0xffffffffu);
  a.W = grid_blocks(D, G, Hk, block_size, off32 ? 1 : 0, c.elem_bytes);
  a.qscale = scale * kLog2e;
  LSH_CHECK(a.W >= 1, "paged_attention: no resident workgroups");
  hipStream_t st = lsh::as_stream(stream);
  const bool ok = with_shape(D, G, [&]<int Dv, int Gv>() {
    if (int8)
      launch_decode<int8_t, Dv, Gv>(a, scalar, off32, fo, st);
    else
      launch_decode<float, Dv, Gv>(a, scalar, off32, fo, st);
  });
  LSH_CHECK(ok, "paged_attention: unsupported G=%lld", (long long)G);
  return lsh::launch_status(int8 ? "paged_attention_decode_int8" : "paged_attention_decode");
}

int decode_int8(const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
                const float* v_scale, const int64_t* block_tables, const int64_t* context_lens,
                float* out, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots,
                int64_t max_blocks, int64_t block_size, float scale, int64_t partition_size,
                const float* q_mult, const FragOut& fo, void* workspace, int64_t workspace_bytes,
                void* stream) {
  return decode_paged(q, CacheView{k_cache, v_cache, k_scale, v_scale, 1}, block_tables,
                      RowMap{nullptr, 0}, context_lens, out, B, Hq, Hk, D, num_slots, max_blocks,
                      block_size, scale, partition_size, q_mult, fo, workspace, workspace_bytes,
                      stream);
}

}  // namespace

extern "C" int llmserve_paged_attention_decode_int8(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, int64_t partition_size, const float* q_mult, void* workspace,
    int64_t workspace_bytes, void* stream) {
  return decode_int8(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, out, B, Hq,
                     Hk, D, num_slots, max_blocks, block_size, scale, partition_size, q_mult,
                     FragOut{nullptr, nullptr}, workspace, workspace_bytes, stream);
}

extern "C" int llmserve_paged_attention_decode_int8_xfrag(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    const float* act_inv, void* xfrag, int64_t B, int64_t Hq, int64_t Hk, int64_t D,
    int64_t num_slots, int64_t max_blocks, int64_t block_size, float scale,
    int64_t partition_size, const float* q_mult, void* workspace, int64_t workspace_bytes,
    void* stream) {
  LSH_CHECK(D == 128 || D == 256,
            "paged_attention_decode_int8_xfrag: head_dim %lld not 128 or 256", (long long)D);
  LSH_CHECK(B >= 0 && Hq >= 1 && B * Hq * D < (1LL << 31),
            "paged_attention_decode_int8_xfrag: bad or too large shape");
  LSH_CHECK(B == 0 || (xfrag != nullptr && lsh::aligned16(xfrag)),
            "paged_attention_decode_int8_xfrag: xfrag must be a 16-byte aligned buffer");
  return decode_int8(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, out, B, Hq,
                     Hk, D, num_slots, max_blocks, block_size, scale, partition_size, q_mult,
                     FragOut{act_inv, xfrag}, workspace, workspace_bytes, stream);
}

extern "C" int llmserve_paged_attention_decode(
    const float* q, const float* k_cache, const float* v_cache, const int64_t* block_tables,
    const int64_t* context_lens, float* out, int64_t B, int64_t Hq, int64_t Hk, int64_t D,
    int64_t num_slots, int64_t max_blocks, int64_t block_size, float scale,
    int64_t partition_size, void* workspace, int64_t workspace_bytes, void* stream) {
  return decode_paged(q, CacheView{k_cache, v_cache, nullptr, nullptr, 4}, block_tables,
                      RowMap{nullptr, 0}, context_lens, out, B, Hq, Hk, D, num_slots, max_blocks,
                      block_size, scale, partition_size, nullptr, FragOut{nullptr, nullptr},
                      workspace, workspace_bytes, stream);
}

extern "C" int llmserve_paged_attention_rows_int8(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, int64_t table_rows,
    const int64_t* row_table, const int64_t* row_context, float* out, int64_t R, int64_t Hq,
    int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks, int64_t block_size,
    float scale, const float* q_mult, void* workspace, int64_t workspace_bytes, void* stream) {
  LSH_CHECK(row_table != nullptr || R == 0, "paged_attention_rows_int8: row_table is required");
  return decode_paged(q, CacheView{k_cache, v_cache, k_scale, v_scale, 1}, block_tables,
                      RowMap{row_table, table_rows}, row_context, out, R, Hq, Hk, D, num_slots,
                      max_blocks, block_size, scale, 0, q_mult, FragOut{nullptr, nullptr},
                      workspace, workspace_bytes, stream);
}

extern "C" int llmserve_paged_attention_rows_f32(
    const float* q, const float* k_cache, const float* v_cache, const int64_t* block_tables,
    int64_t table_rows, const int64_t* row_table, const int64_t* row_context, float* out,
    int64_t R, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, const float* q_mult, void* workspace,
    int64_t workspace_bytes, void* stream) {
  LSH_CHECK(row_table != nullptr || R == 0, "paged_attention_rows_f32: row_table is required");
  return decode_paged(q, CacheView{k_cache, v_cache, nullptr, nullptr, 4}, block_tables,
                      RowMap{row_table, table_rows}, row_context, out, R, Hq, Hk, D, num_slots,
                      max_blocks, block_size, scale, 0, q_mult, FragOut{nullptr, nullptr},
                      workspace, workspace_bytes, stream);
}

// ---- allocation-free variant --------------------------------------------------------------
// Callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops) get the split-context partials from this file-scope array instead of a workspace:
// each GPU the library runs on holds its own copy until the process ends. Calls that overlap
// on one GPU share it and race; nothing in it needs clearing (the merge reads only partials
// the same call's decode kernel wrote).
constexpr int64_t kNoAllocScratchBytes = 32LL << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// The device address of `scratch` on the current device, looked up once per device (the
// array's name in host code is only a stand-in for the symbol).
void* noalloc_scratch() {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    lsh::set_error("paged_attention_decode_int8_noalloc: no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      lsh::set_error("paged_attention_decode_int8_noalloc: hipGetSymbolAddress failed (%s)",
                     hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

}  // namespace

extern "C" int64_t llmserve_paged_attention_noalloc_scratch_bytes(void) {
  return kNoAllocScratchBytes;
}

extern "C" int llmserve_paged_attention_decode_int8_noalloc(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, int64_t partition_size, const float* q_mult, void* stream) {
  const int64_t need = llmserve_paged_attention_workspace_bytes(B, Hq, Hk, D, max_blocks,
                                                                block_size, partition_size);
  LSH_CHECK(need <= kNoAllocScratchBytes,
            "paged_attention_decode_int8_noalloc: the call needs %lld bytes of partials, more "
            "than the library's %lld-byte scratch array (use the workspace entry point)",
            (long long)need, (long long)kNoAllocScratchBytes);
  if (B == 0) return LLMSERVE_OK;
  void* ws = noalloc_scratch();
  if (ws == nullptr) return LLMSERVE_ERR_HIP;
  return decode_int8(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, out, B, Hq,
                     Hk, D, num_slots, max_blocks, block_size, scale, partition_size, q_mult,
                     FragOut{nullptr, nullptr}, ws, kNoAllocScratchBytes, stream);
}
