// Split-context paged attention over an int8 or fp32 KV cache: the per-wavefront core shared
// by the decode / row kernels (paged_decode.hip) and the decode chain (decode_chain.hip). A
// wavefront runs the tokens [t0, t1) of one (query row, kv head) as an online softmax for the
// head's G query heads (the reference's decode_partition, paged_attention.cpp:191-346, with the
// float operations in this build's order; the scheme is described in paged_decode.hip).
#pragma once

#include <type_traits>

#include "common.h"

namespace {

using lsh::kWave;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;        // the reference's initial running max
constexpr float kLazy2 = 8.0f * kLog2e;  // lazy running-max headroom (log2 units: e^8)
constexpr int kWin = 64;                 // block ids of a window, one per lane
// steps of K/V loads in flight per wavefront (fewer for wide GQA groups and fp32 rows, which
// hold four times the bytes per lane: register budget)
template <int G, bool kF32>
constexpr int ring_depth() {
  if constexpr (kF32) return G <= 2 ? 2 : 1;
  return G <= 2 ? 4 : (G <= 4 ? 3 : 2);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kNT = 2;  // buffer-load cache policy: non-temporal (streamed once)

// Raw buffer resource over `bytes` bytes at p (loads past the end return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes),
                                           0x00020000);
}

// 16 int8 values, one sign-extending byte-select conversion each (left to itself the compiler
// takes the odd bytes of the V words through a 16-bit shift first: 8 more instructions per
// step).
__device__ __forceinline__ void unpack16(const u32x4& w, float (&f)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = w[i];
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(f[4 * i]) : "v"(u));
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(f[4 * i + 1]) : "v"(u));
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(f[4 * i + 2]) : "v"(u));
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(f[4 * i + 3]) : "v"(u));
  }
}

// 16 floats. The element goes through a named temporary: this compiler's __builtin_bit_cast of
// a vector element expression (w[i][b]) reads element 0 whatever the subscript.
__device__ __forceinline__ void unpack16(const u32x4 (&w)[4], float (&f)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t u = w[i][b];
      f[4 * i + b] = __builtin_bit_cast(float, u);
    }
}

struct DecodeArgs {
  const float* q;
  const void* kc;  // int8 or float32 [num_slots, Hk, D]
  const void* vc;
  const float* ks;  // [num_slots, Hk] (int8 caches only)
  const float* vs;
  const int64_t* bt;
  const int64_t* row_tab;  // nullable [B]: block-table row of query row b (else b)
  int64_t tab_rows;        // rows of bt when row_tab is given
  const int64_t* cl;
  const float* q_mult;
  float* out;
  float* part_ml;   // [slots, G, 2]  (running max in log2 units, sum)
  float* part_acc;  // [slots, G, D]
  int* unit_n;      // [B * NHG]: ranges of each (row, head group) unit, set by its first range
  int kcap;         // partial slots per unit (bound on its ranges)
  int64_t num_slots;
  int64_t range;  // tokens per work range; 0: the balanced plan (paged_decode.hip)
  int B, Hq, Hk, max_blocks, bs, bs_shift;  // bs_shift = log2(bs), or -1
  int HB, NHG;  // kv heads per workgroup, head groups (Hk = HB * NHG)
  int W;        // decode workgroups (all resident)
  float qscale;                                 // scale * log2(e)
};

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Context length of query row b, clamped to [0, max_blocks * block_size]; 0 for a row whose
// block-table row (row map) is outside the table.
__device__ __forceinline__ int64_t seq_ctx(const DecodeArgs& a, int b) {
  const int64_t cap = static_cast<int64_t>(a.max_blocks) * a.bs;
  const int64_t c = a.cl[b];
  if (a.row_tab != nullptr) {
    const int64_t t = a.row_tab[b];
    if (t < 0 || t >= a.tab_rows) return 0;
  }
  return c < 0 ? 0 : (c > cap ? cap : c);
}

// One token step of one lane: its 16 K and V elements and the row's two scales (1 for an
// fp32 cache).
template <typename E>
struct Tok;
template <>
struct Tok<int8_t> {
  u32x4 k, v;
  float ks, vs;
  bool valid;  // this lane's token is in the segment and its block id is inside the cache
};
template <>
struct Tok<float> {
  u32x4 k[4], v[4];
  float ks, vs;
  bool valid;
};

// An opaque use of a ring entry's registers (see the ring loop).
__device__ __forceinline__ void pin(Tok<int8_t>& c) {
  asm volatile("" : "+v"(c.k), "+v"(c.v), "+v"(c.ks), "+v"(c.vs));
}
__device__ __forceinline__ void pin(Tok<float>& c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(c.k[i]), "+v"(c.v[i]));
}

// The online-softmax state of tokens [t0, t1) of (query row b, kv head h) for its G query
// heads, merged over the wavefront's row slots: running max (log2 units), sum and the 16
// accumulator dims of this lane's segment (lanes with r = lane / (D / 16) == 0 hold the row).
template <int G>
struct SegState {
  float m[G], lt[G], acc[G][16];
};

// Runs tokens [t0, t1) of (b, h) into `st`.
// kOff32: the K / V caches and their scales are each under 4 GB, so one buffer resource per
// tensor (built once) with the step's slot offset in the scalar offset register addresses a
// step; else the resources are rebuilt per step from 64-bit bases.
template <typename E, int D, int G, bool kScalarBlk, bool kOff32>
__device__ __forceinline__ void segment_state(const DecodeArgs& a, int b, int h, int t0, int t1,
                                              SegState<G>& st) {
  constexpr bool kF32 = std::is_same_v<E, float>;
  constexpr int kEB = sizeof(E);    // bytes per cache element
  constexpr int LPR = D / 16;       // lanes per token row
  constexpr int RPW = kWave / LPR;  // row slots per wavefront
  constexpr int kRing = ring_depth<G, kF32>();
  const int64_t tab_row = a.row_tab ? uniform64(a.row_tab[b]) : b;
  const int lane = threadIdx.x % kWave;
  const int r = lane / LPR, seg = lane % LPR;
  const int bs = a.bs;

  float qv[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t qo = (static_cast<int64_t>(b) * a.Hq + h * G + g) * D + seg * 16;
    const float4* qp = reinterpret_cast<const float4*>(a.q + qo);
    const float4* mp =
        a.q_mult ? reinterpret_cast<const float4*>(a.q_mult + (h * G + g) * D + seg * 16) : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 v = qp[i];
      if (mp) {
        const float4 s = mp[i];
        v.x = __fmul_rn(v.x, s.x);
        v.y = __fmul_rn(v.y, s.y);
        v.z = __fmul_rn(v.z, s.z);
        v.w = __fmul_rn(v.w, s.w);
      }
      qv[g][4 * i] = v.x * a.qscale;
      qv[g][4 * i + 1] = v.y * a.qscale;
      qv[g][4 * i + 2] = v.z * a.qscale;
      qv[g][4 * i + 3] = v.w * a.qscale;
    }
  }

  float m[G], mt[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    mt[g] = kNegBig;  // m + kLazy2 (kNegBig absorbs the headroom)
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }

  const int64_t row_stride = static_cast<int64_t>(a.Hk) * D * kEB;  // bytes between slots
  // Per-lane offsets inside a step: row slot r, head h, dims of segment seg.
  const uint32_t kv_lane = static_cast<uint32_t>(r * row_stride + (h * D + seg * 16) * kEB);
  const uint32_t sc_lane = static_cast<uint32_t>((r * a.Hk + h) * sizeof(float));
  const int64_t head_off = (static_cast<int64_t>(h) * D + seg * 16) * kEB;
  const char* kc = static_cast<const char*>(a.kc);
  const char* vc = static_cast<const char*>(a.vc);
  const uint32_t step_bytes = static_cast<uint32_t>(RPW * row_stride);
  const uint32_t sc_bytes = static_cast<uint32_t>(RPW * a.Hk * sizeof(float));
  // kOff32 resources over whole tensors (the byte counts fit 32 bits by the host's choice)
  const uint32_t rs32 = static_cast<uint32_t>(row_stride), hk4 = static_cast<uint32_t>(a.Hk * 4);
  const __amdgpu_buffer_rsrc_t rk = rsrc(a.kc, static_cast<uint32_t>(a.num_slots * row_stride));
  const __amdgpu_buffer_rsrc_t rv = rsrc(a.vc, static_cast<uint32_t>(a.num_slots * row_stride));
  const __amdgpu_buffer_rsrc_t rks = rsrc(a.ks, static_cast<uint32_t>(a.num_slots * a.Hk * 4));
  const __amdgpu_buffer_rsrc_t rvs = rsrc(a.vs, static_cast<uint32_t>(a.num_slots * a.Hk * 4));

  for (int wb = t0 / bs; static_cast<int64_t>(wb) * bs < t1; wb += kWin) {
    const int ws = t0 > wb * bs ? t0 : wb * bs;
    const int we =
        static_cast<int64_t>(t1) < static_cast<int64_t>(wb + kWin) * bs ? t1 : (wb + kWin) * bs;
    int my_blk = -1;  // block id of window block `lane` (-1: outside the cache)
    {
      const int nwin = (we - wb * bs + bs - 1) / bs;
      if (lane < nwin) {
        const int64_t id = a.bt[tab_row * a.max_blocks + wb + lane];
        my_blk = (id >= 0 && id < a.num_slots / bs) ? static_cast<int>(id) : -1;
      }
    }
    // q and the block ids are in registers before any K/V load is issued: otherwise the
    // loop header, which merges this entry path with its back edge, would wait for all
    // outstanding loads (vmcnt counts in issue order) on every iteration.
    __builtin_amdgcn_s_waitcnt(0);

    // Issues the loads of step k into o. Steps past the window read slot rows of block 0
    // (in bounds, masked). The loads are unconditional on purpose: with a predicated load
    // the compiler folds the consumer's byte unpacking into the load's block and waits for
    // the data right there, which serialises the ring of in-flight steps.
    auto fetch = [&](int k, Tok<E>& o) {
      const int tk = k * RPW;
      const int t = tk + r;
      if constexpr (kScalarBlk) {
        // the step's rows are slots sb .. sb + RPW - 1 of one block: buffer loads from a
        // scalar base, each lane at its own 32-bit offset
        const int bi = (tk >> a.bs_shift) - wb;  // wave-uniform
        const int id = bi < kWin ? __builtin_amdgcn_readlane(my_blk, bi) : -1;
        o.valid = id >= 0 && t >= ws && t < we;
        if constexpr (kOff32) {
          const uint32_t sb = static_cast<uint32_t>(id >= 0 ? id : 0) * bs + (tk & (bs - 1));
          if constexpr (kF32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              o.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rk, kv_lane + 16 * i, sb * rs32, kNT));
              o.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rv, kv_lane + 16 * i, sb * rs32, kNT));
            }
            o.ks = o.vs = 1.f;
          } else {
            o.k = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, kv_lane, sb * rs32, kNT));
            o.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, kv_lane, sb * rs32, kNT));
            o.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, sc_lane, sb * hk4, 0));
            o.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, sc_lane, sb * hk4, 0));
          }
        } else {
          const int64_t sb = static_cast<int64_t>(id >= 0 ? id : 0) * bs + (tk & (bs - 1));
          const __amdgpu_buffer_rsrc_t sk = rsrc(kc + sb * row_stride, step_bytes);
          const __amdgpu_buffer_rsrc_t sv = rsrc(vc + sb * row_stride, step_bytes);
          if constexpr (kF32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              o.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sk, kv_lane + 16 * i, 0, kNT));
              o.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sv, kv_lane + 16 * i, 0, kNT));
            }
            o.ks = o.vs = 1.f;
          } else {
            o.k = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sk, kv_lane, 0, kNT));
            o.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sv, kv_lane, 0, kNT));
            o.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 rsrc(a.ks + sb * a.Hk, sc_bytes), sc_lane, 0, 0));
            o.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 rsrc(a.vs + sb * a.Hk, sc_bytes), sc_lane, 0, 0));
          }
        }
      } else {
        // every lane takes part in the shuffle (a lane's block id is read even when that
        // lane has no token of its own in this step)
        const int tt = t < we ? t : ws;
        const int bi = (a.bs_shift >= 0 ? tt >> a.bs_shift : tt / bs) - wb;
        const int id = __shfl(my_blk, bi, kWave);
        o.valid = id >= 0 && t >= ws && t < we;
        const int off = a.bs_shift >= 0 ? t & (bs - 1) : t % bs;
        const int64_t sl = o.valid ? static_cast<int64_t>(id) * bs + off : 0;
        const u32x4* kp = reinterpret_cast<const u32x4*>(kc + sl * row_stride + head_off);
        const u32x4* vp = reinterpret_cast<const u32x4*>(vc + sl * row_stride + head_off);
        if constexpr (kF32) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            o.k[i] = __builtin_nontemporal_load(kp + i);
            o.v[i] = __builtin_nontemporal_load(vp + i);
          }
          o.ks = o.vs = 1.f;
        } else {
          o.k = __builtin_nontemporal_load(kp);
          o.v = __builtin_nontemporal_load(vp);
          o.ks = a.ks[sl * a.Hk + h];
          o.vs = a.vs[sl * a.Hk + h];
        }
      }
    };

    // One step. A row outside the segment or the cache gets the score -inf (p = 0, and it
    // never raises the max) and the value scale 0 (its bytes, whatever they hold, add 0).
    auto consume = [&](const Tok<E>& c) {
      float kf[16];
      unpack16(c.k, kf);
      float s[G];
      bool raise = false;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d += qv[g][i] * kf[i];
        d = lsh::group_sum<LPR>(d);
        s[g] = c.valid ? c.ks * d : -__builtin_inff();
        raise |= s[g] > mt[g];
      }
      if (__builtin_amdgcn_ballot_w64(raise)) {  // rare: the running max moves
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const bool up = s[g] > mt[g];
          const float alpha = up ? __builtin_amdgcn_exp2f(m[g] - s[g]) : 1.f;
          m[g] = up ? s[g] : m[g];
          mt[g] = m[g] + kLazy2;
          l[g] *= alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[g][i] *= alpha;
        }
      }
      float vf[16];
      unpack16(c.v, vf);
      const float vsc = c.valid ? c.vs : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = __builtin_amdgcn_exp2f(s[g] - m[g]);
        l[g] += pr;
        const float pv = pr * vsc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[g][i] += pv * vf[i];
      }
    };

    const int k0 = ws / RPW, k1 = (we + RPW - 1) / RPW;
    Tok<E> ring[kRing];
#pragma unroll
    for (int u = 0; u < kRing; ++u) fetch(k0 + u, ring[u]);
    // Whole rounds of kRing steps; steps past the window are fully masked.
    for (int k = k0; k < k1; k += kRing) {
#pragma unroll
      for (int u = 0; u < kRing; ++u) {
        Tok<E>& c = ring[u];
        // Consume the ring entry here and not earlier: an opaque use stops the compiler from
        // folding the unpacking into the loop latch, where it would wait for loads issued
        // only this round (vmcnt counts in issue order).
        pin(c);
        consume(c);
        fetch(k + u + kRing, c);
      }
    }
  }

  // merge the RPW row-slot states (lanes with equal seg)
  float lt[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mx = lsh::wave_max_from<LPR>(m[g]);
    const float w = __builtin_amdgcn_exp2f(m[g] - mx);
    m[g] = mx;
    lt[g] = lsh::wave_sum_from<LPR>(w * l[g]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = lsh::wave_sum_from<LPR>(w * acc[g][i]);
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    st.m[g] = m[g];
    st.lt[g] = lt[g];
#pragma unroll
    for (int i = 0; i < 16; ++i) st.acc[g][i] = acc[g][i];
  }
}

}  // namespace
