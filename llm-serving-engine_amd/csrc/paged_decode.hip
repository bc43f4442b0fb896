// int8-KV paged decode attention (split context + online softmax) and the partition merge.
//
// Work item = one wavefront per (sequence b, kv head h, context partition p); a 256-thread
// workgroup holds the wavefronts of 4 consecutive kv heads of the same (b, p), so one
// workgroup streams 4 x 128 B of every cache slot it touches.
//
// Lane layout inside a wavefront (D = head dim, LPR = D / 16 lanes per token row):
//   lane = r * LPR + seg : row slot r of the RPW = 64 / LPR tokens of one step, dims
//                          [16 seg, 16 seg + 16) of that token.
// Each lane loads 16 bytes of the token's K row and 16 bytes of its V row per step (one
// dwordx4 each, non-temporal: the wave reads RPW whole rows). Every row slot runs its own
// online softmax over the tokens it sees (t = r, r + RPW, ...), so a step needs no
// cross-row communication:
//   * q.k: 16-dim partial dot per query head, summed over the LPR lanes of the row with DPP;
//   * the running max is raised only when a score exceeds it by more than kLazy (the
//     exponentials stay <= e^kLazy); the rescale of (sum, acc) then runs under a
//     wave-uniform branch, so most steps skip it;
//   * acc += (p * v_scale) * v_int8 in the lane's 16 dims.
// Up to four steps of K/V loads are kept in flight (a ring of registers, refilled as each
// step is consumed), and the partition's block ids (<= 64 blocks) sit one per lane, read with a
// lane shuffle. At the end the RPW row-slot states are merged (DPP / permlane swaps), then
// written as the output (one partition) or as a partial for the merge kernel.
// Scores follow the reference's order of operations: s = (scale * k_scale) * (q . k_int8),
// acc += (p * v_scale) * v_int8 (paged_attention.cpp:301-355).
#include "common.h"

namespace {

using lsh::kWave;
constexpr int kWavesPerBlock = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;  // the reference's initial running max
constexpr float kLazy = 8.0f;       // headroom of the lazy running max (natural-log units)
constexpr int kMaxPartBlocks = 64;  // block ids of one partition held one per lane
// steps of K/V loads in flight per wavefront (fewer for wide GQA groups: register budget)
template <int G>
constexpr int ring_depth() { return G <= 2 ? 4 : (G <= 4 ? 3 : 2); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void unpack_i8x16(const u32x4& w, float (&f)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      f[4 * i + b] = static_cast<float>(static_cast<int8_t>((w[i] >> (8 * b)) & 0xffu));
}

struct DecodeArgs {
  const float* q;
  const int8_t* kc;
  const int8_t* vc;
  const float* ks;
  const float* vs;
  const int64_t* bt;
  const int64_t* cl;
  const float* q_mult;
  float* out;
  float* part_ml;   // [B, Hk, NP, G, 2]  (max, sum)
  float* part_acc;  // [B, Hk, NP, G, D]
  int64_t num_slots;
  int B, Hq, Hk, max_blocks, bs, bs_shift, P, NP;  // bs_shift = log2(bs), or -1
  float scale;
};

// One token step of one lane: its 16 K and V bytes and the row's two scales.
struct Tok {
  u32x4 k, v;
  float ks, vs;
  bool valid;
};

// One work item: sequence b, kv head h, context partition p, on one wavefront.
template <int D, int G>
__device__ __forceinline__ void decode_item(const DecodeArgs& a, int b, int h, int p) {
  constexpr int LPR = D / 16;       // lanes per token row
  constexpr int RPW = kWave / LPR;  // row slots per wavefront
  constexpr int kRing = ring_depth<G>();
  const int lane = threadIdx.x % kWave;
  const int r = lane / LPR, seg = lane % LPR;

  int64_t ctx = a.cl[b];
  const int64_t cap = static_cast<int64_t>(a.max_blocks) * a.bs;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int t0 = p * a.P;
  const int t1 = static_cast<int>(ctx < t0 + a.P ? ctx : t0 + a.P);
  const int64_t pidx = (static_cast<int64_t>(b) * a.Hk + h) * a.NP + p;

  if (t0 >= t1) {  // partition past this sequence's end (or an empty context)
    if (a.NP > 1) {
      if (lane < G) {
        a.part_ml[(pidx * G + lane) * 2] = kNegBig;
        a.part_ml[(pidx * G + lane) * 2 + 1] = 0.f;
      }
    } else if (r == 0) {  // ctx == 0: the reference yields 0 * (1 / 0)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a.out[(static_cast<int64_t>(b) * a.Hq + h * G + g) * D + seg * 16 + i] = __builtin_nanf("");
    }
    return;
  }

  // block ids of this partition, one per lane (-1: outside the cache)
  const int blk0 = t0 / a.bs;  // t0 is a block multiple
  const int nblk = (t1 - t0 + a.bs - 1) / a.bs;
  int my_blk = -1;
  if (lane < nblk) {
    const int64_t id = a.bt[static_cast<int64_t>(b) * a.max_blocks + blk0 + lane];
    my_blk = (id >= 0 && id < a.num_slots / a.bs) ? static_cast<int>(id) : -1;
  }

  const int64_t row_stride = static_cast<int64_t>(a.Hk) * D;  // bytes between slots
  const int64_t head_off = static_cast<int64_t>(h) * D + seg * 16;
  // Issues the loads of token t into o. A lane without a token (t >= t1 or a block id
  // outside the cache) reads slot 0 instead — the same 16 bytes for every such lane, one
  // cached line — and o.valid masks it. The loads are unconditional on purpose: with a
  // predicated load the compiler folds the consumer's byte unpacking into the load's block
  // and waits for the data right there, which serialises the ring of in-flight steps.
  auto fetch = [&](int t, Tok& o) {
    // every lane takes part in the shuffle (a lane's block id is read even when that lane
    // has no token of its own in this step)
    const int rel = t < t1 ? t - t0 : 0;
    int id = __shfl(my_blk, a.bs_shift >= 0 ? rel >> a.bs_shift : rel / a.bs, kWave);
    if (t >= t1) id = -1;
    o.valid = id >= 0;
    const int off = a.bs_shift >= 0 ? t & (a.bs - 1) : t % a.bs;
    const int64_t slot = o.valid ? static_cast<int64_t>(id) * a.bs + off : 0;
    o.k = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.kc + slot * row_stride + head_off));
    o.v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.vc + slot * row_stride + head_off));
    o.ks = a.ks[slot * a.Hk + h];
    o.vs = a.vs[slot * a.Hk + h];
  };

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
      qv[g][4 * i] = v.x;
      qv[g][4 * i + 1] = v.y;
      qv[g][4 * i + 2] = v.z;
      qv[g][4 * i + 3] = v.w;
    }
  }

  // q and the block ids are in registers before any K/V load is issued: otherwise the
  // loop header, which merges this entry path with its back edge, would wait for all
  // outstanding loads (vmcnt counts in issue order) on every iteration.
  __builtin_amdgcn_s_waitcnt(0);

  Tok ring[kRing];
#pragma unroll
  for (int u = 0; u < kRing; ++u) fetch(t0 + u * RPW + r, ring[u]);

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }

  // Whole rounds of kRing steps; steps past t1 are fully masked (no loads, p = 0).
  for (int tb = t0; tb < t1; tb += kRing * RPW) {
#pragma unroll
    for (int u = 0; u < kRing; ++u) {
      const int tcur = tb + u * RPW;
      Tok& c = ring[u];
      // Consume the ring entry here and not earlier: an opaque use stops the compiler from
      // folding the unpacking into the loop latch, where it would wait for loads issued
      // only this round (vmcnt counts in issue order).
      asm volatile("" : "+v"(c.k), "+v"(c.v), "+v"(c.ks), "+v"(c.vs));
      float kf[16];
      unpack_i8x16(c.k, kf);
      float s[G];
      bool raise = false;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d += qv[g][i] * kf[i];
        d = lsh::group_sum<LPR>(d);
        s[g] = c.valid ? (a.scale * c.ks) * d : kNegBig;
        raise |= s[g] > m[g] + kLazy;
      }
      if (__builtin_amdgcn_ballot_w64(raise)) {  // rare: the running max moves
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const bool up = s[g] > m[g] + kLazy;
          const float alpha = up ? __builtin_amdgcn_exp2f((m[g] - s[g]) * kLog2e) : 1.f;
          m[g] = up ? s[g] : m[g];
          l[g] *= alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[g][i] *= alpha;
        }
      }
      float vf[16];
      unpack_i8x16(c.v, vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = c.valid ? __builtin_amdgcn_exp2f((s[g] - m[g]) * kLog2e) : 0.f;
        l[g] += pr;
        const float pv = c.valid ? pr * c.vs : 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[g][i] += pv * vf[i];
      }
      fetch(tcur + kRing * RPW + r, c);
    }
  }

  // merge the RPW row-slot states (lanes with equal seg)
  float lt[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mx = lsh::wave_max_from<LPR>(m[g]);
    const float w = __builtin_amdgcn_exp2f((m[g] - mx) * kLog2e);
    m[g] = mx;
    lt[g] = lsh::wave_sum_from<LPR>(w * l[g]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = lsh::wave_sum_from<LPR>(w * acc[g][i]);
  }
  if (a.NP == 1) {
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
      float4* o = reinterpret_cast<float4*>(a.part_acc + (pidx * G + g) * D + seg * 16);
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
    a.part_ml[(pidx * G + lane) * 2] = mm;
    a.part_ml[(pidx * G + lane) * 2 + 1] = ll;
  }
}

// Persistent decode kernel: a grid sized to the GPU (resident workgroups) strides over the
// work items (b, group of 4 kv heads, p), p fastest. Each wavefront of a workgroup takes one
// head of the group. Items past a sequence's end are cheap, so the strided assignment keeps
// the waves evenly loaded without a second round of workgroups.
template <int D, int G>
__global__ __launch_bounds__(256) void paged_decode_int8_kernel(DecodeArgs a) {
  const int wave = threadIdx.x / kWave;
  const int hgroups = (a.Hk + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t items = static_cast<int64_t>(a.B) * hgroups * a.NP;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int p = static_cast<int>(it % a.NP);
    const int64_t bh = it / a.NP;
    const int h = static_cast<int>(bh % hgroups) * kWavesPerBlock + wave;
    const int b = static_cast<int>(bh / hgroups);
    if (h < a.Hk) decode_item<D, G>(a, b, h, p);  // no barriers: waves proceed independently
  }
}

// Merge of the partitions (paged_attention.cpp:432-455): one wavefront per (b, q head).
//   M = max_p m_p;  w_p = exp(m_p - M);  out = sum_p w_p acc_p / sum_p w_p l_p  (l_p = 0 skipped)
// Lanes first read the (m, l) of 64 partitions at a time; the weighted sum over the
// partitions' acc rows then runs with all loads of a 64-partition batch independent.
template <int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a, int B) {
  constexpr int PER = (D + kWave - 1) / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= static_cast<int64_t>(B) * a.Hq) return;
  const int b = static_cast<int>(item / a.Hq), hq = static_cast<int>(item % a.Hq);
  const int G = a.Hq / a.Hk;
  const int h = hq / G, g = hq % G;
  const int64_t base = (static_cast<int64_t>(b) * a.Hk + h) * a.NP;
  float M = kNegBig;
  for (int p = lane; p < a.NP; p += kWave) M = fmaxf(M, a.part_ml[((base + p) * G + g) * 2]);
  M = lsh::wave_max_from<1>(M);
  float L = 0.f, o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  for (int p0 = 0; p0 < a.NP; p0 += kWave) {
    const int pl = p0 + lane;
    float w = 0.f;
    if (pl < a.NP) {
      const int64_t pi = (base + pl) * G + g;
      const float lp = a.part_ml[pi * 2 + 1];
      w = lp == 0.f ? 0.f : __builtin_amdgcn_exp2f((a.part_ml[pi * 2] - M) * kLog2e);
      L += w * lp;
    }
    const int n = a.NP - p0 < kWave ? a.NP - p0 : kWave;
#pragma unroll 8
    for (int j = 0; j < n; ++j) {
      const float wj = __shfl(w, j, kWave);
      if (wj == 0.f) continue;  // wave-uniform
      const float* src = a.part_acc + ((base + p0 + j) * G + g) * D;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int d = lane + i * kWave;
        if (d < D) o[i] += wj * src[d];
      }
    }
  }
  L = lsh::wave_sum_from<1>(L);
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + i * kWave;
    if (d < D) a.out[item * D + d] = o[i] * inv;
  }
}

// Partition size: a block multiple of at most kMaxPartBlocks blocks. Auto: ~8k wavefronts
// over the context bound (max_blocks * block_size), at least 128 tokens each.
int64_t round_partition(int64_t P, int64_t B, int64_t Hk, int64_t max_blocks, int64_t bs) {
  const int64_t max_ctx = max_blocks * bs;
  if (P <= 0) {
    const int64_t parts = (8192 + B * Hk - 1) / (B * Hk);
    P = (max_ctx + parts - 1) / parts;
    if (P < 128) P = 128;
  }
  P = ((P + bs - 1) / bs) * bs;
  if (P > kMaxPartBlocks * bs) P = kMaxPartBlocks * bs;
  if (P > max_ctx && max_ctx > 0) P = ((max_ctx + bs - 1) / bs) * bs;
  return P < bs ? bs : P;
}

// Resident workgroups of a kernel on the current device: CUs x blocks per CU (cached).
template <typename K>
int resident_blocks(K kernel) {
  static int cached[64][2] = {};  // [device] = {cus, blocks per CU}
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev][0] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kWavesPerBlock * kWave, 0) !=
            hipSuccess || per < 1)
      per = 1;
    cached[dev][1] = per;
    cached[dev][0] = cus;
  }
  return cached[dev][0] * cached[dev][1];
}

template <int D, int G>
void launch_decode(const DecodeArgs& a, int B, hipStream_t st) {
  const int64_t items = static_cast<int64_t>(B) * ((a.Hk + kWavesPerBlock - 1) / kWavesPerBlock) * a.NP;
  const int64_t resident = resident_blocks(paged_decode_int8_kernel<D, G>);
  const unsigned grid = static_cast<unsigned>(items < resident ? items : resident);
  lsh::launch(paged_decode_int8_kernel<D, G>, dim3(grid), dim3(kWavesPerBlock * kWave), 0, st,
              a.NP == 1, a);
  if (a.NP > 1) {
    const int64_t items = static_cast<int64_t>(B) * a.Hq;
    lsh::launch(paged_decode_merge_kernel<D>,
                dim3(static_cast<unsigned>((items + kWavesPerBlock - 1) / kWavesPerBlock)),
                dim3(kWavesPerBlock * kWave), 0, st, true, a, B);
  }
}

template <int D>
bool dispatch_g(int G, const DecodeArgs& a, int B, hipStream_t st) {
  switch (G) {
    case 1: launch_decode<D, 1>(a, B, st); return true;
    case 2: launch_decode<D, 2>(a, B, st); return true;
    case 3: launch_decode<D, 3>(a, B, st); return true;
    case 4: launch_decode<D, 4>(a, B, st); return true;
    case 5: launch_decode<D, 5>(a, B, st); return true;
    case 6: launch_decode<D, 6>(a, B, st); return true;
    case 7: launch_decode<D, 7>(a, B, st); return true;
    case 8: launch_decode<D, 8>(a, B, st); return true;
    default: return false;
  }
}

}  // namespace

extern "C" int64_t llmserve_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hk,
                                                            int64_t D, int64_t max_blocks,
                                                            int64_t block_size,
                                                            int64_t partition_size) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || D <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  const int64_t P = round_partition(partition_size, B, Hk, max_blocks, block_size);
  const int64_t NP = (max_blocks * block_size + P - 1) / P;
  if (NP <= 1) return 0;
  return B * Hq * NP * (D + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int llmserve_paged_attention_decode_int8(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, int64_t partition_size, const float* q_mult, void* workspace,
    int64_t workspace_bytes, void* stream) {
  LSH_CHECK(B >= 0 && Hq >= 1 && Hk >= 1 && D >= 1, "paged_attention: bad shape");
  LSH_CHECK(Hq % Hk == 0, "Hq must be a multiple of Hk");
  LSH_CHECK(block_size >= 1 && max_blocks >= 0 && num_slots >= 0, "paged_attention: bad cache shape");
  if (B == 0) return LLMSERVE_OK;
  LSH_CHECK(max_blocks >= 1 && num_slots >= block_size,
            "paged_attention: empty block table or cache");
  const int64_t G = Hq / Hk;
  LSH_CHECK(G <= 8, "paged_attention_decode_int8: at most 8 query heads per kv head (got %lld)",
            (long long)G);
  LSH_CHECK(D == 16 || D == 32 || D == 64 || D == 128 || D == 256,
            "paged_attention_decode_int8: head_dim %lld not in {16, 32, 64, 128, 256}", (long long)D);
  LSH_CHECK(B <= 65535 && Hk <= 65535 * kWavesPerBlock, "paged_attention: grid too large");
  LSH_CHECK(max_blocks * block_size < (1LL << 31) && num_slots / block_size < (1LL << 31),
            "paged_attention: context or cache too long");
  LSH_CHECK(q && k_cache && v_cache && k_scale && v_scale && block_tables && context_lens && out,
            "paged_attention: null pointer");
  LSH_CHECK(lsh::aligned16(q) && lsh::aligned16(k_cache) && lsh::aligned16(v_cache) &&
                lsh::aligned16(out) && (q_mult == nullptr || lsh::aligned16(q_mult)),
            "paged_attention: q, caches, out and q_mult must be 16-byte aligned");
  const int64_t P = round_partition(partition_size, B, Hk, max_blocks, block_size);
  const int64_t NP = (max_blocks * block_size + P - 1) / P;
  const int64_t need =
      llmserve_paged_attention_workspace_bytes(B, Hq, Hk, D, max_blocks, block_size, partition_size);
  LSH_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr),
            "paged_attention: workspace of %lld bytes needed, %lld given", (long long)need,
            (long long)workspace_bytes);
  LSH_CHECK(need == 0 || lsh::aligned16(workspace), "paged_attention: workspace must be 16-byte aligned");
  LSH_CHECK(NP < (1LL << 31), "paged_attention: too many partitions");

  DecodeArgs a{};
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.ks = k_scale;
  a.vs = v_scale;
  a.bt = block_tables;
  a.cl = context_lens;
  a.q_mult = q_mult;
  a.out = out;
  float* ws = static_cast<float*>(workspace);
  a.part_ml = NP > 1 ? ws : nullptr;
  a.part_acc = NP > 1 ? ws + B * Hq * NP * 2 : nullptr;
  a.num_slots = num_slots;
  a.B = static_cast<int>(B);
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.max_blocks = static_cast<int>(max_blocks);
  a.bs = static_cast<int>(block_size);
  a.bs_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1LL << sh) == block_size) a.bs_shift = sh;
  a.P = static_cast<int>(P);
  a.NP = static_cast<int>(NP);
  a.scale = scale;
  hipStream_t st = lsh::as_stream(stream);
  const int Bi = static_cast<int>(B), Gi = static_cast<int>(G);
  bool ok = false;
  switch (D) {
    case 16: ok = dispatch_g<16>(Gi, a, Bi, st); break;
    case 32: ok = dispatch_g<32>(Gi, a, Bi, st); break;
    case 64: ok = dispatch_g<64>(Gi, a, Bi, st); break;
    case 128: ok = dispatch_g<128>(Gi, a, Bi, st); break;
    default: ok = dispatch_g<256>(Gi, a, Bi, st); break;
  }
  LSH_CHECK(ok, "paged_attention: unsupported G=%lld", (long long)G);
  return lsh::launch_status("paged_attention_decode_int8");
}
