// int8-KV paged decode attention (split context + online softmax) and the partition merge.
//
// Work item = one wavefront per (sequence b, kv head h, context partition p); a 256-thread
// workgroup holds the wavefronts of 4 consecutive kv heads of the same (b, p), so one
// workgroup streams 4 x 128 B of every cache slot it touches.
//
// Lane layout inside a wavefront (D = head dim, LPR = D / 16 lanes per token row):
//   lane = r * LPR + seg : token row r of the current group of RPW = 64 / LPR tokens,
//                          dims [16 seg, 16 seg + 16) of that token.
// Each lane loads 16 bytes of the token's K row and 16 bytes of its V row (one dwordx4
// each; the wave reads RPW whole 2*D-byte rows per step), dequantizes them in registers,
// and
//   * q.k: 16-dim partial dot for each of the G query heads, summed over the LPR lanes of
//     the row with xor-shuffles (every lane of the row ends with the full score);
//   * online softmax: the step's max over the RPW rows (shuffles over the row bits), the
//     running max is wave-uniform, exp via exp2 (v_exp_f32);
//   * p.v: each lane accumulates p * v_scale * v into its 16 dims; partial sums over the
//     rows are folded together once at the end of the partition.
// Scores follow the reference's order of operations: s = (scale * k_scale) * (q . k_int8),
// acc += (p * v_scale) * v_int8 (paged_attention.cpp:301-355).
#include "common.h"

namespace {

using lsh::kWave;
constexpr int kWavesPerBlock = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;  // the reference's initial running max

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
  float* part_ml;   // [B, Hk, NP, G, 2]  (running max, sum)
  float* part_acc;  // [B, Hk, NP, G, D]
  int64_t num_slots;
  int Hq, Hk, max_blocks, bs, P, NP;
  float scale;
};

template <int D, int G>
__global__ __launch_bounds__(256) void paged_decode_int8_kernel(DecodeArgs a) {
  constexpr int LPR = D / 16;      // lanes per token row
  constexpr int RPW = kWave / LPR;  // token rows per wave step
  const int lane = threadIdx.x % kWave;
  const int h = blockIdx.y * kWavesPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.z, p = blockIdx.x;
  if (h >= a.Hk) return;  // no barriers below: a wave may leave on its own
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

  float qv[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t qo = (static_cast<int64_t>(b) * a.Hq + h * G + g) * D + seg * 16;
    const float4* qp = reinterpret_cast<const float4*>(a.q + qo);
    const float4* mp = a.q_mult ? reinterpret_cast<const float4*>(a.q_mult + (h * G + g) * D + seg * 16)
                                : nullptr;
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

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = 0.f;
  }

  const int64_t* bt = a.bt + static_cast<int64_t>(b) * a.max_blocks;
  const int64_t num_blocks = a.num_slots / a.bs;
  const int64_t row_stride = static_cast<int64_t>(a.Hk) * D;  // bytes between slots
  const int64_t head_off = static_cast<int64_t>(h) * D + seg * 16;

  for (int tb = t0; tb < t1; tb += RPW) {
    const int t = tb + r;
    bool valid = t < t1;
    int64_t slot = 0;
    if (valid) {
      const int64_t pb = bt[t / a.bs];
      valid = pb >= 0 && pb < num_blocks;
      slot = valid ? pb * a.bs + t % a.bs : 0;
    }
    const u32x4 kw = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(a.kc + slot * row_stride + head_off));
    const u32x4 vw = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(a.vc + slot * row_stride + head_off));
    const float ksc = a.ks[slot * a.Hk + h];
    const float vsc = a.vs[slot * a.Hk + h];

    float kf[16];
    unpack_i8x16(kw, kf);
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) d += qv[g][i] * kf[i];
      d = lsh::group_sum<LPR>(d);
      s[g] = valid ? (a.scale * ksc) * d : kNegBig;
    }
    float vf[16];
    unpack_i8x16(vw, vf);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float bm = lsh::wave_max_from<LPR>(s[g]);
      const float mn = fmaxf(m[g], bm);
      const float alpha = __builtin_amdgcn_exp2f((m[g] - mn) * kLog2e);
      const float pr = valid ? __builtin_amdgcn_exp2f((s[g] - mn) * kLog2e) : 0.f;
      l[g] = l[g] * alpha + pr;
      const float pv = pr * vsc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[g][i] = acc[g][i] * alpha + pv * vf[i];
      m[g] = mn;
    }
  }

  // fold the per-row partial sums (lanes with equal seg)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = lsh::wave_sum_from<LPR>(l[g]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] = lsh::wave_sum_from<LPR>(acc[g][i]);
  }
  if (a.NP == 1) {
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float inv = 1.f / l[g];
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
    float mm = m[0], ll = l[0];
#pragma unroll
    for (int g = 1; g < G; ++g)
      if (lane == g) {
        mm = m[g];
        ll = l[g];
      }
    a.part_ml[(pidx * G + lane) * 2] = mm;
    a.part_ml[(pidx * G + lane) * 2 + 1] = ll;
  }
}

// Merge of the partitions (paged_attention.cpp:432-455): one wavefront per (b, q head).
//   M = max_p m_p;  w_p = exp(m_p - M);  out = sum_p w_p acc_p / sum_p w_p l_p  (l_p = 0 skipped)
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
  for (int p = 0; p < a.NP; ++p) {
    const int64_t pi = (base + p) * G + g;
    const float lp = a.part_ml[pi * 2 + 1];
    if (lp == 0.f) continue;
    const float w = __builtin_amdgcn_exp2f((a.part_ml[pi * 2] - M) * kLog2e);
    L += w * lp;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int d = lane + i * kWave;
      if (d < D) o[i] += w * a.part_acc[pi * D + d];
    }
  }
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + i * kWave;
    if (d < D) a.out[item * D + d] = o[i] * inv;
  }
}

int auto_partition(int64_t B, int64_t Hk, int64_t max_ctx, int64_t bs) {
  // aim for ~8k wavefronts over the context bound, with >= 128 tokens per partition
  const int64_t target = 8192;
  const int64_t parts = (target + B * Hk - 1) / (B * Hk);
  int64_t P = (max_ctx + parts - 1) / parts;
  if (P < 128) P = 128;
  return static_cast<int>(P);
}

int64_t round_partition(int64_t P, int64_t B, int64_t Hk, int64_t max_blocks, int64_t bs) {
  const int64_t max_ctx = max_blocks * bs;
  if (P <= 0) P = auto_partition(B, Hk, max_ctx, bs);
  P = ((P + bs - 1) / bs) * bs;
  if (P > max_ctx && max_ctx > 0) P = ((max_ctx + bs - 1) / bs) * bs;
  return P < bs ? bs : P;
}

template <int D, int G>
void launch_decode(const DecodeArgs& a, int B, hipStream_t st) {
  const dim3 grid(a.NP, (a.Hk + kWavesPerBlock - 1) / kWavesPerBlock, B);
  hipLaunchKernelGGL((paged_decode_int8_kernel<D, G>), grid, dim3(kWavesPerBlock * kWave), 0, st, a);
  if (a.NP > 1) {
    const int64_t items = static_cast<int64_t>(B) * a.Hq;
    hipLaunchKernelGGL(paged_decode_merge_kernel<D>,
                       dim3(static_cast<unsigned>((items + kWavesPerBlock - 1) / kWavesPerBlock)),
                       dim3(kWavesPerBlock * kWave), 0, st, a, B);
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
  LSH_CHECK(max_blocks * block_size < (1LL << 31), "paged_attention: context too long");
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
  LSH_CHECK(NP <= 65535, "paged_attention: too many partitions");

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
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.max_blocks = static_cast<int>(max_blocks);
  a.bs = static_cast<int>(block_size);
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
