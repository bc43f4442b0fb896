// One decoder layer for a decode batch of at most 4 sequences, as ONE persistent launch: the
// layer's attention over its int8 paged cache, o_proj, residual add + post-attention RMSNorm,
// gate_up and silu * up, down_proj, residual add + the next layer's input RMSNorm, then the
// next layer's qkv projection with its q/k RMSNorm, RoPE at each sequence's position and the
// int8 K/V write (the reference's _forward_fused order, models/transformer.py:157-189, with
// the decode attention of paged_attention.cpp:191-420, the int4 linears of quant.py:134-151
// and the cache write of attention.py:241-246). At one to four rows each of these matrices is
// 1-3 MB: a kernel per op spends its time in launch and dependent-latency gaps (~3 us each,
// ten per layer), not in HBM. Here the weights of every stage are requested as soon as a
// workgroup is free, and the stages hand their small vectors to each other inside the launch.
//
// Workgroups (512 threads = 8 wavefronts, one per CU, all resident at once):
//   attention first:        workgroup w < M R runs one range of Q tokens of one row (a
//                           wavefront per kv head), the last M n_q workgroups merge one
//                           (row, query head) each (see "this layer's attention" below);
//   MLP groups w < H / 8:   o_proj rows 8w..8w+7 (a wavefront per row), gate rows and up rows
//                           of channels [C w, C (w + 1)) (C = I / (H / 8)), down rows
//                           8w..8w+7; for the last layer also those residual channels and
//                           their final norm.
//   head groups (after):    one q, k or v head of the next layer's qkv projection each (128
//                           rows, 16 per wavefront), a 1 / (n_q + 2 n_k) share of the new
//                           residual channels, the head's norm / RoPE / cache write.
// Hand-offs: a producer stores each output value as one 8-byte word (float bits | launch tag
// << 32) with a device-scope store; a consumer polls the words it needs with device-scope
// loads until every one carries this launch's tag, so data and readiness travel together and
// no counter or fence is needed. Five hand-offs per layer: attention partials (exa), merged
// attention rows (exb, Kq words per row), o_proj out (ex1, H words), silu * up (ex2, I words),
// down_proj out (ex3, H words). Every wait is bounded by `spin_limit` polls; a wait that runs
// out sets the error word and the workgroup returns, so the grid always drains. The launch tag
// is ctl[0] + 1 (never 0, the value of cleared words); the last workgroup to finish (ctl[1]
// counts them) resets the count and advances ctl[0], so the next launch on the stream uses a
// new tag. The caller's workspace holds ctl and the exchange buffers; launches that overlap
// on one workspace race.
//
// Layouts: int4 weights are the reference buffers (nibbles [N, K/2], even channel low;
// group scale / zero [N, K/128]); x' = x * inv_act_scale is staged in LDS with each
// 32-channel slice's eight 16-byte chunks rotated by half the slice index (conflict-free
// ds_read_b128); a lane holds 16-byte weight chunks (32 channels of one group) and computes
// s * sum x'q + (z - 8 s) * sum x' (int8_gemv.cpp:48-52), partial sums reduced with DPP.
#include <cmath>

#include "common.h"
#include "kv_quant.h"
#include "paged_core.h"
#include "rope.h"

namespace {

using lsh::kWave;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;  // 8
constexpr int kMaxRows = 4;   // sequences per launch
constexpr int kHeadDim = 128;
constexpr int kGroup = 128;   // quantization group (channels)
constexpr int kMaxH = 1024;   // hidden size: two channels per thread; gate_up / qkv rows are one
                              // 32-chunk half wavefront
constexpr int kMaxKq = 2048;  // o_proj input: one 64-chunk wavefront
constexpr int kMaxI = 4096;   // down_proj input: at most two chunks per lane
constexpr int kMaxGuPass = 4; // gate_up rows per workgroup <= 16 * kMaxGuPass
constexpr int kHeadPasses = kHeadDim / (2 * kWaves);  // 8: two qkv rows per wavefront per pass
constexpr int kGqa = 2;                   // query heads per kv head
constexpr int kPartWords = kHeadDim + 2;  // an attention partial: running max, sum, accumulator
constexpr int kMaxRanges = 128;           // attention ranges per row
constexpr int kMinRange = 64;             // tokens per attention range, at least
constexpr int kAccPerWave = kMaxRanges / kWaves;  // partials a merge wavefront accumulates
// words of the attention partials: [kMaxRows][kMaxRanges][kWaves][kGqa][kPartWords]
constexpr int64_t kExaWords = static_cast<int64_t>(kMaxRows) * kMaxRanges * kWaves * kGqa * kPartWords;


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct ChainArgs {
  // this layer's attention (MLP part): q [M, nq, D] as the previous launch wrote it, the
  // layer's int8 cache and the smoothing product q_mult [nq, D] (nullable)
  const float* q_in;
  const int8_t *akc, *avc;
  const float *aks, *avs;
  const float* q_mult;
  float qscale;     // softmax scale * log2(e)
  int bs_shift;     // log2(bs)
  // residual stream and outputs
  const float* x_in;   // [M, H] residual stream before this layer's o_proj (MLP part)
  const int64_t* ids;  // [M] token ids: embedding mode (no MLP part)
  const float* embed;  // [V, H]
  int64_t vocab;
  float* x_out;        // [M, H] residual after the down_proj add (or the embedding rows)
  float* h_out;        // [M, H] the final norm's output (last layer) or null
  // this layer: o_proj, post-attention norm, gate_up, down_proj; then the next norm
  const uint8_t* o_nib;
  const float *o_s, *o_z, *o_inv;
  const float* post_w;
  const uint8_t* gu_nib;
  const float *gu_s, *gu_z, *gu_inv;
  const uint8_t* dn_nib;
  const float *dn_s, *dn_z, *dn_inv;
  const float* next_w;
  // the next layer's qkv projection, q/k norm, RoPE and cache write
  const uint8_t* qkv_nib;
  const float *qkv_s, *qkv_z, *qkv_inv;
  const float *q_w, *k_w;
  const float *cos_t, *sin_t;
  int64_t max_pos;
  const int64_t* ctx;  // [M] context length including the token (position ctx - 1)
  const int64_t* bt;   // [M, max_blocks]
  int64_t max_blocks, bs, num_slots;
  const float* smooth;  // [nk, D] or null
  float* q_out;         // [M, nq, D]
  int8_t *kc, *vc;
  float *ks, *vs;
  // hand-offs and control words
  uint64_t *ex1, *ex2, *ex3;  // [kCopies][kMaxRows][H], [..][I], [..][H] words
  uint64_t* exa;              // attention partials, kExaWords words
  uint64_t* exb;              // merged attention rows [kCopies][kMaxRows][Kq] words
  uint32_t* ctl;              // tag base, finished workgroups, error
  uint32_t spin_limit;
  int M, H, Kq, I, nq, nk;
  int mlp_groups;   // H / 8, or 0 (embedding mode)
  int head_groups;  // nq + 2 nk, or 0 (last layer)
  int grid;         // mlp_groups + head_groups
  float eps;
};

// ---- hand-off words --------------------------------------------------------------------------
// Each hand-off vector is written in kCopies replicas and a consumer reads the replica of its
// workgroup index modulo kCopies (the XCD it most likely runs on): every replica's lines are
// polled by an eighth of the consumers. A consumer polls two words per 16-byte device-scope
// load (each 8-byte word is stored whole, so each half of a load is one word as stored).

constexpr int kCopies = 8;
// words of the merged attention rows: [kCopies][kMaxRows][kMaxKq]
constexpr int64_t kExbWords = static_cast<int64_t>(kCopies) * kMaxRows * kMaxKq;
constexpr int kPolicyDevice = 16;  // buffer-load cache policy: device scope (sc1)

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void put(uint64_t* base, int64_t stride, int64_t idx, float v,
                                    uint32_t tag) {
  const uint64_t w = (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
#pragma unroll
  for (int c = 0; c < kCopies; ++c)
    __hip_atomic_store(base + c * stride + idx, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls the word pairs at byte offsets off(i) of `src` (a 16-byte aligned buffer resource)
// for the i set in `need` (N <= 32) until both words carry `tag`, handing each pair's values to
// sink(i, lo, hi) as it arrives. Every round issues the loads of all missing pairs together.
// Returns false when the poll budget runs out (the error word is then set).
template <int N, typename Off, typename Sink>
__device__ bool take(__amdgpu_buffer_rsrc_t src, uint32_t need, uint32_t tag, const ChainArgs& a,
                     Off off, Sink sink) {
  static_assert(N <= 32, "take: at most 32 pairs per thread");
  uint32_t ready = 0;
  for (uint32_t spin = 0;; ++spin) {
    u32x4v w[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((need & ~ready) >> i & 1u)
        w[i] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(
                                              src, static_cast<uint32_t>(off(i)), 0, kPolicyDevice));
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (!((need & ~ready) >> i & 1u)) continue;
      const uint32_t t0 = w[i][1], t1 = w[i][3], v0 = w[i][0], v1 = w[i][2];
      if (t0 == tag && t1 == tag) {
        sink(i, __builtin_bit_cast(float, v0), __builtin_bit_cast(float, v1));
        ready |= 1u << i;
      }
    }
    if (ready == need) return true;
    if (spin >= a.spin_limit) {
      __hip_atomic_fetch_or(a.ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// True in every thread when `v` is true in any thread of the block. `slots` holds kWaves ints
// of LDS that no other code uses. (The runtime's __syncthreads_or reads the workgroup size
// from the dispatch packet with a global load on every call: a memory round trip on the
// critical path after each hand-off.)
__device__ __forceinline__ bool block_any(bool v, int* slots) {
  const bool w = __builtin_amdgcn_ballot_w64(v) != 0;
  __syncthreads();  // the previous call's reads are done
  if (threadIdx.x % kWave == 0) slots[threadIdx.x / kWave] = w;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r |= slots[i];
  return r != 0;
}

// A long wait, thinned: wavefront 0 alone polls a few sentinel pairs (take's `need` and
// `off` for its lanes) while the other wavefronts wait at the barrier; the full take that
// follows then normally completes in its first round. Device-scope polls are served beyond
// the XCD's L2, so a whole workgroup polling every word it needs through a wait of several
// microseconds puts megabytes per round on the fabric, in the way of the loads of the
// workgroups still computing. (Polling the sentinels faster, several rounds in flight, was
// measured slower for the same reason.) Returns the block-wide verdict (false: the error word
// is set).
template <int N, typename Off>
__device__ bool gate(__amdgpu_buffer_rsrc_t src, uint32_t need, uint32_t tag, const ChainArgs& a,
                     Off off, int* flags) {
  bool ok = true;
  if (threadIdx.x < kWave) ok = take<N>(src, need, tag, a, off, [](int, float, float) {});
  return !block_any(!ok, flags);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t replica(const uint64_t* base, int64_t words) {
  const int c = blockIdx.x % kCopies;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base + c * words), 0,
                                           static_cast<int>(words * 8), 0x00020000);
}

// ---- staging and dot products ------------------------------------------------------------------

// LDS offset of channel k of a staged row: 32-channel slice sl = k / 32 keeps its eight
// 16-byte chunks rotated by sl / 2 (the two slices of a 256-byte LDS row share a rotation),
// which SQ_LDS_BANK_CONFLICT shows conflict-free for a wavefront reading chunk j of
// consecutive slices on gfx950 (a rotation by sl costs 4 conflict cycles per ds_read_b128).
// Channels 2p and 2p + 1 stay adjacent.
__device__ __forceinline__ int chunk_rot(int sl) { return sl >> 1; }
__device__ __forceinline__ int xoff(int k) {
  const int sl = k >> 5, j = (k >> 2) & 7;
  return (sl << 5) + (((j + chunk_rot(sl)) & 7) << 2) + (k & 3);
}

__device__ __forceinline__ float4 lds4(const float* p) {
  return *static_cast<const float4*>(__builtin_assume_aligned(p, 16));
}

__device__ __forceinline__ float4 mul4(float4 v, float4 t) {
  return make_float4(__fmul_rn(v.x, t.x), __fmul_rn(v.y, t.y), __fmul_rn(v.z, t.z),
                     __fmul_rn(v.w, t.w));
}

// A lane's 16-byte weight chunk (32 channels of one group) with the group scale s and z - 8 s;
// `on` false: no chunk (the loads are clamped in bounds, the terms zeroed).
struct Chunk {
  u32x4 w;
  float s, zc;
  bool on;
};

__device__ __forceinline__ Chunk fetch(const uint8_t* nib, const float* gs, const float* gz,
                                       int K, int64_t row, int c, bool on) {
  const int G = K / kGroup;
  const int cc = on ? c : 0;
  Chunk f;
  f.w = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(nib + row * (K / 2) + static_cast<int64_t>(cc) * 16));
  const float s = gs[row * G + cc / 4], z = gz[row * G + cc / 4];
  f.s = s;
  f.zc = z - 8.f * s;
  f.on = on;
  return f;
}

// The lane's terms s * sum x'q + (z - 8 s) * sum x' of chunk c (channels 32c..32c+31) of
// the staged rows m < MT of K channels; sum x' is the chunk's sum cs[m * K / 32 + c], staged
// with the row (it is the same for every weight row).
template <int MT>
__device__ __forceinline__ void chunk_terms(const Chunk& f, int c, const float* xs, const float* cs,
                                            int K, float (&v)[MT]) {
  float q[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = f.w[i];
    uint32_t lo = u & 0x0f0f0f0fu, hi = (u >> 4) & 0x0f0f0f0fu;
    // hides the masks: each value is then one byte-select conversion (v_cvt_f32_ubyteN)
    // instead of a bit-field extract and a conversion; the asm emits nothing
    asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      q[8 * i + 2 * b] = static_cast<float>((lo >> (8 * b)) & 0xffu);
      q[8 * i + 2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xffu);
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float* row = xs + m * K + (c << 5);
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 x = lds4(row + (((j + chunk_rot(c)) & 7) << 2));
      d += x.x * q[4 * j] + x.y * q[4 * j + 1] + x.z * q[4 * j + 2] + x.w * q[4 * j + 3];
    }
    v[m] = f.on ? f.s * d + f.zc * cs[m * (K >> 5) + c] : 0.f;
  }
}

// Rows [0, MT) of a [M, K] source (K <= kMaxKq; rows >= M repeat row M - 1 and are never
// summed) times inv (nullable; the reference's separate float32 multiply), as float4 chunks in
// registers: loaded before any later stage's weights, so that the LDS stores wait for these
// loads only.
template <int MT>
struct Staged {
  static constexpr int kN = MT * kMaxKq / 4 / kThreads;
  float4 v[kN];
};

template <int MT>
__device__ __forceinline__ void stage_load(Staged<MT>& st, const float* src, const float* inv,
                                           int K, int M) {
  const int n4 = MT * K / 4;
#pragma unroll
  for (int u = 0; u < Staged<MT>::kN; ++u) {
    const int q = min(static_cast<int>(threadIdx.x) + u * kThreads, n4 - 1);
    const int m = (q * 4) / K, k = (q * 4) % K;
    st.v[u] = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(min(m, M - 1)) * K + k);
    if (inv) st.v[u] = mul4(st.v[u], *reinterpret_cast<const float4*>(inv + k));
  }
}

// The staged rows -> LDS (xoff layout) and their chunk sums -> cs (a chunk is the float4s of
// 8 consecutive threads; K is a multiple of 128, so those 8 are all in or all out).
template <int MT>
__device__ __forceinline__ void stage_store(const Staged<MT>& st, float* xs, float* cs, int K) {
  const int n4 = MT * K / 4;
#pragma unroll
  for (int u = 0; u < Staged<MT>::kN; ++u) {
    const int q = static_cast<int>(threadIdx.x) + u * kThreads;
    const float4 x = st.v[u];
    const float sum = lsh::group_sum<8>((x.x + x.y) + (x.z + x.w));
    if (q < n4) {
      const int m = (q * 4) / K, k = (q * 4) % K;
      *reinterpret_cast<float4*>(xs + m * K + xoff(k)) = x;
      if (q % 8 == 0) cs[m * (K >> 5) + (k >> 5)] = sum;
    }
  }
}

// Block sum of one value per thread in a fixed order; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = lsh::wave_sum_from<1>(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

// Residual rows: thread t holds channels 2t and 2t + 1 of rows m < MT.
template <int MT>
struct Resid {
  float v[MT][2];
};

template <int MT>
__device__ __forceinline__ void row_inv_rms(const Resid<MT>& r, int H, int M, float eps,
                                            float* red, float (&inv)[MT]) {
  const bool own = 2 * static_cast<int>(threadIdx.x) < H;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float ss = own && m < M ? r.v[m][0] * r.v[m][0] + r.v[m][1] * r.v[m][1] : 0.f;
    const float tot = block_sum(ss, red);
    inv[m] = 1.f / sqrtf(tot / static_cast<float>(H) + eps);
  }
}

// A thread's two channels of a [H] vector (zero past H; null gives `dflt`).
__device__ __forceinline__ float2 chan2(const float* p, int H, float dflt) {
  const int k0 = 2 * threadIdx.x;
  if (p == nullptr) return make_float2(dflt, dflt);
  return k0 < H ? *reinterpret_cast<const float2*>(p + k0) : make_float2(0.f, 0.f);
}

// The RMSNorm w * (r * inv) of the residual rows times act_inv (when given) -> LDS (xoff),
// and each 32-channel chunk's sum (16 consecutive threads; H is a multiple of 128) -> cs.
template <int MT>
__device__ __forceinline__ void norm_to_lds(const Resid<MT>& r, float2 wv, float2 iv, bool inv_on,
                                            float eps, int H, int M, float* xs, float* cs,
                                            float* red) {
  float inv[MT];
  row_inv_rms(r, H, M, eps, red, inv);
  const int t = threadIdx.x, k0 = 2 * t;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float h0 = wv.x * (r.v[m][0] * inv[m]), h1 = wv.y * (r.v[m][1] * inv[m]);
    if (inv_on) {
      h0 = __fmul_rn(h0, iv.x);
      h1 = __fmul_rn(h1, iv.y);
    }
    const float sum = lsh::group_sum<16>(h0 + h1);
    if (k0 < H) {
      *reinterpret_cast<float2*>(xs + m * H + xoff(k0)) = make_float2(h0, h1);
      if (t % 16 == 0) cs[m * (H >> 5) + (t >> 4)] = sum;
    }
  }
}

template <int MT>
__device__ __forceinline__ void load_rows(const float* src, int H, int M, Resid<MT>& x) {
  const int k0 = 2 * threadIdx.x;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float2 v = (m < M && k0 < H)
                         ? *reinterpret_cast<const float2*>(src + static_cast<int64_t>(m) * H + k0)
                         : make_float2(0.f, 0.f);
    x.v[m][0] = v.x;
    x.v[m][1] = v.y;
  }
}

// Writes the residual channels [lo, hi) of rows m < M (thread t owns 2t, 2t + 1).
template <int MT>
__device__ __forceinline__ void store_rows(const Resid<MT>& x, float* out, int H, int M, int lo,
                                           int hi) {
  const int k0 = 2 * threadIdx.x;
  if (k0 < lo || k0 >= hi || k0 >= H) return;
#pragma unroll
  for (int m = 0; m < MT; ++m)
    if (m < M)
      *reinterpret_cast<float2*>(out + static_cast<int64_t>(m) * H + k0) =
          make_float2(x.v[m][0], x.v[m][1]);
}

// Marks this workgroup finished; the last one advances the tag base (skipping the value whose
// tag would wrap to 0) for the next launch. Every workgroup read the base before it counted itself.
__device__ __forceinline__ void finish(const ChainArgs& a) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t n = __hip_atomic_fetch_add(a.ctl + 1, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    if (n + 1 == static_cast<uint32_t>(a.grid)) {
      const uint32_t cur = __hip_atomic_load(a.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctl, cur >= 0xfffffffeu ? 0u : cur + 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// This launch's tag: the base the previous launch left, plus one. Read after a workgroup has
// requested its weights, so that those loads do not queue behind this device-scope read.
__device__ __forceinline__ uint32_t launch_tag(const ChainArgs& a) {
  return __hip_atomic_load(a.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

// Bits 0 .. n-1.
__device__ __forceinline__ uint32_t low_bits(int n) { return n >= 32 ? ~0u : (1u << n) - 1u; }

// ---- this layer's attention -----------------------------------------------------------------
// The rows' contexts are cut into ranges of Q tokens, R per row (Q from the longest context,
// the same in every workgroup): workgroup w < M R runs range j = w % R of row m = w / R,
// tokens [j Q, (j + 1) Q), its wavefront h < nk taking kv head h (the split-context decode of
// paged_core.h: a range's eight wavefronts read each token's whole row of kv heads). Each
// (m, j, h, g) leaves a partial of kPartWords tagged words (running max, sum, accumulator) in
// exa. Ranges past a row's context write nothing: the merge reads only the ceil(ctx / Q)
// ranges with tokens.

__device__ __forceinline__ int64_t part_word(const ChainArgs& a, int m, int j, int h, int g) {
  return ((((static_cast<int64_t>(m) * kMaxRanges + j) * a.nk + h) * kGqa) + g) * kPartWords;
}

__device__ __forceinline__ int row_context(const ChainArgs& a, int m) {
  const int64_t cap = a.max_blocks * a.bs;
  const int64_t c = uniform64(a.ctx[m]);
  return static_cast<int>(c < 0 ? 0 : (c > cap ? cap : c));
}

// Q: at least kMinRange tokens, at most floor(grid / M) ranges per row (so that the M R
// ranges have a workgroup each) and at most kMaxRanges; a multiple of 16.
struct AttnPlan {
  int Q, R;
};

__device__ __forceinline__ AttnPlan attn_plan(const ChainArgs& a) {
  int mx = 0;
  for (int m = 0; m < a.M; ++m) mx = max(mx, row_context(a, m));
  const int per = a.grid / a.M;
  int q = max(kMinRange, max((mx + per - 1) / per, (mx + kMaxRanges - 1) / kMaxRanges));
  q = (q + 15) & ~15;
  return {q, (mx + q - 1) / q};
}

__device__ void attention_range(const ChainArgs& a, const AttnPlan& pl, uint32_t tag) {
  const int w = blockIdx.x;
  if (w >= a.M * pl.R) return;
  const int m = w / pl.R, j = w % pl.R;
  const int h = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (h >= a.nk) return;
  const int ctx = row_context(a, m);
  const int t0 = j * pl.Q;
  if (t0 >= ctx) return;
  const int t1 = min(t0 + pl.Q, ctx);
  DecodeArgs d{};
  d.q = a.q_in;
  d.kc = a.akc;
  d.vc = a.avc;
  d.ks = a.aks;
  d.vs = a.avs;
  d.bt = a.bt;
  d.row_tab = nullptr;
  d.cl = a.ctx;
  d.q_mult = a.q_mult;
  d.num_slots = a.num_slots;
  d.B = a.M;
  d.Hq = a.nq;
  d.Hk = a.nk;
  d.max_blocks = static_cast<int>(a.max_blocks);
  d.bs = static_cast<int>(a.bs);
  d.bs_shift = a.bs_shift;
  d.qscale = a.qscale;
  SegState<kGqa> st;
  segment_state<int8_t, kHeadDim, kGqa, true, true>(d, m, h, t0, t1, st);
  constexpr int LPR = kHeadDim / 16;
  const int r = lane / LPR, seg = lane % LPR;
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < kGqa; ++g) {
      uint64_t* p = a.exa + part_word(a, m, j, h, g) + 2 + seg * 16;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint64_t wv = (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, st.acc[g][i]);
        __hip_atomic_store(p + i, wv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (lane < kGqa) {
    const float mm = lane == 0 ? st.m[0] : st.m[1];
    const float ll = lane == 0 ? st.lt[0] : st.lt[1];
    uint64_t* p = a.exa + part_word(a, m, j, h, lane);
    __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, mm),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, ll),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Merge i = grid - 1 - w of (row m, query head qh), i < M nq, by all 8 wavefronts of workgroup
// w (the last workgroups, whose own weights are needed last): wavefront 0 first waits for the
// (max, sum) words of the row's np partials (the producers store them after the
// accumulators), then every wavefront takes the (max, sum) words (lane p) and the
// accumulators of partials v, v + 8, ... (wavefront v) in one polling round, and the merge is
// the decode merge's (paged_decode.hip, merge_unit): M = max_p m_p, w_p = exp2(m_p - M) (0
// where the sum is 0), out = (sum_p w_p acc_p) / (sum_p w_p l_p), the wavefronts' sums added
// in wavefront order (a row without context gets NaN). The row goes to exb (all replicas) for
// the o_proj stage. `red2` is 2 kThreads floats of LDS. Returns false when a wait ran out of
// polls.
__device__ bool merge_attention(const ChainArgs& a, const AttnPlan& pl, uint32_t tag, float* red2,
                                int* flags) {
  const int i = a.grid - 1 - static_cast<int>(blockIdx.x);
  if (i < 0 || i >= a.M * a.nq) return true;
  const int m = i / a.nq, qh = i % a.nq, h = qh / kGqa, g = qh % kGqa;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int ctx = row_context(a, m);
  const int np = (ctx + pl.Q - 1) / pl.Q;
  const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
      a.exa, 0, static_cast<int>(kExaWords * 8), 0x00020000);
  // pairs 0, 1: (max, sum) of partials lane and lane + 64; pairs 2..: this lane's accumulator
  // pair (dims 2 lane, 2 lane + 1) of partials wave + 8 t
  const int64_t ml0 = part_word(a, m, lane, h, g) * 8;
  const int64_t ml_step = part_word(a, 0, kWave, 0, 0) * 8;  // 64 partials further on
  const uint32_t need_ml = (lane < np ? 1u : 0u) | (lane + kWave < np ? 2u : 0u);
  if (!gate<2>(src, need_ml, tag, a, [=](int k) { return ml0 + k * ml_step; }, flags))
    return false;
  constexpr int N = 2 + kAccPerWave;
  uint32_t need = need_ml;
  for (int t = 0; t < kAccPerWave; ++t)
    if (wave + kWaves * t < np) need |= 1u << (2 + t);
  float pm[2] = {kNegBig, kNegBig}, ps[2] = {0.f, 0.f};
  float av[kAccPerWave][2] = {};
  const bool ok = take<N>(
      src, need, tag, a,
      [&](int k) {
        if (k < 2) return ml0 + k * ml_step;
        return (part_word(a, m, wave + kWaves * (k - 2), h, g) + 2 + 2 * lane) * 8;
      },
      [&](int k, float v0, float v1) {
        if (k < 2) {
          pm[k] = v0;
          ps[k] = v1;
        } else {
          av[k - 2][0] = v0;
          av[k - 2][1] = v1;
        }
      });
  float mx = fmaxf(pm[0], pm[1]);
  mx = lsh::wave_max_from<1>(mx);
  float wt[2], L = 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    wt[k] = ps[k] == 0.f ? 0.f : __builtin_amdgcn_exp2f(pm[k] - mx);
    L += wt[k] * ps[k];
  }
  L = lsh::group_sum<kWave>(L);
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int t = 0; t < kAccPerWave; ++t) {
    const int p = wave + kWaves * t;
    const float wp = __shfl(p < kWave ? wt[0] : wt[1], p % kWave, kWave);
    if (p < np) {
      o0 += wp * av[t][0];
      o1 += wp * av[t][1];
    }
  }
  __syncthreads();
  red2[(wave * kWave + lane) * 2] = o0;
  red2[(wave * kWave + lane) * 2 + 1] = o1;
  __syncthreads();
  if (wave == 0) {
    float s0 = red2[lane * 2], s1 = red2[lane * 2 + 1];
    for (int v = 1; v < kWaves; ++v) {
      s0 += red2[(v * kWave + lane) * 2];
      s1 += red2[(v * kWave + lane) * 2 + 1];
    }
    const float inv = np > 0 ? 1.f / L : __builtin_nanf("");
    const int64_t s = static_cast<int64_t>(kMaxRows) * a.Kq;
    const int64_t at = static_cast<int64_t>(m) * a.Kq + qh * kHeadDim + 2 * lane;
    put(a.exb, s, at, np > 0 ? s0 * inv : inv, tag);
    put(a.exb, s, at + 1, np > 0 ? s1 * inv : inv, tag);
  }
  __syncthreads();
  return ok;
}

// ---- the two kinds of workgroup ----------------------------------------------------------------

template <int MT>
__device__ void mlp_group(const ChainArgs& a, float* xs, float* cs, float* rows, float* red,
                          int* flags) {
  const int w = blockIdx.x;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int H = a.H, Kq = a.Kq, I = a.I, M = a.M;
  const int C = I / a.mlp_groups;  // gate (and up) channels of this workgroup
  const int passes = 2 * C / (2 * kWaves);
  const int half = lane / 32, hl = lane % 32;
  const int k0 = 2 * threadIdx.x;
  const int64_t s1 = static_cast<int64_t>(kMaxRows) * H, s2 = static_cast<int64_t>(kMaxRows) * I;
  constexpr int kPairs = kMaxI / 2 / kThreads;  // down-input word pairs per thread per row

  constexpr int kOPairs = kMaxKq / 2 / kThreads;  // o_proj-input word pairs per thread per row

  // 1. every weight and small vector a stage needs, so that no stage after a hand-off waits
  //    for memory
  const int orow = 8 * w + wave;
  const Chunk fo = fetch(a.o_nib, a.o_s, a.o_z, Kq, orow, lane, lane < Kq / 32);
  float2 o_inv[kOPairs];
#pragma unroll
  for (int i = 0; i < kOPairs; ++i) {
    const int pr = static_cast<int>(threadIdx.x) + i * kThreads;  // channels 2pr, 2pr + 1
    o_inv[i] = (a.o_inv && 2 * pr < Kq) ? *reinterpret_cast<const float2*>(a.o_inv + 2 * pr)
                                        : make_float2(1.f, 1.f);
  }
  Chunk fg[kMaxGuPass];
#pragma unroll
  for (int p = 0; p < kMaxGuPass; ++p) {
    const int r = 16 * p + 2 * wave + half;  // gate rows 0..C-1, then up rows
    const bool on = p < passes && hl < H / 32;
    const int row = p < passes ? (r < C ? C * w + r : I + C * w + (r - C)) : C * w;
    fg[p] = fetch(a.gu_nib, a.gu_s, a.gu_z, H, row, hl, on);
  }
  const Chunk fd0 = fetch(a.dn_nib, a.dn_s, a.dn_z, I, orow, lane, lane < I / 32);
  const Chunk fd1 = fetch(a.dn_nib, a.dn_s, a.dn_z, I, orow, lane + kWave, lane + kWave < I / 32);
  Resid<MT> x;
  load_rows(a.x_in, H, M, x);
  const float2 post_w = chan2(a.post_w, H, 1.f), gu_inv = chan2(a.gu_inv, H, 1.f);
  const float2 next_w = chan2(a.next_w, H, 1.f);
  float2 dn_inv[kPairs];
#pragma unroll
  for (int i = 0; i < kPairs; ++i) {
    const int pr = static_cast<int>(threadIdx.x) + i * kThreads;  // channels 2pr, 2pr + 1
    dn_inv[i] = (a.dn_inv && 2 * pr < I) ? *reinterpret_cast<const float2*>(a.dn_inv + 2 * pr)
                                         : make_float2(1.f, 1.f);
  }
  const uint32_t tag = launch_tag(a);

  // 2. the merged attention rows times o_proj's inv -> LDS (xoff) with their chunk sums
  {
    uint32_t need = 0;
#pragma unroll
    for (int i = 0; i < MT * kOPairs; ++i)
      if (i / kOPairs < M && 2 * (static_cast<int>(threadIdx.x) + (i % kOPairs) * kThreads) < Kq)
        need |= 1u << i;
    const int64_t sb = static_cast<int64_t>(kMaxRows) * Kq;
    const __amdgpu_buffer_rsrc_t rb = replica(a.exb, sb);
    // sentinels: the first pair of each merged head row (lane i: row i / nq, head i % nq)
    const int soff = ((lane / a.nq) * Kq + (lane % a.nq) * kHeadDim) * 8;
    if (!gate<1>(rb, lane < M * a.nq ? 1u : 0u, tag, a, [=](int) { return soff; }, flags))
      return finish(a);
    const bool ok = take<MT * kOPairs>(
        rb, need, tag, a,
        [&](int i) {
          return ((i / kOPairs) * Kq + 2 * (static_cast<int>(threadIdx.x) + (i % kOPairs) * kThreads)) * 8;
        },
        [&](int i, float v0, float v1) {
          const int k = 2 * (static_cast<int>(threadIdx.x) + (i % kOPairs) * kThreads);
          const float2 iv = o_inv[i % kOPairs];
          *reinterpret_cast<float2*>(xs + (i / kOPairs) * Kq + xoff(k)) =
              a.o_inv ? make_float2(__fmul_rn(v0, iv.x), __fmul_rn(v1, iv.y)) : make_float2(v0, v1);
        });
    if (block_any(!ok, flags)) return finish(a);
#pragma unroll
    for (int i = 0; i < MT * kOPairs; ++i) {
      const int pr = static_cast<int>(threadIdx.x) + (i % kOPairs) * kThreads;
      const bool in = (need >> i) & 1u;
      float2 v = make_float2(0.f, 0.f);
      if (in) v = *reinterpret_cast<const float2*>(xs + (i / kOPairs) * Kq + xoff(2 * pr));
      const float sum = lsh::group_sum<16>(v.x + v.y);
      if (in && pr % 16 == 0) cs[(i / kOPairs) * (Kq >> 5) + (pr >> 4)] = sum;
    }
    __syncthreads();
  }

  // 3. o_proj row 8w + wave -> ex1
  {
    float v[MT];
    chunk_terms<MT>(fo, lane, xs, cs, Kq, v);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float t = lsh::group_total<kWave>(v[m]);
      if (m < M && lane == kWave - 1) put(a.ex1, s1, m * H + orow, t, tag);
    }
  }

  // 4. x += o (all channels, all rows), post-attention norm times gate_up's inv -> LDS
  {
    float o[MT][2];
    const bool ok = take<MT>(
        replica(a.ex1, s1), k0 < H ? low_bits(M) : 0u, tag, a,
        [&](int m) { return (m * H + k0) * 8; },
        [&](int m, float v0, float v1) {
          o[m][0] = v0;
          o[m][1] = v1;
        });
    if (block_any(!ok, flags)) return finish(a);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      x.v[m][0] = x.v[m][0] + o[m][0];
      x.v[m][1] = x.v[m][1] + o[m][1];
    }
    norm_to_lds(x, post_w, gu_inv, a.gu_inv != nullptr, a.eps, H, M, xs, cs, red);
    __syncthreads();
  }

  // 5. gate_up rows (16 per pass), silu(gate) * up of the workgroup's C channels -> ex2
  {
#pragma unroll
    for (int p = 0; p < kMaxGuPass; ++p) {
      if (p >= passes) break;
      float v[MT];
      chunk_terms<MT>(fg[p], hl, xs, cs, H, v);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float t = lsh::group_total<32>(v[m]);
        if (hl == 31) rows[(16 * p + 2 * wave + half) * MT + m] = t;
      }
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < C * M) {
      const int j = t % C, m = t / C;
      const float g = rows[j * MT + m], u = rows[(C + j) * MT + m];
      put(a.ex2, s2, m * I + C * w + j, g / (1.f + expf(-g)) * u, tag);
    }
  }

  // 6. down_proj row 8w + wave over the I channels of silu * up -> ex3
  {
    uint32_t need = 0;
#pragma unroll
    for (int i = 0; i < MT * kPairs; ++i)
      if (i / kPairs < M && 2 * (static_cast<int>(threadIdx.x) + (i % kPairs) * kThreads) < I)
        need |= 1u << i;
    __syncthreads();  // every wavefront is done with the gate_up stage's LDS rows
    const bool ok = take<MT * kPairs>(
        replica(a.ex2, s2), need, tag, a,
        [&](int i) {
          return ((i / kPairs) * I + 2 * (static_cast<int>(threadIdx.x) + (i % kPairs) * kThreads)) * 8;
        },
        [&](int i, float v0, float v1) {
          const int k = 2 * (static_cast<int>(threadIdx.x) + (i % kPairs) * kThreads);
          const float2 iv = dn_inv[i % kPairs];
          *reinterpret_cast<float2*>(xs + (i / kPairs) * I + xoff(k)) =
              a.dn_inv ? make_float2(__fmul_rn(v0, iv.x), __fmul_rn(v1, iv.y)) : make_float2(v0, v1);
        });
    if (block_any(!ok, flags)) return finish(a);
    float v0[MT], v1[MT];
    // each 32-channel chunk's sum: the pairs of 16 consecutive threads (I is a multiple of 512,
    // so those 16 are all in or all out)
#pragma unroll
    for (int i = 0; i < MT * kPairs; ++i) {
      const int pr = static_cast<int>(threadIdx.x) + (i % kPairs) * kThreads;
      const bool in = (need >> i) & 1u;
      float2 v = make_float2(0.f, 0.f);
      if (in) v = *reinterpret_cast<const float2*>(xs + (i / kPairs) * I + xoff(2 * pr));
      const float sum = lsh::group_sum<16>(v.x + v.y);
      if (in && pr % 16 == 0) cs[(i / kPairs) * (I >> 5) + (pr >> 4)] = sum;
    }
    __syncthreads();
    chunk_terms<MT>(fd0, lane, xs, cs, I, v0);
    chunk_terms<MT>(fd1, lane + kWave, xs, cs, I, v1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float t = lsh::group_total<kWave>(v0[m] + v1[m]);
      if (m < M && lane == kWave - 1) put(a.ex3, s1, m * H + orow, t, tag);
    }
  }

  // 7. the last layer: x += down, the residual channels 8w..8w+7 and their final norm
  if (a.head_groups == 0) {
    float dv[MT][2];
    const bool ok = take<MT>(
        replica(a.ex3, s1), k0 < H ? low_bits(M) : 0u, tag, a,
        [&](int m) { return (m * H + k0) * 8; },
        [&](int m, float v0, float v1) {
          dv[m][0] = v0;
          dv[m][1] = v1;
        });
    if (block_any(!ok, flags)) return finish(a);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      x.v[m][0] = x.v[m][0] + dv[m][0];
      x.v[m][1] = x.v[m][1] + dv[m][1];
    }
    store_rows(x, a.x_out, H, M, 8 * w, 8 * w + 8);
    if (a.h_out) {
      float inv[MT];
      row_inv_rms(x, H, M, a.eps, red, inv);
      if (k0 >= 8 * w && k0 < 8 * w + 8) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < M)
            *reinterpret_cast<float2*>(a.h_out + static_cast<int64_t>(m) * H + k0) =
                make_float2(next_w.x * (x.v[m][0] * inv[m]), next_w.y * (x.v[m][1] * inv[m]));
      }
    }
  }
  finish(a);
}

template <int MT>
__device__ void head_group(const ChainArgs& a, float* xs, float* cs, float* out, float* red,
                           int* flags) {
  const int hh = blockIdx.x - a.mlp_groups;  // q heads, then k heads, then v heads
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int H = a.H, M = a.M;
  const int half = lane / 32, hl = lane % 32;
  const int k0 = 2 * threadIdx.x;
  constexpr int D = kHeadDim;
  const int64_t s1 = static_cast<int64_t>(kMaxRows) * H;
  const bool is_q = hh < a.nq, is_k = !is_q && hh < a.nq + a.nk;

  // 1. the head's 128 qkv rows (a lane: chunk hl of rows 16 wave + 2 p + half), then every
  //    small vector the later stages need: the norm weight and qkv's inv, and for wavefront
  //    m < M the position, slot, RoPE row, q/k norm weight and smoothing of sequence m
  Chunk fq[kHeadPasses];
#pragma unroll
  for (int p = 0; p < kHeadPasses; ++p)
    fq[p] = fetch(a.qkv_nib, a.qkv_s, a.qkv_z, H, static_cast<int64_t>(hh) * D + 16 * wave + 2 * p + half,
                  hl, hl < H / 32);
  const float2 next_w = chan2(a.next_w, H, 1.f), qkv_inv = chan2(a.qkv_inv, H, 1.f);
  const int m = wave;  // stage 4: one wavefront per sequence
  int64_t pos = -1, slot = -1;
  float cosv[2] = {0.f, 0.f}, sn[2] = {0.f, 0.f}, nw[2] = {1.f, 1.f}, sm[2] = {1.f, 1.f};
  const float* nwp = is_q ? a.q_w : (is_k ? a.k_w : nullptr);
  const int kvh = is_k ? hh - a.nq : hh - a.nq - a.nk;
  if (m < M) {
    pos = a.ctx[m] - 1;
    if (pos >= 0 && pos < a.max_pos && pos / a.bs < a.max_blocks) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        cosv[i] = a.cos_t[pos * D + lane + i * kWave];
        sn[i] = a.sin_t[pos * D + lane + i * kWave];
        if (nwp) nw[i] = nwp[lane + i * kWave];
        if (is_k && a.smooth) sm[i] = a.smooth[static_cast<int64_t>(kvh) * D + lane + i * kWave];
      }
      if (!is_q) {
        const int64_t blk = a.bt[m * a.max_blocks + pos / a.bs];
        slot = blk * a.bs + pos % a.bs;
        if (blk < 0 || slot >= a.num_slots) slot = -1;
      }
    } else {
      pos = -1;
    }
  }
  const uint32_t tag = launch_tag(a);
  // 2. the residual rows: (x + o) + down, or the embedding rows
  Resid<MT> x;
  if (a.mlp_groups == 0) {
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      const int64_t id = r < M ? a.ids[r] : 0;
      float2 v = make_float2(0.f, 0.f);
      if (r < M && k0 < H)
        v = (id >= 0 && id < a.vocab) ? *reinterpret_cast<const float2*>(a.embed + id * H + k0)
                                      : make_float2(__builtin_nanf(""), __builtin_nanf(""));
      x.v[r][0] = v.x;
      x.v[r][1] = v.y;
    }
  } else {
    load_rows(a.x_in, H, M, x);
    float dv[MT][2], ov[MT][2];
    // o_proj's hand-off completes long before down_proj's: it is taken first, while down_proj
    // still runs (taken second, it would add a poll round trip after the last hand-off). The
    // wait for it spans this layer's attention: gated on one pair per MLP group (the first two
    // rows of group w, written by its wavefronts 0 and 1, in the last sequence row).
    const uint32_t need = (lane < a.mlp_groups ? 1u : 0u) | (lane + kWave < a.mlp_groups ? 2u : 0u);
    const int off0 = ((M - 1) * H + 8 * lane) * 8;  // bytes; the next sentinel 64 groups on
    bool ok = gate<2>(replica(a.ex1, s1), need, tag, a,
                      [=](int k) { return off0 + k * (8 * kWave * 8); }, flags);
    ok = ok && take<MT>(
        replica(a.ex1, s1), k0 < H ? low_bits(M) : 0u, tag, a,
        [&](int r) { return (r * H + k0) * 8; },
        [&](int r, float v0, float v1) {
          ov[r][0] = v0;
          ov[r][1] = v1;
        });
    ok = ok && take<MT>(
        replica(a.ex3, s1), k0 < H ? low_bits(M) : 0u, tag, a,
        [&](int r) { return (r * H + k0) * 8; },
        [&](int r, float v0, float v1) {
          dv[r][0] = v0;
          dv[r][1] = v1;
        });
    if (block_any(!ok, flags)) return finish(a);
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      x.v[r][0] = (x.v[r][0] + ov[r][0]) + dv[r][0];
      x.v[r][1] = (x.v[r][1] + ov[r][1]) + dv[r][1];
    }
  }
  // 3. the next layer's input norm times qkv's inv -> LDS, then the head's 128 rows
  norm_to_lds(x, next_w, qkv_inv, a.qkv_inv != nullptr, a.eps, H, M, xs, cs, red);
  __syncthreads();
#pragma unroll
  for (int p = 0; p < kHeadPasses; ++p) {
    float v[MT];
    chunk_terms<MT>(fq[p], hl, xs, cs, H, v);
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      const float t = lsh::group_total<32>(v[r]);
      if (hl == 31) out[(16 * wave + 2 * p + half) * MT + r] = t;
    }
  }
  __syncthreads();

  // 4. one wavefront per sequence: q/k norm + RoPE at position ctx - 1 (norm_rope's
  //    arithmetic on the prefetched rows), then q out or the int8 cache write (the quantizer
  //    of llmserve_kv_quantize_write)
  if (m < M) {
    float v[2];
    v[0] = out[lane * MT + m];
    v[1] = out[(lane + kWave) * MT + m];
    if (pos >= 0) {
      if (is_q || is_k) {
        if (nwp) {
          const float ss = lsh::wave_sum_from<1>(v[0] * v[0] + v[1] * v[1]);
          const float inv = 1.f / sqrtf(ss / static_cast<float>(D) + a.eps);
          v[0] = nw[0] * (v[0] * inv);
          v[1] = nw[1] * (v[1] * inv);
        }
        // rotate_half: element d < D/2 pairs with d + D/2, the other register of the lane
        const float r0 = v[0] * cosv[0] - v[1] * sn[0];
        const float r1 = v[1] * cosv[1] + v[0] * sn[1];
        v[0] = r0;
        v[1] = r1;
      }
      if (is_q) {
        float* o = a.q_out + (static_cast<int64_t>(m) * a.nq + hh) * D;
        o[lane] = v[0];
        o[lane + kWave] = v[1];
      } else if (slot >= 0) {
        const int64_t at = slot * a.nk + kvh;
        if (is_k) {
          float u[2] = {v[0], v[1]};
          lsh::kv_quant_row_smoothed(u, sm, a.smooth != nullptr, a.kc + at * D, a.ks + at);
        } else {
          float u[2] = {v[0], v[1]};
          lsh::kv_quant_row_smoothed(u, sm, false, a.vc + at * D, a.vs + at);
        }
      }
    } else if (is_q) {  // a position outside the tables: a NaN q, visible in the logits
      float* o = a.q_out + (static_cast<int64_t>(m) * a.nq + hh) * D;
      o[lane] = __builtin_nanf("");
      o[lane + kWave] = __builtin_nanf("");
    }
  }
  {  // this group's share of the new residual channels, stored last: a later wait on loads
     // (vmcnt counts stores too) would otherwise also wait for this store
    const int share = H / a.head_groups;
    store_rows(x, a.x_out, H, M, hh * share, (hh + 1) * share);
  }
  finish(a);
}

template <int MT>
__global__ __launch_bounds__(kThreads) void decode_chain_kernel(ChainArgs a) {
  // staged rows ([MT][K] floats, K up to kMaxI) and a stage's row results
  __shared__ __align__(16) float xs[MT * kMaxI];
  __shared__ float cs[MT * kMaxI / 32];  // the staged rows' 32-channel chunk sums
  __shared__ __align__(16) float rows[kHeadDim * MT];
  __shared__ float red[kWaves];
  __shared__ int flags[kWaves];
  if (a.mlp_groups > 0) {
    // this layer's attention first (before any workgroup requests its weights): its ranges,
    // then the merges of the last workgroups. The tag is read with the contexts, its round
    // trip overlapping theirs.
    const uint32_t tag = launch_tag(a);
    const AttnPlan pl = attn_plan(a);
    attention_range(a, pl, tag);
    if (block_any(!merge_attention(a, pl, tag, xs, flags), flags)) return finish(a);
  }
  if (static_cast<int>(blockIdx.x) < a.mlp_groups)
    mlp_group<MT>(a, xs, cs, rows, red, flags);
  else
    head_group<MT>(a, xs, cs, rows, red, flags);
}

template <int MT>
int launch_chain(const ChainArgs& a, int grid, hipStream_t st) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, decode_chain_kernel<MT>, kThreads, 0) !=
          hipSuccess) {
    lsh::set_error("decode_chain: device query failed");
    return LLMSERVE_ERR_HIP;
  }
  // every workgroup must be resident at once (they wait for each other)
  LSH_CHECK(static_cast<int64_t>(cus) * per >= grid,
            "decode_chain: %d workgroups do not fit at once (%d CUs x %d)", grid, cus, per);
  lsh::launch(decode_chain_kernel<MT>, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st,
              true, a);
  return lsh::launch_status("decode_chain");
}

}  // namespace

// Workspace words: control, the three linear hand-offs (kCopies replicas each), the merged
// attention rows (kCopies replicas) and the attention partials.

extern "C" int64_t llmserve_decode_chain_workspace_bytes(int64_t H, int64_t I) {
  if (H <= 0 || I <= 0) return 0;
  return 256 + (static_cast<int64_t>(kCopies) * kMaxRows * (2 * H + I) + kExbWords + kExaWords) * 8;
}

extern "C" int llmserve_decode_chain(
    const float* q_in, const int8_t* attn_k_cache, const int8_t* attn_v_cache,
    const float* attn_k_scale, const float* attn_v_scale, const float* q_mult, float scale,
    const float* x_in, const int64_t* ids, const float* embed, int64_t vocab,
    float* x_out, float* h_out, const uint8_t* o_nib, const float* o_s, const float* o_z,
    const float* o_inv, const float* post_w, const uint8_t* gu_nib, const float* gu_s,
    const float* gu_z, const float* gu_inv, const uint8_t* dn_nib, const float* dn_s,
    const float* dn_z, const float* dn_inv, const float* next_w, const uint8_t* qkv_nib,
    const float* qkv_s, const float* qkv_z, const float* qkv_inv, const float* q_w,
    const float* k_w, const float* cos_t, const float* sin_t, int64_t max_pos,
    const int64_t* context_lens, const int64_t* block_tables, int64_t max_blocks,
    int64_t block_size, const float* k_smooth, float* q_out, int8_t* k_cache, int8_t* v_cache,
    float* k_scale, float* v_scale, int64_t num_slots, int64_t M, int64_t H, int64_t I,
    int64_t n_q, int64_t n_k, int64_t head_dim, int64_t group_size, float eps, void* workspace,
    int64_t workspace_bytes, int64_t spin_limit, void* stream) {
  const bool mlp = q_in != nullptr, next = qkv_nib != nullptr;
  LSH_CHECK(M >= 1 && M <= kMaxRows, "decode_chain: 1 to %d rows (got %lld)", kMaxRows, (long long)M);
  LSH_CHECK(head_dim == kHeadDim && group_size == kGroup,
            "decode_chain: head_dim and group_size must be 128 (got %lld, %lld)",
            (long long)head_dim, (long long)group_size);
  LSH_CHECK(H >= 256 && H <= kMaxH && H % 128 == 0, "decode_chain: hidden size %lld not in "
            "{256, 384, ..., 1024}", (long long)H);
  LSH_CHECK(n_q >= 1 && n_k >= 1 && n_q % n_k == 0, "decode_chain: bad head counts");
  LSH_CHECK(H % (2 * (n_q + 2 * n_k)) == 0,
            "decode_chain: H must split evenly over the n_q + 2 n_k head groups");
  const int64_t Kq = n_q * head_dim;
  const int64_t mlp_groups = mlp ? H / 8 : 0;
  LSH_CHECK(mlp || next, "decode_chain: nothing to do (no attention input and no qkv)");
  if (mlp) {
    LSH_CHECK(Kq <= kMaxKq && Kq % 128 == 0, "decode_chain: n_q * head_dim = %lld above %d",
              (long long)Kq, kMaxKq);
    LSH_CHECK(I % kThreads == 0 && I <= kMaxI && I % mlp_groups == 0,
              "decode_chain: intermediate size %lld must be a multiple of %d and of H / 8, "
              "at most %d", (long long)I, kThreads, kMaxI);
    const int64_t C = I / mlp_groups;
    LSH_CHECK(C % kWaves == 0 && 2 * C <= 2 * kWaves * kMaxGuPass,
              "decode_chain: %lld gate channels per workgroup (need a multiple of %d, <= %d)",
              (long long)C, kWaves, kWaves * kMaxGuPass);
    LSH_CHECK(x_in && o_nib && o_s && o_z && post_w && gu_nib && gu_s && gu_z && dn_nib && dn_s &&
                  dn_z && next_w,
              "decode_chain: null MLP pointer");
    // this layer's attention: a wavefront per kv head, kGqa query heads each, steps of 8 slot
    // rows inside one block, 32-bit offsets into the caches, a merge workgroup per query head
    LSH_CHECK(attn_k_cache && attn_v_cache && attn_k_scale && attn_v_scale && context_lens &&
                  block_tables,
              "decode_chain: null attention pointer");
    LSH_CHECK(n_q == kGqa * n_k && n_k <= kWaves,
              "decode_chain: the fused attention needs n_q = %d n_k and n_k <= %d (got %lld, %lld)",
              kGqa, kWaves, (long long)n_q, (long long)n_k);
    LSH_CHECK(block_size >= 8 && (block_size & (block_size - 1)) == 0,
              "decode_chain: block_size %lld must be a power of two >= 8", (long long)block_size);
    LSH_CHECK(max_blocks >= 1 && max_blocks * block_size < (int64_t{1} << 31),
              "decode_chain: block tables of %lld x %lld tokens", (long long)max_blocks,
              (long long)block_size);
    LSH_CHECK(num_slots >= block_size && num_slots * n_k * head_dim < (int64_t{1} << 32),
              "decode_chain: KV cache of %lld slots not addressable with 32-bit offsets",
              (long long)num_slots);
    LSH_CHECK(M * n_q <= mlp_groups + (next ? n_q + 2 * n_k : 0),
              "decode_chain: %lld attention merges do not fit the grid", (long long)(M * n_q));
    LSH_CHECK(std::isfinite(scale) && scale > 0.f, "decode_chain: bad softmax scale");
  } else {
    LSH_CHECK(ids && embed && vocab > 0, "decode_chain: the embedding mode needs ids and embed");
  }
  if (next) {
    LSH_CHECK(qkv_s && qkv_z && next_w && cos_t && sin_t && context_lens && block_tables &&
                  q_out && k_cache && v_cache && k_scale && v_scale,
              "decode_chain: null qkv pointer");
    LSH_CHECK(max_blocks >= 1 && block_size >= 1 && max_pos >= 1, "decode_chain: empty tables");
  } else {
    LSH_CHECK(mlp, "decode_chain: the last layer needs the MLP part");
  }
  LSH_CHECK(x_out != nullptr, "decode_chain: null x_out");
  LSH_CHECK(workspace && lsh::aligned16(workspace) &&
                workspace_bytes >= llmserve_decode_chain_workspace_bytes(H, I),
            "decode_chain: workspace of %lld bytes needed",
            (long long)llmserve_decode_chain_workspace_bytes(H, I));
  auto al = [](const void* p) { return p == nullptr || lsh::aligned16(p); };
  LSH_CHECK(al(q_in) && al(q_mult) && al(attn_k_cache) && al(attn_v_cache) && al(x_in) && al(embed) && al(o_nib) && al(gu_nib) && al(dn_nib) &&
                al(qkv_nib) && al(o_inv) && al(gu_inv) && al(dn_inv) && al(qkv_inv) &&
                al(post_w) && al(next_w),
            "decode_chain: weights, activations and norm weights must be 16-byte aligned");

  ChainArgs a{};
  a.q_in = q_in;
  a.akc = attn_k_cache;
  a.avc = attn_v_cache;
  a.aks = attn_k_scale;
  a.avs = attn_v_scale;
  a.q_mult = q_mult;
  a.qscale = scale * kLog2e;
  a.bs_shift = 0;
  while ((int64_t{1} << a.bs_shift) < block_size) ++a.bs_shift;
  a.x_in = x_in;
  a.ids = ids;
  a.embed = embed;
  a.vocab = vocab;
  a.x_out = x_out;
  a.h_out = h_out;
  a.o_nib = o_nib;
  a.o_s = o_s;
  a.o_z = o_z;
  a.o_inv = o_inv;
  a.post_w = post_w;
  a.gu_nib = gu_nib;
  a.gu_s = gu_s;
  a.gu_z = gu_z;
  a.gu_inv = gu_inv;
  a.dn_nib = dn_nib;
  a.dn_s = dn_s;
  a.dn_z = dn_z;
  a.dn_inv = dn_inv;
  a.next_w = next_w;
  a.qkv_nib = qkv_nib;
  a.qkv_s = qkv_s;
  a.qkv_z = qkv_z;
  a.qkv_inv = qkv_inv;
  a.q_w = q_w;
  a.k_w = k_w;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.max_pos = max_pos;
  a.ctx = context_lens;
  a.bt = block_tables;
  a.max_blocks = max_blocks;
  a.bs = block_size;
  a.num_slots = num_slots;
  a.smooth = k_smooth;
  a.q_out = q_out;
  a.kc = k_cache;
  a.vc = v_cache;
  a.ks = k_scale;
  a.vs = v_scale;
  char* ws = static_cast<char*>(workspace);
  a.ctl = reinterpret_cast<uint32_t*>(ws);
  a.ex1 = reinterpret_cast<uint64_t*>(ws + 256);  // kCopies replicas of each
  a.ex2 = a.ex1 + static_cast<int64_t>(kCopies) * kMaxRows * H;
  a.ex3 = a.ex2 + static_cast<int64_t>(kCopies) * kMaxRows * I;
  a.exb = a.ex3 + static_cast<int64_t>(kCopies) * kMaxRows * H;
  a.exa = a.exb + kExbWords;
  a.spin_limit = static_cast<uint32_t>(spin_limit < 0 ? 0 : (spin_limit > 0x7fffffff ? 0x7fffffff : spin_limit));
  a.M = static_cast<int>(M);
  a.H = static_cast<int>(H);
  a.Kq = static_cast<int>(Kq);
  a.I = static_cast<int>(I);
  a.nq = static_cast<int>(n_q);
  a.nk = static_cast<int>(n_k);
  a.mlp_groups = static_cast<int>(mlp_groups);
  a.head_groups = next ? static_cast<int>(n_q + 2 * n_k) : 0;
  a.eps = eps;
  a.grid = a.mlp_groups + a.head_groups;
  const int grid = a.grid;
  hipStream_t st = lsh::as_stream(stream);
  switch (M) {
    case 1: return launch_chain<1>(a, grid, st);
    case 2: return launch_chain<2>(a, grid, st);
    default: return launch_chain<4>(a, grid, st);
  }
}

// The error word of a chain workspace (1 when a hand-off wait ran out of polls since the
// workspace was cleared). Synchronizes with the device.
extern "C" int llmserve_decode_chain_error(const void* workspace, int* error) {
  LSH_CHECK(workspace && error, "decode_chain_error: null pointer");
  uint32_t ctl[3] = {0, 0, 0};
  if (hipMemcpy(ctl, workspace, sizeof(ctl), hipMemcpyDeviceToHost) != hipSuccess) {
    lsh::set_error("decode_chain_error: hipMemcpy failed");
    return LLMSERVE_ERR_HIP;
  }
  *error = static_cast<int>(ctl[2]);
  return LLMSERVE_OK;
}
