// Prefill-sized weight-only int8 linear on the bf16 matrix cores:
//   y[m, n] = scale[n] * sum_k bf16(x[m, k]) * bf16(q[n, k])        (fp32 accumulate)
// The int8 weight converts to bf16 exactly (|q| <= 127); x is rounded to bf16 once (round to
// nearest even) by x_to_bf16 into the workspace. This is Int8Linear's large-M path
// (reference quant.py:71-72, dequantize :78-79: x @ (q * scale[:, None]).T) with the
// per-channel scale moved to the epilogue.
//
// Tiling: a 512-thread workgroup owns a 256 x 256 output tile (or, split-K, one K range of
// it); its eight wavefronts (two per SIMD, so one waits for LDS or a barrier while the other
// issues MFMAs) own 128 x 64 parts, each a grid of 8 x 4 v_mfma_f32_16x16x32_bf16 tiles (128
// fp32 accumulators per lane, in AGPRs). K advances 64 per stage:
// A = 256 rows x 64 bf16 of x, B = 256 rows x 64 weights widened int8 -> fp32 -> bf16 on the
// way into LDS. Two LDS buffers: the global loads of stage s + 1 are in flight (in registers)
// while the 128 MFMAs per wavefront of stage s run from LDS, then go to the other buffer.
// LDS rows are 128 bytes (eight 16-byte chunks); chunk c of row r sits at position
// c ^ (r & 7). Measured with SQ_LDS_BANK_CONFLICT on gfx950, the fragment loads (16 rows x
// 4 chunks per ds_read_b128) and both stage stores are then conflict-free; with a further
// ^ ((r >> 3) & 1) each fragment load costs 4 conflict cycles.
// MFMA operands (16x16x32 bf16): lane l supplies row l % 16 of the A tile and column l % 16
// of the B tile, k = 8 (l / 16) .. + 8; the result lane l holds rows 4 (l / 16) + r, column
// l % 16.
// Split-K: when the output has fewer tiles than the GPU has CUs, each tile's K range is split
// (into at most 4, each a multiple of 64) and every split writes fp32 partials that a second
// kernel sums in split order, applying scale[n] (deterministic, no atomics).
// Units map to blocks XCD-aware: block b runs on XCD b % 8, and each XCD gets whole columns
// of units (a tile column and its splits), so a weight panel is read from HBM into one XCD's
// L2 and reused there by every row tile of the column.
#include "common.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64;  // kBN: the widest tile (B rows per stage)
constexpr int kMaxSplits = 4;
constexpr int kThreads = 512;
constexpr int kXcds = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, n, 0x00020000);
}

// x fp32 -> bf16 (round to nearest even), 4 elements per thread per step.
__global__ __launch_bounds__(256) void x_to_bf16(const float* __restrict__ x, __bf16* __restrict__ xb,
                                                 int64_t n4) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    __bf16 o[4] = {static_cast<__bf16>(v.x), static_cast<__bf16>(v.y), static_cast<__bf16>(v.z),
                   static_cast<__bf16>(v.w)};
    reinterpret_cast<uint2*>(xb)[i] = *reinterpret_cast<const uint2*>(o);
  }
}

__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ (row & 7);
}

// 16 int8 -> 16 bf16 (two 16-byte chunks), exact.
__device__ __forceinline__ void widen16(const u32x4& w, u32x4& lo, u32x4& hi) {
  __bf16 b[16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[4 * i + j] = static_cast<__bf16>(static_cast<float>(static_cast<int8_t>((w[i] >> (8 * j)) & 0xffu)));
  lo = *reinterpret_cast<const u32x4*>(&b[0]);
  hi = *reinterpret_cast<const u32x4*>(&b[8]);
}

struct GemmArgs {
  const __bf16* xb;     // [M, K] bf16
  const int8_t* q;      // [N, K]
  const float* scale;   // [N]
  float* y;             // [M, N]
  float* part;          // [splits, M, N] fp32 partials (splits > 1)
  int M, N, K;
  int tiles_m, tiles_n, splits, k_split;  // k_split = K per split (multiple of kBK)
};

// BN: output columns per tile, 256 or 192 (for outputs whose 256-wide tiles would leave CUs
// idle); a stage always stages kBN weight rows (rows past the tile are never read).
template <int BN>
__global__ __launch_bounds__(kThreads, 1) void int8_gemm_bf16(GemmArgs a) {
  constexpr int NJ = BN / 64;  // 16-column MFMA tiles per wavefront (4 wavefront columns)
  // [buf][row][8 chunks of 16 B]; A and B halves of one LDS stage
  __shared__ __attribute__((aligned(16))) char lds[2 * 2 * kBM * 128];
  constexpr int kBufBytes = 2 * kBM * 128;  // one stage: A (32 KB) then B (32 KB)
  constexpr int kBOff = kBM * 128;

  // XCD-aware unit order over "columns" (tile column, split): block b runs on XCD b % 8,
  // XCD x takes columns [x * cols / 8, (x + 1) * cols / 8) when cols is a multiple of 8.
  const int cols = a.tiles_n * a.splits;
  const int b = blockIdx.x;
  int tm, col;
  if (cols % kXcds == 0) {
    const int x = b % kXcds, idx = b / kXcds;
    tm = idx % a.tiles_m;
    col = x * (cols / kXcds) + idx / a.tiles_m;
  } else {
    tm = b % a.tiles_m;
    col = b / a.tiles_m;
  }
  const int tn = col / a.splits, split = col % a.splits;
  const int m0 = tm * kBM, n0 = tn * BN;
  const int kbeg = split * a.k_split;

  const int t = threadIdx.x;
  const int lane = t % 64, wave = t / 64;
  const int wm = wave / 4, wn = wave % 4;  // 128 x 16 NJ part of the tile
  const int K = a.K;

  // Global loads: a lane-constant byte offset, the stage's k (and the row block i) in the
  // scalar offset. A: rows t / 8 + 64 i, chunk t % 8; B: rows t / 4 + 128 i, 16 bytes t % 4.
  const auto ra = rsrc(a.xb, static_cast<int64_t>(a.M) * K * 2);
  const auto rb = rsrc(a.q, static_cast<int64_t>(a.N) * K);
  const int ga_off = ((m0 + t / 8) * K + 8 * (t % 8)) * 2;
  const int gb_off = (n0 + t / 4) * K + 16 * (t % 4);
  auto load_a = [&](u32x4 (&ga)[4], int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ga[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            ra, ga_off, (k0 + i * 64 * K) * 2, 0));
  };
  auto load_b = [&](u32x4 (&gb)[2], int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      gb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rb, gb_off, k0 + i * 128 * K, 0));
  };
  // LDS stores: the swizzle of rows t / 8 + 64 i (A) and t / 4 + 128 i (B) depends on t only.
  const int sa_off = (t / 8) * 128 + swz(t / 8, t % 8) * 16;
  const int sb_off0 = (t / 4) * 128 + swz(t / 4, 2 * (t % 4)) * 16;
  const int sb_off1 = (t / 4) * 128 + swz(t / 4, 2 * (t % 4) + 1) * 16;
  auto store_stage = [&](const u32x4 (&ga)[4], const u32x4 (&gb)[2], int buf) {
    char* base = lds + buf * kBufBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(base + sa_off + i * 64 * 128) = ga[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      u32x4 lo, hi;
      widen16(gb[i], lo, hi);
      *reinterpret_cast<u32x4*>(base + kBOff + sb_off0 + i * 128 * 128) = lo;
      *reinterpret_cast<u32x4*>(base + kBOff + sb_off1 + i * 128 * 128) = hi;
    }
  };

  f32x4 acc[8][NJ];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment reads: rows wm * 128 + 16 i + fr (A) and wn * 16 NJ + 16 j + fr (B); the swizzle
  // of such a row depends on fr only, so each substep has one lane offset per operand.
  const int fr = lane % 16, fc = lane / 16;
  int fa_off[kBK / 32], fb_off[kBK / 32];
#pragma unroll
  for (int sub = 0; sub < kBK / 32; ++sub) {
    fa_off[sub] = (wm * 128 + fr) * 128 + swz(fr, 4 * sub + fc) * 16;
    fb_off[sub] = kBOff + (wn * 16 * NJ + fr) * 128 + swz(fr, 4 * sub + fc) * 16;
  }
  auto compute = [&](int buf) {
    const char* base = lds + buf * kBufBytes;
#pragma unroll
    for (int sub = 0; sub < kBK / 32; ++sub) {
      bf16x8 fa[8], fb[NJ];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        fa[i] = *reinterpret_cast<const bf16x8*>(base + fa_off[sub] + i * 16 * 128);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fb[j] = *reinterpret_cast<const bf16x8*>(base + fb_off[sub] + j * 16 * 128);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

  // While stage s is computed from LDS, A of stage s + 1 and B (the weights, the loads that
  // miss in L2) of stage s + 2 are loaded into registers; then A of s + 1 and B of s + 1
  // (loaded one stage earlier; two B register sets used in turn) go to the other LDS buffer.
  // The loads are unconditional (past the end they reload stage n - 1, unused): a load under a
  // branch makes the waits count conservatively; vmcnt counts in issue order, so waiting for
  // A of s + 1 leaves B of s + 2 in flight. One barrier per stage.
  const int n = a.k_split / kBK;
  auto kofs = [&](int st) { return kbeg + (st < n ? st : n - 1) * kBK; };
  u32x4 ga[4], gb0[2], gb1[2];
  load_a(ga, kofs(0));
  load_b(gb0, kofs(0));
  load_b(gb1, kofs(1));
  store_stage(ga, gb0, 0);
  __syncthreads();
  auto step = [&](int kt, const u32x4 (&nxtb)[2], u32x4 (&farb)[2]) {
    load_a(ga, kofs(kt + 1));
    __builtin_amdgcn_sched_barrier(0);
    load_b(farb, kofs(kt + 2));
    __builtin_amdgcn_sched_barrier(0);
    compute(kt & 1);
    store_stage(ga, nxtb, (kt + 1) & 1);
    __syncthreads();
  };
  int kt = 0;
  for (; kt + 1 < n; kt += 2) {
    step(kt, gb1, gb0);
    step(kt + 1, gb0, gb1);
  }
  if (kt < n) step(kt, gb1, gb0);

  // epilogue: lane holds rows 4 (lane / 16) + r, column lane % 16 of each 16 x 16 tile
  float* dst = a.splits > 1 ? a.part + static_cast<int64_t>(split) * a.M * a.N : a.y;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int nn = n0 + wn * 16 * NJ + 16 * j + fr;
    if (nn >= a.N) continue;
    const float sc = a.splits > 1 ? 1.f : a.scale[nn];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 128 + 16 * i + 4 * fc + r;
        if (m < a.M) dst[static_cast<int64_t>(m) * a.N + nn] = acc[i][j][r] * sc;
      }
    }
  }
}

// y[m, n] = scale[n] * sum_s part[s, m, n], summed in split order.
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ part,
                                                     const float* __restrict__ scale,
                                                     float* __restrict__ y, int64_t MN, int N,
                                                     int splits) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < MN; i += stride) {
    float s = part[i];
    for (int k = 1; k < splits; ++k) s += part[k * MN + i];
    y[i] = s * scale[i % N];
  }
}

// K splits for an M x N x K problem: enough (tile, split) units to give every CU one, at most
// kMaxSplits, each split a multiple of kBK.
int device_cus() {
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
      cus = c;
  }
  return cus;
}

// Tile width: 192 when 256-wide tiles leave CUs idle and 192-wide ones fill between 3/4 and
// all of them (qkv at config 3: 192 -> 256 tiles), else 256.
int pick_bn(int64_t M, int64_t N) {
  const int64_t cus = device_cus(), tm = (M + kBM - 1) / kBM;
  const int64_t t256 = tm * ((N + 255) / 256), t192 = tm * ((N + 191) / 192);
  return (t256 < cus && 4 * t192 > 3 * cus && t192 <= cus) ? 192 : 256;
}

int prefill_splits(int64_t M, int64_t N, int64_t K) {
  const int cus = device_cus();
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + pick_bn(M, N) - 1) / pick_bn(M, N));
  int s = 1;
  while (s < kMaxSplits && tiles * s * 2 <= cus && K % (static_cast<int64_t>(2 * s) * kBK) == 0) s *= 2;
  return s;
}

}  // namespace

extern "C" int64_t llmserve_int8_linear_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t xb = (M * K * 2 + 255) / 256 * 256;  // bf16 copy of x
  const int s = prefill_splits(M, N, K);
  return xb + (s > 1 ? s * M * N * static_cast<int64_t>(sizeof(float)) : 0);
}

extern "C" int llmserve_int8_linear_prefill(const float* x, const int8_t* qweight,
                                            const float* scale, float* y, int64_t M, int64_t N,
                                            int64_t K, void* workspace, int64_t workspace_bytes,
                                            void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 0, "int8_linear_prefill: negative size");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(K > 0 && K % kBK == 0, "int8_linear_prefill: K (%lld) must be a positive multiple of %d",
            (long long)K, kBK);
  LSH_CHECK(x && qweight && scale && y, "int8_linear_prefill: null pointer");
  LSH_CHECK(lsh::aligned16(x) && lsh::aligned16(qweight),
            "int8_linear_prefill: x and qweight must be 16-byte aligned");
  // buffer offsets are 32-bit: the bf16 copy of x and the weight stay under 2 GiB
  LSH_CHECK((M + kBM) * K * 2 < (1LL << 31) && (N + kBN) * K < (1LL << 31),
            "int8_linear_prefill: x (bf16) or weight over 2 GiB");
  const int64_t need = llmserve_int8_linear_prefill_workspace_bytes(M, N, K);
  LSH_CHECK(workspace != nullptr && workspace_bytes >= need && lsh::aligned16(workspace),
            "int8_linear_prefill: 16-byte aligned workspace of %lld bytes needed, %lld given",
            (long long)need, (long long)workspace_bytes);
  hipStream_t st = lsh::as_stream(stream);
  __bf16* xb = static_cast<__bf16*>(workspace);
  const int64_t n4 = M * K / 4;
  const int64_t cgrid = (n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096;
  lsh::launch(x_to_bf16, dim3(static_cast<unsigned>(cgrid)), dim3(256), 0, st, false, x, xb, n4);
  const int splits = prefill_splits(M, N, K);
  GemmArgs a{};
  a.xb = xb;
  a.q = qweight;
  a.scale = scale;
  a.y = y;
  a.part = splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                 (M * K * 2 + 255) / 256 * 256)
                      : nullptr;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  const int bn = pick_bn(M, N);
  a.tiles_n = static_cast<int>((N + bn - 1) / bn);
  a.splits = splits;
  a.k_split = static_cast<int>(K / splits);
  const int64_t units = static_cast<int64_t>(a.tiles_m) * a.tiles_n * splits;
  LSH_CHECK(units < (1LL << 31), "int8_linear_prefill: too many tiles");
  if (bn == 192)
    lsh::launch(int8_gemm_bf16<192>, dim3(static_cast<unsigned>(units)), dim3(kThreads), 0, st,
                splits == 1, a);
  else
    lsh::launch(int8_gemm_bf16<256>, dim3(static_cast<unsigned>(units)), dim3(kThreads), 0, st,
                splits == 1, a);
  if (splits > 1) {
    const int64_t MN = M * N;
    const int64_t rgrid = (MN + 255) / 256 < 8192 ? (MN + 255) / 256 : 8192;
    lsh::launch(splitk_reduce, dim3(static_cast<unsigned>(rgrid)), dim3(256), 0, st, true,
                static_cast<const float*>(a.part), scale, y, MN, static_cast<int>(N), splits);
  }
  return lsh::launch_status("int8_linear_prefill");
}
