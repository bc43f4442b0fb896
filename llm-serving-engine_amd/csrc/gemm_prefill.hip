// Prefill-sized weight-only int8 linear on the bf16 matrix cores:
//   y[m, n] = scale[n] * sum_k bf16(x[m, k]) * bf16(q[n, k])        (fp32 accumulate)
// The int8 weight converts to bf16 exactly (|q| <= 127); x is rounded to bf16 once (round to
// nearest even) by x_to_bf16 into the workspace. This is Int8Linear's large-M path
// (reference quant.py:71-72, dequantize :78-79: x @ (q * scale[:, None]).T) with the
// per-channel scale moved to the epilogue.
//
// Tiling: a 256-thread workgroup owns a 256 x 256 output tile; its four wavefronts own
// 128 x 128 quadrants, each a grid of 8 x 8 v_mfma_f32_16x16x32_bf16 tiles (256 fp32
// accumulators per lane). K advances 32 at a time through two LDS stages (A: 256 rows x 32
// bf16 of x; B: 256 rows x 32 weights, widened int8 -> fp32 -> bf16 on the way into LDS):
// while the wavefronts run the 64 MFMAs of one stage, the next stage's global loads are in
// flight. LDS rows are 64 bytes (four 16-byte chunks); chunk c of row r sits at position
// c ^ ((r >> 1) & 3), so the 8 rows a ds_read_b128 quarter-wave touches hit distinct banks.
// MFMA operands (16x16x32 bf16): lane l supplies row l % 16 of the A tile and column l % 16
// of the B tile, k = 8 (l / 16) .. + 8; the result lane l holds rows 4 (l / 16) + r, column
// l % 16.
// Tiles map to blocks XCD-aware: block b runs on XCD b % 8, and each XCD gets whole columns of
// tiles, so a weight panel is read from HBM into one XCD's L2 and reused there by every row
// tile of the column.
#include "common.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kThreads = 256;
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

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

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
  int M, N, K;
  int tiles_m, tiles_n;
};

__global__ __launch_bounds__(kThreads, 1) void int8_gemm_bf16(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) u32x4 lds_a[2][kBM * 4];  // [stage][row * 4 + chunk]
  __shared__ __attribute__((aligned(16))) u32x4 lds_b[2][kBN * 4];

  // XCD-aware tile order: block b runs on XCD b % 8; XCD x takes tile columns
  // [x * tiles_n / 8, (x + 1) * tiles_n / 8) when tiles_n is a multiple of 8.
  const int b = blockIdx.x;
  int tm, tn;
  if (a.tiles_n % kXcds == 0) {
    const int x = b % kXcds, idx = b / kXcds;
    tm = idx % a.tiles_m;
    tn = x * (a.tiles_n / kXcds) + idx / a.tiles_m;
  } else {
    tm = b % a.tiles_m;
    tn = b / a.tiles_m;
  }
  const int m0 = tm * kBM, n0 = tn * kBN;

  const int t = threadIdx.x;
  const int lane = t % 64, wave = t / 64;
  const int wm = wave / 2, wn = wave % 2;  // 128 x 128 quadrant

  // global -> register loads of one K stage. A: thread t loads rows t / 4 + 64 i (i < 4),
  // chunk t % 4 (8 bf16). B: rows t / 2 + 128 i (i < 2), bytes 16 (t % 2) .. + 16.
  const int64_t K = a.K;
  const auto ra = rsrc(a.xb, static_cast<int64_t>(a.M) * K * 2);
  const auto rb = rsrc(a.q, static_cast<int64_t>(a.N) * K);
  u32x4 ga[4], gb[2];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = t / 4 + 64 * i;
      const int64_t off = ((m0 + row) * K + k0 + 8 * (t % 4)) * 2;  // bytes
      // rows past M read zeros (buffer bound); offsets past 2^31 cannot occur (checked on host)
      ga[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, static_cast<int>(off), 0, 0));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = t / 2 + 128 * i;
      const int64_t off = (n0 + row) * K + k0 + 16 * (t % 2);
      gb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, static_cast<int>(off), 0, 0));
    }
  };
  auto store_stage = [&](int s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = t / 4 + 64 * i;
      lds_a[s][row * 4 + swz(row, t % 4)] = ga[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = t / 2 + 128 * i;
      u32x4 lo, hi;
      widen16(gb[i], lo, hi);
      lds_b[s][row * 4 + swz(row, 2 * (t % 2))] = lo;
      lds_b[s][row * 4 + swz(row, 2 * (t % 2) + 1)] = hi;
    }
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kt_n = a.K / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  const int fr = lane % 16, fc = lane / 16;  // fragment row, k chunk
  for (int kt = 0; kt < kt_n; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < kt_n) load_stage((kt + 1) * kBK);
    bf16x8 fa[8], fb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ra_row = wm * 128 + 16 * i + fr;
      fa[i] = __builtin_bit_cast(bf16x8, lds_a[s][ra_row * 4 + swz(ra_row, fc)]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int rb_row = wn * 128 + 16 * j + fr;
      fb[j] = __builtin_bit_cast(bf16x8, lds_b[s][rb_row * 4 + swz(rb_row, fc)]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    if (kt + 1 < kt_n) store_stage(s ^ 1);
    __syncthreads();
  }

  // epilogue: y = acc * scale[n]; lane holds rows 4 (lane / 16) + r, column lane % 16
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = n0 + wn * 128 + 16 * j + fr;
    if (n >= a.N) continue;
    const float sc = a.scale[n];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 128 + 16 * i + 4 * fc + r;
        if (m < a.M) a.y[static_cast<int64_t>(m) * a.N + n] = acc[i][j][r] * sc;
      }
    }
  }
}

}  // namespace

extern "C" int64_t llmserve_int8_linear_prefill_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return M * K * 2;
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
  // buffer offsets are 32-bit: the bf16 copy of x and the weight must stay under 2 GiB
  LSH_CHECK((M + kBM) * K * 2 < (1LL << 31) && (N + kBN) * K < (1LL << 31),
            "int8_linear_prefill: x (bf16) or weight over 2 GiB");
  const int64_t need = llmserve_int8_linear_prefill_workspace_bytes(M, K);
  LSH_CHECK(workspace != nullptr && workspace_bytes >= need && lsh::aligned16(workspace),
            "int8_linear_prefill: 16-byte aligned workspace of %lld bytes needed, %lld given",
            (long long)need, (long long)workspace_bytes);
  hipStream_t st = lsh::as_stream(stream);
  __bf16* xb = static_cast<__bf16*>(workspace);
  const int64_t n4 = M * K / 4;
  const int64_t cgrid = (n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096;
  lsh::launch(x_to_bf16, dim3(static_cast<unsigned>(cgrid)), dim3(256), 0, st, false, x, xb, n4);
  GemmArgs a{};
  a.xb = xb;
  a.q = qweight;
  a.scale = scale;
  a.y = y;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  a.tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  const int64_t tiles = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
  LSH_CHECK(tiles < (1LL << 31), "int8_linear_prefill: too many tiles");
  lsh::launch(int8_gemm_bf16, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, st, true, a);
  return lsh::launch_status("int8_linear_prefill");
}
