// fp32 LM head of the decode step on activation fragments (replaces the tied-embedding
// lm_head of models/transformer.py:192-193, F.linear(h, embed.weight)):
//   y[m, v] = sum_k x[m, k] * W[v, k]      W fp32 [V, K] row-major (the embedding matrix)
// x arrives as the bf16 fragments of xfrag.h (x = xh + xm + xl to ~2^-26 relative); each W
// value is split the same way in registers (W = wh + wm + wl), and the six products whose
// weight is at least 2^-16 of wh*xh -- wh*xh, wh*xm, wm*xh, wh*xl, wl*xh, wm*xm -- go through
// v_mfma_f32_16x16x32_bf16 (each product of two bf16 values is exact in fp32) with fp32
// accumulation. What is left out (wm*xl, wl*xm, wl*xl and the ~2^-26 split residuals) is
// below 2^-23 of each product: every product is the fp32 product up to fp32's own rounding,
// as in the reference's fp32 F.linear.
//
// The kernel streams W once (622 MB at Qwen3-0.6B: HBM-bound). A workgroup of 8 wavefronts
// (about one per CU, looping over vocab tiles) owns 128 vocab rows at a time, 16 per
// wavefront, and up to 4 row tiles of x (64 rows, the B operand, straight from the fragment
// layout). Per block of 128 channels:
//   * x (8 KB per row tile) is staged in LDS for all wavefronts, double-buffered, one block
//     ahead;
//   * each lane loads its A operand directly, two blocks ahead (8 KB per wavefront): row
//     l % 16, channels 16 i + 4 (l / 16) .. + 4 for i = 0 .. 7, so that one load instruction
//     reads 64 contiguous bytes of each of 16 rows (16 cache lines; a lane-contiguous 128 bytes
//     per lane would touch 64 lines per instruction and stall the address unit);
//   * the products' k order is therefore permuted: step q's lane group g = l / 16 takes
//     channels 32 q + 4 g .. + 4 and 32 q + 16 + 4 g .. + 4, and x's fragments are rearranged
//     to match as they are staged (8-byte halves of the fragment pieces);
//   * 4 steps x 4 row tiles x 6 products = 96 MFMAs.
// The output lane holds vocab rows 4 (l / 16) .. + 4 of batch row l % 16: one 16-byte store.
#include "common.h"
#include "xfrag.h"

namespace {

using lsh::kWave;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;                 // wavefronts per workgroup
constexpr int kVRows = 16 * kWaves;       // vocab rows per workgroup
constexpr int kMaxTiles = 4;              // 16-row tiles of x per pass (64 rows)
constexpr int kXParts = lsh::kFragPieces;           // hi, mid, lo of x
constexpr int kTilePieces = 4 * kXParts * 64;  // 16-byte pieces of one (row tile, block)
constexpr int kBlkElems = 4 * lsh::kFragPieces * kWave * 8;  // bf16 of one (row tile, block)

struct LmArgs {
  const __bf16* xf;  // fragments of x [mp, K]
  const float* w;    // [V, K]
  float* y;          // [M, V]
  int M, V, K, nblk;
};

// W row chunk -> bf16 hi / mid / lo A operands of step q (8 channels; W = hi + mid + lo to
// ~2^-26).
__device__ __forceinline__ void split_w(const u32x4& p0, const u32x4& p1, bf16x8& hi, bf16x8& mid,
                                        bf16x8& lo) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t u = e < 4 ? p0[e] : p1[e - 4];
    v[e] = __builtin_bit_cast(float, u);
  }
  uint32_t h[4], m[4], l[4];
  lsh::split3_words<8>(v, h, m, l);  // two channels per packed conversion
  hi = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
  mid = __builtin_bit_cast(bf16x8, u32x4{m[0], m[1], m[2], m[3]});
  lo = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
}

// T: row tiles of this pass (blockIdx.y selects which). Workgroup g runs the vocab tiles
// g, g + gridDim.x, ... as one stream of (tile, block) steps, so the loads ahead run across
// tile boundaries; a tile's logits are stored after its last block.
template <int T>
__global__ __launch_bounds__(kWaves * kWave) void lm_head_f32_kernel(LmArgs a) {
  __shared__ u32x4 xs[2][T * kTilePieces];
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int tile0 = blockIdx.y * kMaxTiles;
  const int ntiles = (a.V + kVRows - 1) / kVRows;
  const int mine = (ntiles - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) /
                   static_cast<int>(gridDim.x);  // >= 1: the host launches at most ntiles
  const int nsteps = mine * a.nblk;
  const int lastw = nsteps - 1;
  const u32x4* xg = reinterpret_cast<const u32x4*>(a.xf);

  // W rows of step s: vocab tile blockIdx.x + (s / nblk) gridDim.x, block s % nblk
  auto vtile = [&](int s) { return static_cast<int>(blockIdx.x) + (s / a.nblk) * static_cast<int>(gridDim.x); };

  // x staging: 16-byte piece p = tid + 512 i of the hi, mid and lo parts of the T (row tile,
  // block) fragments; within one, piece (3 q + h) * 64 + lane comes from step q, part h
  // (lane = fr + 16 fc: row fr, channels 32 fc + 8 q .. + 8)
  constexpr int kPieces = T * kTilePieces;
  constexpr int kPer = (kPieces + kWaves * kWave - 1) / (kWaves * kWave);
  auto load_x = [&](int b, u32x4 (&r)[kPer]) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int p = tid + i * kWaves * kWave;
      if (kPieces % (kWaves * kWave) != 0 && p >= kPieces) continue;  // last round's tail
      const int t = p / kTilePieces, within = p % kTilePieces;
      const int qh = within / kWave, l = within % kWave;  // qh = 3 q + h
      r[i] = xg[((static_cast<int64_t>(tile0 + t) * a.nblk + b) * 4 + qh / kXParts) *
                    (lsh::kFragPieces * kWave) + (qh % kXParts) * kWave + l];
    }
  };
  // Staged in the products' k order: source piece (step q', part h, lane fr + 16 fc) holds
  // channels 32 fc + 8 q' + 4 hf .. + 4 in its half hf; they belong to step fc, lane group
  // g = 2 (q' & 1) + hf, in the low half of that piece when q' < 2, else the high half.
  auto store_x = [&](int buf, const u32x4 (&r)[kPer]) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int p = tid + i * kWaves * kWave;
      if (kPieces % (kWaves * kWave) != 0 && p >= kPieces) continue;
      const int t = p / kTilePieces, within = p % kTilePieces;
      const int qh = within / kWave, l = within % kWave;
      const int qs = qh / kXParts, h = qh % kXParts, fr = l % 16, fc = l / 16;
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int g = 2 * (qs & 1) + hf;
        u32x2* d = reinterpret_cast<u32x2*>(&xs[buf][t * kTilePieces + (kXParts * fc + h) * kWave + fr + 16 * g]);
        d[qs >> 1] = u32x2{r[i][2 * hf], r[i][2 * hf + 1]};
      }
    }
  };
  // a lane's W channels 16 i + 4 (lane / 16) .. + 4 (i = 0 .. 7) of its row in the block
  auto load_w = [&](int s, u32x4 (&r)[8]) {
    const int v = vtile(s) * kVRows + wave * 16 + lane % 16;
    const int vr = v < a.V ? v : a.V - 1;  // loads stay in bounds
    const u32x4* p = reinterpret_cast<const u32x4*>(a.w + static_cast<int64_t>(vr) * a.K +
                                                    (s % a.nblk) * lsh::kFragBlk + 4 * (lane / 16));
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = p[4 * i];
  };

  f32x4 acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // lane: vocab rows 4 (lane / 16) .. + 4 of the wavefront's 16, batch row 16 t + lane % 16
  auto store_tile = [&](int s) {
    const int vo = vtile(s) * kVRows + wave * 16 + 4 * (lane / 16);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int m = 16 * (tile0 + t) + lane % 16;
      if (m < a.M) {
        float* yo = a.y + static_cast<int64_t>(m) * a.V + vo;
        if (vo + 3 < a.V && (a.V & 3) == 0) {
          *reinterpret_cast<f32x4*>(yo) = acc[t];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (vo + r < a.V) yo[r] = acc[t][r];
        }
      }
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // W runs two steps ahead in three register sets used in turn (a copy from one set to
  // another would wait for the loads); x runs one step ahead through the LDS buffers.
  u32x4 w0[8], w1[8], w2[8], xn[kPer];
  load_w(0, w0);
  load_x(0, xn);
  load_w(lastw < 1 ? lastw : 1, w1);
  store_x(0, xn);
  __syncthreads();
  auto step = [&](int s, const u32x4 (&wc)[8], u32x4 (&wn)[8]) {
    const int cur = s & 1;
    const int sx = s + 1 < lastw ? s + 1 : lastw;  // past the end: reload the last (unused)
    const int sw = s + 2 < lastw ? s + 2 : lastw;
    // The loads ahead go out before this step's products: x first, so that its LDS store
    // after the products waits for x (and the older W) only -- vmcnt counts in issue order --
    // and W of step s + 2 stays in flight over the barrier; the scheduling barriers keep
    // that order and keep the loads from sinking.
    load_x(sx % a.nblk, xn);
    __builtin_amdgcn_sched_barrier(0);
    load_w(sw, wn);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 wh, wm, wl;
      split_w(wc[2 * q], wc[2 * q + 1], wh, wm, wl);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const u32x4* xq = &xs[cur][t * kTilePieces + (q * kXParts) * kWave + lane];
        const bf16x8 xh = __builtin_bit_cast(bf16x8, xq[0]);
        const bf16x8 xm = __builtin_bit_cast(bf16x8, xq[kWave]);
        const bf16x8 xl = __builtin_bit_cast(bf16x8, xq[2 * kWave]);
        // smallest terms first: each is added to an accumulator of its own magnitude
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wm, xm, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl, xh, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, xl, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wm, xh, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, xm, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, xh, acc[t], 0, 0, 0);
      }
    }
    if (s % a.nblk == a.nblk - 1) store_tile(s);
    store_x(cur ^ 1, xn);  // every wavefront finished reading this buffer before the last barrier
    __syncthreads();
  };
  int s = 0;
  for (; s + 2 < nsteps; s += 3) {
    step(s, w0, w2);
    step(s + 1, w1, w0);
    step(s + 2, w2, w1);
  }
  if (s < nsteps) step(s, w0, w2);
  if (s + 1 < nsteps) step(s + 1, w1, w0);
}

// Resident workgroups of the kernel on the current device (cached per device).
template <int T>
int lm_resident() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, lm_head_f32_kernel<T>, kWaves * kWave, 0) !=
            hipSuccess || per < 1)
      per = 1;
    cached[dev] = cus * per;
  }
  return cached[dev];
}

template <int T>
void launch_lm(const LmArgs& a, int passes, bool last, hipStream_t st) {
  const int ntiles = (a.V + kVRows - 1) / kVRows;
  const int res = lm_resident<T>();
  const int g = ntiles < res ? ntiles : res;
  lsh::launch(lm_head_f32_kernel<T>, dim3(static_cast<unsigned>(g), static_cast<unsigned>(passes)),
              dim3(kWaves * kWave), 0, st, last, a);
}

// ---- the fp32 head at 1-4 rows: a plain fp32 GEMV --------------------------------------------
// At a decode batch of 1-4 rows the 622 MB matrix is read once for a few dot products per
// row: a GEMV, bound by HBM. Each wavefront takes kGvRows vocab rows at a time; lane l holds
// channels [16 NF l, 16 NF (l + 1)) ... as NF float4 chunks at stride 64 float4 (so a load
// instruction reads 1 KB of a row contiguously), multiplies them by the same channels of the
// M x rows (held in registers for the whole launch) and the row sums are reduced over the
// wavefront. All the loads of a group of rows go out before its first product; the rows of
// the next group are loaded while this group is reduced (two register sets). Exact fp32
// products and sums (up to the summation order).
constexpr int kGvWaves = 8;   // wavefronts per workgroup
constexpr int kGvRows = 4;    // vocab rows per wavefront and group

template <int M, int NF>
__global__ __launch_bounds__(kGvWaves * kWave) void lm_head_gemv_kernel(const float* __restrict__ x,
                                                                          const float* __restrict__ w,
                                                                          float* __restrict__ y, int V) {
  constexpr int K = NF * 4 * kWave;
  const int lane = threadIdx.x % kWave;
  const int gw = blockIdx.x * kGvWaves + static_cast<int>(threadIdx.x) / kWave;
  const int nw = gridDim.x * kGvWaves;
  f32x4 xv[M][NF];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int f = 0; f < NF; ++f)
      xv[m][f] = *reinterpret_cast<const f32x4*>(x + static_cast<int64_t>(m) * K + (f * kWave + lane) * 4);
  auto load = [&](int v0, f32x4 (&r)[kGvRows][NF]) {
#pragma unroll
    for (int i = 0; i < kGvRows; ++i) {
      const int v = v0 + i < V ? v0 + i : V - 1;  // in bounds; the sums of rows past V are dropped
      const f32x4* p = reinterpret_cast<const f32x4*>(w + static_cast<int64_t>(v) * K) + lane;
#pragma unroll
      for (int f = 0; f < NF; ++f) r[i][f] = __builtin_nontemporal_load(p + f * kWave);
    }
  };
  auto reduce_store = [&](int v0, const f32x4 (&r)[kGvRows][NF]) {
#pragma unroll
    for (int i = 0; i < kGvRows; ++i) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float d = 0.f;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const f32x4 a = r[i][f], b = xv[m][f];
          d += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
        }
        d = lsh::group_total<kWave>(d);
        if (lane == kWave - 1 && v0 + i < V) y[static_cast<int64_t>(m) * V + v0 + i] = d;
      }
    }
  };
  f32x4 r0[kGvRows][NF], r1[kGvRows][NF];
  int v = gw * kGvRows;
  const int step = nw * kGvRows;
  if (v >= V) return;
  load(v, r0);
  for (;;) {
    const int vn = v + step;
    if (vn < V) load(vn, r1);
    reduce_store(v, r0);
    if (vn >= V) break;
    v = vn;
    const int vm = v + step;
    if (vm < V) load(vm, r0);
    reduce_store(v, r1);
    if (vm >= V) break;
    v = vm;
  }
}

template <int M, int NF>
void launch_gemv_head(const float* x, const float* w, float* y, int V, hipStream_t st) {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, lm_head_gemv_kernel<M, NF>,
                                                     kGvWaves * kWave, 0) != hipSuccess || per < 1)
      per = 1;
    cached[dev] = cus * per;
  }
  const int groups = (V + kGvRows * kGvWaves - 1) / (kGvRows * kGvWaves);
  const int g = groups < cached[dev] ? groups : cached[dev];
  lsh::launch(lm_head_gemv_kernel<M, NF>, dim3(static_cast<unsigned>(g)), dim3(kGvWaves * kWave), 0,
              st, true, x, w, y, V);
}

template <int NF>
void gemv_head_rows(int64_t M, const float* x, const float* w, float* y, int V, hipStream_t st) {
  switch (M) {
    case 1: launch_gemv_head<1, NF>(x, w, y, V, st); break;
    case 2: launch_gemv_head<2, NF>(x, w, y, V, st); break;
    case 3: launch_gemv_head<3, NF>(x, w, y, V, st); break;
    default: launch_gemv_head<4, NF>(x, w, y, V, st); break;
  }
}

}  // namespace

extern "C" int llmserve_lm_head_f32_xfrag(const void* xfrag, const float* w, float* y, int64_t M,
                                          int64_t V, int64_t K, void* stream) {
  LSH_CHECK(M >= 0 && V >= 1 && K >= 1, "lm_head_f32_xfrag: bad shape");
  LSH_CHECK(K % lsh::kFragBlk == 0, "lm_head_f32_xfrag: K must be a multiple of 128");
  LSH_CHECK(M < (1LL << 24) && V < (1LL << 31) && V * K < (1LL << 40) && M * V < (1LL << 40),
            "lm_head_f32_xfrag: shape too large");
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(xfrag && w && y, "lm_head_f32_xfrag: null pointer");
  LSH_CHECK(lsh::aligned16(xfrag) && lsh::aligned16(w) && lsh::aligned16(y),
            "lm_head_f32_xfrag: xfrag, w and y must be 16-byte aligned");
  LmArgs a{static_cast<const __bf16*>(xfrag), w, y, static_cast<int>(M), static_cast<int>(V),
           static_cast<int>(K), static_cast<int>(K / lsh::kFragBlk)};
  const int64_t tiles = lsh::frag_rows(M) / 16;
  hipStream_t st = lsh::as_stream(stream);
  if (tiles >= kMaxTiles) {
    // full passes of 4 row tiles; a remainder of 1-3 tiles runs as one more launch
    const int full = static_cast<int>(tiles / kMaxTiles);
    const int rem = static_cast<int>(tiles % kMaxTiles);
    launch_lm<kMaxTiles>(a, full, rem == 0, st);
    if (rem > 0) {
      LmArgs r = a;
      const int64_t off_tiles = static_cast<int64_t>(full) * kMaxTiles;
      r.xf = a.xf + off_tiles * a.nblk * kBlkElems;
      r.y = a.y + off_tiles * 16 * V;
      r.M = static_cast<int>(M - off_tiles * 16);
      if (rem == 1) launch_lm<1>(r, 1, true, st);
      else if (rem == 2) launch_lm<2>(r, 1, true, st);
      else launch_lm<3>(r, 1, true, st);
    }
  } else if (tiles == 1) {
    launch_lm<1>(a, 1, true, st);
  } else if (tiles == 2) {
    launch_lm<2>(a, 1, true, st);
  } else {
    launch_lm<3>(a, 1, true, st);
  }
  return lsh::launch_status("lm_head_f32_xfrag");
}

// The fp32 LM head for a decode batch of 1-4 rows (the same product as llmserve_lm_head_f32_xfrag
// in exact fp32 arithmetic, on x itself).
extern "C" int llmserve_lm_head_f32(const float* x, const float* w, float* y, int64_t M,
                                    int64_t V, int64_t K, void* stream) {
  LSH_CHECK(M >= 0 && M <= 4, "lm_head_f32: 1 to 4 rows (got %lld)", (long long)M);
  LSH_CHECK(V >= 1 && V < (1LL << 31) && V * K < (1LL << 40), "lm_head_f32: bad V");
  LSH_CHECK(K == 256 || K == 512 || K == 1024,
            "lm_head_f32: K must be 256, 512 or 1024 (got %lld)", (long long)K);
  if (M == 0) return LLMSERVE_OK;
  LSH_CHECK(x && w && y, "lm_head_f32: null pointer");
  LSH_CHECK(lsh::aligned16(x) && lsh::aligned16(w), "lm_head_f32: x and w must be 16-byte aligned");
  hipStream_t st = lsh::as_stream(stream);
  const int Vi = static_cast<int>(V);
  switch (K) {
    case 256: gemv_head_rows<1>(M, x, w, y, Vi, st); break;
    case 512: gemv_head_rows<2>(M, x, w, y, Vi, st); break;
    default: gemv_head_rows<4>(M, x, w, y, Vi, st); break;
  }
  return lsh::launch_status("lm_head_f32");
}
