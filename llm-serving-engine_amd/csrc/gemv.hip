// Weight-only int8 / int4 GEMV for decode (M <= 64 activation rows; one launch covers all
// of them in tiles of up to 16 rows, grid.y = row tiles).
//
// Decode is bound by HBM and, at the Qwen3-0.6B layer sizes (1-6 MB per matrix), by the
// latency of one kernel: back-to-back launches of an empty kernel already take ~2.3 us on
// MI355X, and a kernel that only streams the 3 MB of gate_up nibbles takes no longer. What a
// GEMV adds on top is its dependent chain (weights -> dot products -> reduction -> store),
// so the kernels keep that chain short and the loads wide:
//  * every lane loads 16 weight bytes per load (global_load_dwordx4, non-temporal): 16 int8
//    or 32 int4 input channels, a "slice";
//  * LPR lanes (16, 32 or 64) cover LPR*16 bytes of one output row; a wavefront holds
//    RPW = 64/LPR row slots and each lane owns RPL rows (RPL*RPW rows per wavefront);
//  * the activations of the tile are staged once per workgroup in LDS with direct
//    global->LDS loads (global_load_lds_dwordx4: every load of the stage is in flight at once,
//    none passes through VGPRs); the int4 AWQ pre-scale x * inv_act_scale is applied in LDS
//    after they land. The 16-byte chunks of each slice are stored rotated by a function of
//    the slice index (chunk_pos), so that a wavefront reading the same chunk of consecutive
//    slices has no LDS bank conflict;
//  * a lane unpacks its RPL weight slices once and reuses each x value it reads from LDS
//    for RPL rows (register blocking for M > 2);
//  * the LPR partial sums of a row are reduced with DPP only (butterflies within 16-lane
//    rows, row broadcasts across them).
// The int4 path uses the reference's group decomposition
//   y = sum_g s * sum_{k in g} x q + (z - 8 s) * sum_{k in g} x     (int8_gemv.cpp:48-52)
// per 32-channel slice, which always lies inside one quantization group (group % 32 == 0).
// Shapes the fast path cannot tile go to a generic kernel with scalar loads.
#include <algorithm>

#include "common.h"

namespace {

using lsh::kWave;
constexpr int kMaxWaves = 4;                 // wavefronts per workgroup (at most)
constexpr int kTileRows = 16;                // activation rows per grid.y tile
constexpr int kLdsBudget = 80 * 1024;        // bytes of staged x per workgroup (2 per CU)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Kernel arguments. The kernels read their arguments with scalar loads, and every batch that
// a later field needs is another dependent round trip before the weight loads can go out; the
// fields that address the weights and their group scales (pointers, N, K, G, spg_log2) are the
// first 64 bytes, which the compiler fetches in one batch at entry.
struct GemvArgs {
  const float* x;      // [M, K]
  const float* inv;    // [K] int4 AWQ pre-scale, or null
  const uint8_t* w;    // int8 [N, K] or nibbles [N, K/2]
  const float* s;      // int8: scale [N]; int4: g_scale [N, G]
  const float* z;      // int4: g_zero [N, G]
  float* y;            // [M, N]
  int N, K;
  int G;               // int4: quantization groups per row
  int16_t M;           // activation rows (<= 64)
  int16_t spg_log2;    // int4: log2 of slices (32 channels) per group, -1 if not a power of 2
  // set by the host for the tiled kernel: group size, channels staged per chunk (a multiple
  // of the segment), number of chunks, wavefronts per workgroup
  int group, KC, nchunk, wpb;
};

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Eight nibbles (channels 2b: low nibble of byte b, 2b + 1: high nibble) to fp32: the two
// masked words, then one byte-select conversion (v_cvt_f32_ubyteN) per value. The empty asm
// hides the masks from the compiler, which would otherwise extract each nibble with a
// bit-field extract first (one more instruction per value); it emits nothing.
__device__ __forceinline__ void unpack_nibbles(uint32_t u, float* q) {
  uint32_t lo = u & 0x0f0f0f0fu, hi = (u >> 4) & 0x0f0f0f0fu;
  asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    q[2 * b] = static_cast<float>((lo >> (8 * b)) & 0xffu);
    q[2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xffu);
  }
}

__device__ __forceinline__ void unpack_int8(uint32_t u, float* q) {
#pragma unroll
  for (int b = 0; b < 4; ++b) q[b] = static_cast<float>(static_cast<int8_t>((u >> (8 * b)) & 0xffu));
}

// 16-byte LDS access at a float offset that is a multiple of 4 (the compiler cannot prove
// it from runtime row strides; without the hint it splits the access into ds_read2_b32).
__device__ __forceinline__ float4 lds_ld4(const float* p) {
  return *static_cast<const float4*>(__builtin_assume_aligned(p, 16));
}
__device__ __forceinline__ void lds_st4(float* p, float4 v) {
  *static_cast<float4*>(__builtin_assume_aligned(p, 16)) = v;
}

// Position of chunk c (16 bytes = 4 channels) of slice `sl` within the slice: the slices of
// one 256-byte LDS row (2 int4 slices of 8 chunks, 4 int8 slices of 4 chunks) share a
// rotation and consecutive rows rotate by one chunk, rot = sl / 2 (int4) or sl / 4 (int8).
// Measured with SQ_LDS_BANK_CONFLICT on gfx950: a wavefront reading chunk c of 32 or 64
// consecutive slices this way has no bank conflict; rotating every slice by one more chunk
// (sl + sl / 8, sl / 2 + sl / 8) costs 4 conflict cycles per ds_read_b128. The staging
// stores are conflict-free either way.
template <int CPC>
__device__ __forceinline__ int chunk_pos(int sl, int c) {
  const int rot = CPC == 8 ? sl >> 1 : sl >> 2;
  return (c + rot) & (CPC - 1);
}

// Stages channels [c0, c0 + width) of x rows 0..MT-1 (rows >= Mt repeat row Mt-1; their
// sums are never stored) with direct global->LDS loads and, when `inv` is given, multiplies
// them by inv (rounded as the reference's separate x * inv_act_scale). LDS row m starts at
// float m * kcf; slice sl of a row occupies floats [sl*CPL, (sl+1)*CPL) with its chunks
// placed by chunk_pos. Row MT holds inv. With XSUM (int4), the channel sum of every slice of
// every row, the (z - 8 s) term's factor, is written to xsum[m * kcf / CPL + sl], once per
// workgroup instead of once per weight row. Requires width <= kcf, width % 256 == 0 (a
// wavefront's 64 chunks never straddle two rows) and 16-byte aligned x / inv rows. Ends with
// a barrier.
template <int MT, int CPL, bool XSUM>
__device__ __forceinline__ void stage_x(float* xs, float* xsum, const float* __restrict__ x,
                                        const float* __restrict__ inv, int Mt, int K, int c0,
                                        int width, int kcf, int wpb) {
  constexpr int CPC = CPL / 4;             // chunks per slice
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int bd = wpb * kWave;
  const int wchunks = width / 4;           // chunks staged per row
  const int bpr = wchunks / kWave;         // wavefront loads per row
  const int nblk = (MT + (inv ? 1 : 0)) * bpr;
  for (int b = wave; b < nblk; b += wpb) {
    const int m = b / bpr;                 // wave-uniform row
    const int q0 = (b - m * bpr) * kWave;  // first chunk of this wavefront's 1 KB
    const int p = q0 + lane;
    const int sl = p / CPC, r = p % CPC;
    const int c = (r - chunk_pos<CPC>(sl, 0)) & (CPC - 1);
    const float* src = m < MT ? x + static_cast<int64_t>(min(m, Mt - 1)) * K : inv;
    __builtin_amdgcn_global_load_lds(
        src + c0 + (sl * CPC + c) * 4,
        (__attribute__((address_space(3))) void*)(xs + m * kcf + q0 * 4), 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0): the direct-to-LDS loads have landed
  __syncthreads();
  if (inv || XSUM) {
    const float* iv = xs + MT * kcf;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      for (int q = threadIdx.x; q < wchunks; q += bd) {  // whole wavefronts (wchunks % 64 == 0)
        float* px = xs + m * kcf + q * 4;
        float4 v = lds_ld4(px);
        if (inv) {
          const float4 t = lds_ld4(iv + q * 4);
          v.x = __fmul_rn(v.x, t.x);
          v.y = __fmul_rn(v.y, t.y);
          v.z = __fmul_rn(v.z, t.z);
          v.w = __fmul_rn(v.w, t.w);
          lds_st4(px, v);
        }
        if constexpr (XSUM) {  // the CPC consecutive lanes of a slice
          const float t = lsh::group_sum<CPC>((v.x + v.y) + (v.z + v.w));
          if (q % CPC == 0) xsum[m * (kcf / CPL) + q / CPC] = t;
        }
      }
    __syncthreads();
  }
}

// Rows 0..MT-1 of stage_x_regs: up to 4 chunks per thread in flight per round.
template <int MT, int CPL, bool INV>
__device__ __forceinline__ void stage_rows_regs(float* xs, const float* __restrict__ x,
                                                const float* __restrict__ inv, int Mt, int K,
                                                int c0, int wchunks, int kcf, int bd) {
  constexpr int CPC = CPL / 4;
  const int rounds = (wchunks + bd - 1) / bd;  // uniform: chunks per thread per row
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float* xr = x + static_cast<int64_t>(min(m, Mt - 1)) * K + c0;
    for (int r0 = 0; r0 < rounds; r0 += 4) {
      // the loads are unconditional (address clamped into the row) under a uniform
      // predicate; only the LDS stores depend on the lane
      float4 v[4], t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (r0 + u < rounds) {
          const int q = min(threadIdx.x + (r0 + u) * bd, wchunks - 1);
          v[u] = *reinterpret_cast<const float4*>(xr + q * 4);
          if (INV) t[u] = *reinterpret_cast<const float4*>(inv + c0 + q * 4);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = threadIdx.x + (r0 + u) * bd;
        if (r0 + u < rounds && q < wchunks) {
          if (INV) {
            v[u].x = __fmul_rn(v[u].x, t[u].x);
            v[u].y = __fmul_rn(v[u].y, t[u].y);
            v[u].z = __fmul_rn(v[u].z, t[u].z);
            v[u].w = __fmul_rn(v[u].w, t[u].w);
          }
          const int sl = q / CPC;
          lds_st4(xs + m * kcf + (sl * CPC + chunk_pos<CPC>(sl, q % CPC)) * 4, v[u]);
        }
      }
    }
  }
}

// Register-staged variant for small tiles (MT <= 2): each thread loads up to 4 chunks of a
// row at once, applies inv in registers and writes them rotated; one barrier. Same layout and
// requirements as stage_x.
template <int MT, int CPL>
__device__ __forceinline__ void stage_x_regs(float* xs, const float* __restrict__ x,
                                             const float* __restrict__ inv, int Mt, int K, int c0,
                                             int width, int kcf, int wpb) {
  if (inv)
    stage_rows_regs<MT, CPL, true>(xs, x, inv, Mt, K, c0, width / 4, kcf, wpb * kWave);
  else
    stage_rows_regs<MT, CPL, false>(xs, x, inv, Mt, K, c0, width / 4, kcf, wpb * kWave);
  __syncthreads();
}

// The fast GEMV. INT4 selects the nibble format. Requires: K a multiple of the segment
// (LPR slices), 16-byte aligned rows, and for int4 group % 32 == 0. blockDim.x is 64 * a.wpb
// with wpb a multiple of S (up to kMaxWaves wavefronts); blockIdx.y selects the tile of
// activation rows. The wpb / S row groups of a workgroup each have S wavefronts that split
// the row segments between them (segment j goes to wavefront j % S of the chunk); their
// partial sums meet in LDS and are added in a fixed order, so results do not depend on timing.
template <int MT, int LPR, int RPL, int S, bool INT4>
__global__ __launch_bounds__(kMaxWaves * kWave) void gemv_fast(GemvArgs a) {
  extern __shared__ float4 xs4[];
  float* xs = reinterpret_cast<float*>(xs4);  // [MT + 1][KC] x rows and the inv row
  constexpr int RPW = kWave / LPR;         // row slots per wavefront
  constexpr int CPL = INT4 ? 32 : 16;      // input channels per lane slice (16 bytes)
  constexpr int SEGK = LPR * CPL;          // input channels per row segment
  constexpr int CPC = CPL / 4;             // 16-byte chunks per slice
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int wpb = a.wpb;
  const int rg = wave / S, ks = wave % S;  // row group, segment split
  const int rs = lane / LPR, li = lane % LPR;
  const int row0 = (blockIdx.x * (wpb / S) + rg) * RPL * RPW + rs;  // row r: row0 + r * RPW
  const int m0 = blockIdx.y * kTileRows;
  const int Mt = min(a.M - m0, MT);
  const float* x = a.x + static_cast<int64_t>(m0) * a.K;
  const int RB = INT4 ? a.K / 2 : a.K;
  // weights (and, int4, the group scale / zero of the lane's slice) of segment j
  auto load_seg = [&](int j, u32x4 (&w)[RPL], float (&sc)[RPL], float (&zc)[RPL]) {
#pragma unroll
    for (int r = 0; r < RPL; ++r) {  // rows clamped, not predicated: a predicated
      // load makes the compiler wait for it at the branch join
      const int64_t row = min(row0 + r * RPW, a.N - 1);
      w[r] = load16(a.w + row * RB + j * LPR * 16 + li * 16);
    }
    if constexpr (INT4) {
      const int slice = j * LPR + li;
      const int g = a.spg_log2 >= 0 ? slice >> a.spg_log2 : slice / (a.K / CPL / a.G);
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int64_t row = min(row0 + r * RPW, a.N - 1);
        sc[r] = a.s[row * a.G + g];
        zc[r] = a.z[row * a.G + g];
      }
    }
  };
  // The host guarantees that every wavefront has a segment in the first chunk (S <= its
  // segment count), so the weight loads of segment ks go out before anything else.
  int j = ks;
  u32x4 w[RPL];
  float gs[RPL], gz[RPL];
  load_seg(j, w, gs, gz);
  const int nseg = a.K / SEGK;
  const int spc = a.KC / SEGK;             // segments per staged chunk
  const int nchunk = a.nchunk;
  float acc[RPL][MT];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  for (int c = 0; c < nchunk; ++c) {
    const int c0 = c * spc * SEGK;
    if (c) __syncthreads();
    if constexpr (MT <= 2)
      stage_x_regs<MT, CPL>(xs, x, INT4 ? a.inv : nullptr, Mt, a.K, c0, min(a.KC, a.K - c0),
                            a.KC, wpb);
    else
      stage_x<MT, CPL, false>(xs, nullptr, x, INT4 ? a.inv : nullptr, Mt, a.K, c0,
                              min(a.KC, a.K - c0), a.KC, wpb);
    const int nsc = min(spc, nseg - c * spc);
    for (int js = ks; js < nsc; js += S) {  // here j == c * spc + js
      const int nsn = min(spc, nseg - (c + 1) * spc);  // segments of the next chunk
      const int jn = js + S < nsc ? j + S : (c + 1 < nchunk && ks < nsn ? (c + 1) * spc + ks : -1);
      u32x4 wn[RPL];
      float gsn[RPL], gzn[RPL];
      if (jn >= 0) load_seg(jn, wn, gsn, gzn);
      float sc[RPL], zc[RPL];
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        sc[r] = gs[r];
        zc[r] = gz[r] - 8.f * gs[r];
      }
      const int sl = js * LPR + li;        // this lane's slice within the staged chunk
      const float* xp = xs + sl * CPL;
      float wf[RPL][CPL];
#pragma unroll
      for (int r = 0; r < RPL; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (INT4)
            unpack_nibbles(w[r][i], &wf[r][8 * i]);
          else
            unpack_int8(w[r][i], &wf[r][4 * i]);
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float xv[CPL];
#pragma unroll
        for (int i = 0; i < CPC; ++i) {
          const float4 v = lds_ld4(xp + m * a.KC + 4 * chunk_pos<CPC>(sl, i));
          xv[4 * i] = v.x;
          xv[4 * i + 1] = v.y;
          xv[4 * i + 2] = v.z;
          xv[4 * i + 3] = v.w;
        }
        if constexpr (INT4) {
          float xsum = 0.f;
#pragma unroll
          for (int i = 0; i < CPL; ++i) xsum += xv[i];
#pragma unroll
          for (int r = 0; r < RPL; ++r) {
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) d += xv[i] * wf[r][i];
            acc[r][m] += sc[r] * d + zc[r] * xsum;
          }
        } else {
#pragma unroll
          for (int r = 0; r < RPL; ++r) {
            float t = acc[r][m];
#pragma unroll
            for (int i = 0; i < CPL; ++i) t += xv[i] * wf[r][i];
            acc[r][m] = t;
          }
        }
      }
      if (jn >= 0) {
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
          w[r] = wn[r];
          gs[r] = gsn[r];
          gz[r] = gzn[r];
        }
      }
      j = jn;
    }
  }
  float* red = xs;  // S > 1: [wpb][RPL][RPW][MT] row sums of each wavefront
  if constexpr (S > 1) __syncthreads();  // every wavefront is done with the staged x
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int row = row0 + r * RPW;
    const float sr = (!INT4 && row < a.N) ? a.s[row] : 1.f;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = lsh::group_total<LPR>(acc[r][m]);
      if constexpr (S == 1) {
        if (li == LPR - 1 && m < Mt && row < a.N)
          a.y[static_cast<int64_t>(m0 + m) * a.N + row] = INT4 ? v : v * sr;
      } else {
        if (li == LPR - 1) red[((wave * RPL + r) * RPW + rs) * MT + m] = v;
      }
    }
  }
  if constexpr (S > 1) {
    __syncthreads();
    if (ks == 0 && li == LPR - 1) {
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int row = row0 + r * RPW;
        if (row >= a.N) continue;
        const float sr = INT4 ? 1.f : a.s[row];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float v = red[((wave * RPL + r) * RPW + rs) * MT + m];
#pragma unroll
          for (int k = 1; k < S; ++k) v += red[(((wave + k) * RPL + r) * RPW + rs) * MT + m];
          if (m < Mt) a.y[static_cast<int64_t>(m0 + m) * a.N + row] = INT4 ? v : v * sr;
        }
      }
    }
  }
}

// The decode (M <= 4) GEMV, straight-line: a lane issues the loads of all its NSEG segments
// (and their group scales / zeros) at entry, the workgroup stages all of x (rows of K <= 4096
// channels, at most four chunks per thread per row, times inv in registers), then each lane
// finishes its rows. No loop carries a dependence on memory, so the kernel's time is one
// weight round-trip plus the short tail of dot products, DPP reduction and store.
// Requires K <= kLatMaxK, K == nseg * LPR * CPL with nseg <= NSEG, blockDim.x == 64 * WPB.
constexpr int kLatMaxK = 4096;

// KS > 1: the row's K segments are split over KS wavefronts of the workgroup (wavefront
// w takes segments (w % KS) * NSEG .. + NSEG of the rows of group w / KS), and their row sums
// meet in LDS, added in wavefront order (deterministic): KS times the wavefronts, each with a
// KS-th of the dependent chain (down_proj, K = 3072: three segments per lane otherwise).
template <int MT, int LPR, int NSEG, int WPB, bool INT4, int KS = 1>
__global__ __launch_bounds__(WPB * kWave) void gemv_lat(GemvArgs a) {
  constexpr int RPL = 1;
  extern __shared__ float4 xs4[];          // [MT][K] floats, slices rotated by chunk_pos
  float* xs = reinterpret_cast<float*>(xs4);
  constexpr int RPW = kWave / LPR;
  constexpr int CPL = INT4 ? 32 : 16;
  constexpr int SEGK = LPR * CPL;
  constexpr int CPC = CPL / 4;
  constexpr int BD = WPB * kWave;
  constexpr int UMAX = (kLatMaxK / 4 + BD - 1) / BD;  // x chunks per thread per row, at most
  static_assert(WPB % KS == 0, "gemv_lat: whole row groups per workgroup");
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int rg = wave / KS, kw = wave % KS;  // row group, K part
  const int rs = lane / LPR, li = lane % LPR;
  const bool lead = li == LPR - 1;  // the lane that holds the row total
  const int row0 = (blockIdx.x * (WPB / KS) + rg) * RPL * RPW + rs;
  const int RB = INT4 ? a.K / 2 : a.K;
  const int nseg = a.K / SEGK;
  const int seg0 = kw * NSEG;  // this wavefront's first segment
  const int wchunks = a.K / 4, rounds = (wchunks + BD - 1) / BD;
  const bool has_inv = INT4 && a.inv != nullptr;

  // 1. x (and inv) chunks for the LDS stage, first: the stores below then wait for these
  //    loads only, not for the weights issued after them. Addresses are clamped into the row
  //    under a uniform predicate, so no load sits behind a divergent branch.
  float4 xv4[MT][UMAX], iv4[UMAX];
#pragma unroll
  for (int u = 0; u < UMAX; ++u)
    if (u < rounds) {
      const int q = min(static_cast<int>(threadIdx.x) + u * BD, wchunks - 1);
#pragma unroll
      for (int m = 0; m < MT; ++m)  // rows past M repeat row M-1; their sums are not stored
        xv4[m][u] = *reinterpret_cast<const float4*>(
            a.x + static_cast<int64_t>(min(m, a.M - 1)) * a.K + q * 4);
      if (has_inv) iv4[u] = *reinterpret_cast<const float4*>(a.inv + q * 4);
    }
  // 2. weights of all segments and their group scales / zeros. Loads are unconditional,
  //    with the row and segment clamped into the matrix (rows past N and segments past nseg
  //    are never stored or summed): a predicated load would make the compiler wait for it
  //    at the branch join.
  u32x4 w[NSEG][RPL];
  float gs[NSEG][RPL], gz[NSEG][RPL];
#pragma unroll
  for (int j = 0; j < NSEG; ++j)
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      const int64_t row = min(row0 + r * RPW, a.N - 1);
      w[j][r] = load16(a.w + row * RB + min(seg0 + j, nseg - 1) * LPR * 16 + li * 16);
    }
  if constexpr (INT4) {
#pragma unroll
    for (int j = 0; j < NSEG; ++j) {
      const int slice = (seg0 + j) * LPR + li;
      const int g = a.spg_log2 >= 0 ? slice >> a.spg_log2 : slice / (a.K / CPL / a.G);
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int64_t at = min(row0 + r * RPW, a.N - 1) * static_cast<int64_t>(a.G) +
                           min(g, a.G - 1);
        gs[j][r] = a.s[at];
        gz[j][r] = a.z[at];
      }
    }
  }
  // 3. x * inv into LDS (rotated slices) and, for int4, each slice's channel sum of x * inv
  //    per row (xsl [slice][MT]: the (z - 8 s) factor, the same for every weight row, summed
  //    once per workgroup: the 8 chunk sums of a slice sit in 8 consecutive lanes and meet
  //    with DPP), one barrier
  [[maybe_unused]] float* xsl = xs + MT * a.K;
#pragma unroll
  for (int u = 0; u < UMAX; ++u) {
    if (u >= rounds) continue;  // uniform
    const int q = threadIdx.x + u * BD;
    const bool on = q < wchunks;  // whole slices (K % 32 == 0): a slice's 8 lanes agree
    const int sl = q / CPC;
    float* dst = xs + (sl * CPC + chunk_pos<CPC>(sl, q % CPC)) * 4;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float4 v = xv4[m][u];
      if (has_inv) {
        v.x = __fmul_rn(v.x, iv4[u].x);
        v.y = __fmul_rn(v.y, iv4[u].y);
        v.z = __fmul_rn(v.z, iv4[u].z);
        v.w = __fmul_rn(v.w, iv4[u].w);
      }
      if (on) lds_st4(dst + m * a.K, v);
      if constexpr (INT4) {
        const float cs = lsh::group_sum<CPC>(on ? (v.x + v.y) + (v.z + v.w) : 0.f);
        if (on && q % CPC == 0) xsl[sl * MT + m] = cs;
      }
    }
  }
  __syncthreads();

  float acc[RPL][MT];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
#pragma unroll
  for (int j = 0; j < NSEG; ++j) {
    if (seg0 + j >= nseg) break;
    const int sl = (seg0 + j) * LPR + li;
    auto read_x = [&](int m, float (&xv)[CPL]) {
#pragma unroll
      for (int i = 0; i < CPC; ++i) {
        const float4 v = lds_ld4(xs + m * a.K + sl * CPL + 4 * chunk_pos<CPC>(sl, i));
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
      }
    };
    // One row: its x slice (and slice sum) is requested from LDS before the weights are
    // waited for (left to itself the compiler waits for the weights, widens them and only
    // then computes the LDS addresses and issues these reads, all after the slowest load):
    // config 2 at M = 1 783 -> 825 GB/s. At four rows the same for row 0 measured 574 -> 555.
    float xv0[CPL];
    [[maybe_unused]] float xsum0 = 0.f;
    if constexpr (MT == 1) {
      read_x(0, xv0);
      if constexpr (INT4) xsum0 = xsl[sl * MT];
      __builtin_amdgcn_sched_barrier(0);
    }
    float wf[RPL][CPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (INT4)
          unpack_nibbles(w[j][r][i], &wf[r][8 * i]);
        else
          unpack_int8(w[j][r][i], &wf[r][4 * i]);
      }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float xv[CPL];
      if constexpr (MT == 1) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) xv[i] = xv0[i];
      } else {
        read_x(m, xv);
      }
      if constexpr (INT4) {
        const float xsum = MT == 1 ? xsum0 : xsl[sl * MT + m];
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < CPL; ++i) d += xv[i] * wf[r][i];
          acc[r][m] += gs[j][r] * d + (gz[j][r] - 8.f * gs[j][r]) * xsum;
        }
      } else {
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
          float t = acc[r][m];
#pragma unroll
          for (int i = 0; i < CPL; ++i) t += xv[i] * wf[r][i];
          acc[r][m] = t;
        }
      }
    }
  }
  float tot[RPL][MT];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) tot[r][m] = lsh::group_total<LPR>(acc[r][m]);
  if constexpr (KS > 1) {
    // [row group][row slot][m][K part] after the staged x and slice sums
    float* red = xs + MT * (a.K + (INT4 ? a.K / 32 : 0));
    const int base = ((rg * RPW + rs) * MT) * KS;
    if (lead) {
#pragma unroll
      for (int m = 0; m < MT; ++m) red[base + m * KS + kw] = tot[0][m];
    }
    __syncthreads();
    if (kw != 0) return;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v = red[base + m * KS];
#pragma unroll
      for (int k = 1; k < KS; ++k) v += red[base + m * KS + k];
      tot[0][m] = v;
    }
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int row = row0 + r * RPW;
    const float sr = (!INT4 && row < a.N) ? a.s[row] : 1.f;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (lead && row < a.N && m < a.M)
        a.y[static_cast<int64_t>(m) * a.N + row] = INT4 ? tot[r][m] : tot[r][m] * sr;
    }
  }
}

// Any shape / alignment: one wavefront per output row, lanes stride over k with byte loads.
template <int MT, bool INT4>
__global__ __launch_bounds__(kMaxWaves * kWave) void gemv_generic(GemvArgs a) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kMaxWaves + threadIdx.x / kWave;
  if (row >= a.N) return;  // whole wave; no barriers in this kernel
  const int G = INT4 ? a.K / a.group : 1;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;
  for (int k = lane; k < a.K; k += kWave) {
    float wv, s = 1.f, c = 0.f;
    if constexpr (INT4) {
      const uint8_t b = a.w[static_cast<int64_t>(row) * (a.K / 2) + k / 2];
      wv = static_cast<float>((k & 1) ? (b >> 4) : (b & 0xf));
      const int g = k / a.group;
      s = a.s[static_cast<int64_t>(row) * G + g];
      c = a.z[static_cast<int64_t>(row) * G + g] - 8.f * s;
    } else {
      wv = static_cast<float>(reinterpret_cast<const int8_t*>(a.w)[static_cast<int64_t>(row) * a.K + k]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m < a.M) {
        float xv = a.x[static_cast<int64_t>(m) * a.K + k];
        if (INT4 && a.inv) xv = __fmul_rn(xv, a.inv[k]);
        acc[m] += INT4 ? s * (xv * wv) + c * xv : xv * wv;
      }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float v = lsh::wave_sum_from<1>(acc[m]);
    if (lane == 0 && m < a.M) a.y[static_cast<int64_t>(m) * a.N + row] = INT4 ? v : v * a.s[row];
  }
}

// ---------------------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------------------
struct Config {
  int lpr;  // lanes per row: 16, 32, 64 (0 = generic kernel)
  int rpl;  // rows per lane
  int s;    // wavefronts splitting a row group's segments
  int wpb;  // wavefronts per workgroup
  int kc;   // channels staged per chunk
  int lds;  // LDS budget of the launch
};

constexpr int kLdsBudgetLarge = 160 * 1024;  // MT >= 8: one workgroup per CU if need be

// LDS floats of the tiled kernel for a chunk of kc channels: MT x rows and the inv row.
int lds_floats(bool int4, int MT, int kc) { return (MT + (int4 ? 1 : 0)) * kc; }

int pick_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// Fast-path tiling for a (bits, MT, N, K, group) problem; lpr = 0 when it cannot tile.
//  * LPR: the widest whose segment divides the row and whose staged x fits the LDS budget;
//  * RPL = 2 (register blocking) while that leaves >= 1536 (M <= 2) / 1024 wavefronts;
//  * S: split the segments of a row over 2 or 4 wavefronts until there are >= 1024
//    wavefronts (4 per CU), when the row has the segments and a chunk holds S of them;
//  * workgroups of 4 wavefronts, fewer when that spreads the launch over more CUs.
Config choose(bool int4, int MT, int N, int K, int group, bool aligned) {
  Config c{0, 1, 1, kMaxWaves, 0, MT >= 8 ? kLdsBudgetLarge : kLdsBudget};
  if (!aligned || (int4 && group % 32 != 0)) return c;
  const int cpl = int4 ? 32 : 16;
  const int row_bytes = int4 ? K / 2 : K;
  int seg_bytes = 0;  // LDS bytes of one segment of staged x (+ the inv row)
  for (int lpr : {64, 32, 16}) {
    if (row_bytes % (lpr * 16) != 0) continue;
    seg_bytes = lds_floats(int4, MT, lpr * cpl) * 4;
    if (seg_bytes > c.lds) continue;
    c.lpr = lpr;
    break;
  }
  if (c.lpr == 0) return c;
  const int rpw = kWave / c.lpr, segk = c.lpr * cpl, nseg = K / segk;
  const int chunk_segs = std::min(nseg, c.lds / seg_bytes);
  const int groups1 = (N + rpw - 1) / rpw;
  c.rpl = groups1 / 2 >= (MT <= 2 ? 1536 : 1024) ? 2 : 1;
  const int groups = (N + rpw * c.rpl - 1) / (rpw * c.rpl);
  if (c.rpl == 1)
    while (c.s < 4 && groups * c.s < 1024 && nseg >= 2 * c.s && chunk_segs >= 2 * c.s) c.s *= 2;
  const int waves = groups * c.s;
  c.wpb = waves >= 4 * 256 ? 4 : waves >= 2 * 256 ? std::max(2, c.s) : c.s;
  if (c.wpb < c.s) c.wpb = c.s;
  c.kc = segk * chunk_segs;
  return c;
}

template <int MT, int LPR, int RPL, int S, bool INT4>
int launch_fast(GemvArgs a, const Config& c, hipStream_t st) {
  auto kernel = gemv_fast<MT, LPR, RPL, S, INT4>;
  constexpr int CPL = INT4 ? 32 : 16;
  const int nseg = a.K / (LPR * CPL), spc = c.kc / (LPR * CPL);
  a.KC = c.kc;
  a.nchunk = (nseg + spc - 1) / spc;
  a.wpb = c.wpb;
  if constexpr (INT4) {
    a.G = a.K / a.group;
    const int spg = a.group / CPL;
    a.spg_log2 = static_cast<int16_t>((spg & (spg - 1)) == 0 ? __builtin_ctz(spg) : -1);
  }
  const size_t lds = static_cast<size_t>(lds_floats(INT4, MT, c.kc)) * sizeof(float);
  if (lds > 64 * 1024) {  // beyond the default dynamic-LDS limit: raise it once per kernel
    static const hipError_t raised = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
        kLdsBudgetLarge);
    if (raised != hipSuccess) {
      lsh::set_error("gemv: cannot raise the LDS limit: %s", hipGetErrorString(raised));
      return LLMSERVE_ERR_HIP;
    }
  }
  const int rows_per_block = c.wpb / S * RPL * (kWave / LPR);
  const int tiles = (a.M + kTileRows - 1) / kTileRows;
  lsh::launch(kernel, dim3((a.N + rows_per_block - 1) / rows_per_block, tiles),
              dim3(c.wpb * kWave), lds, st, true, a);
  return LLMSERVE_OK;
}

template <int MT, int LPR, bool INT4>
int launch_lpr(const GemvArgs& a, const Config& c, hipStream_t st) {
  if (c.rpl == 2) return launch_fast<MT, LPR, 2, 1, INT4>(a, c, st);
  switch (c.s) {
    case 4: return launch_fast<MT, LPR, 1, 4, INT4>(a, c, st);
    case 2: return launch_fast<MT, LPR, 1, 2, INT4>(a, c, st);
    default: return launch_fast<MT, LPR, 1, 1, INT4>(a, c, st);
  }
}

template <int MT, bool INT4>
int launch_mt(const GemvArgs& a, const Config& c, hipStream_t st) {
  switch (c.lpr) {
    case 64: return launch_lpr<MT, 64, INT4>(a, c, st);
    case 32: return launch_lpr<MT, 32, INT4>(a, c, st);
    default: return launch_lpr<MT, 16, INT4>(a, c, st);
  }
}

// Scalar-load fallback: one launch per tile of 16 activation rows.
template <bool INT4>
void run_generic(const GemvArgs& a, hipStream_t st) {
  for (int m0 = 0; m0 < a.M; m0 += kTileRows) {
    GemvArgs t = a;
    t.M = static_cast<int16_t>(a.M - m0 < kTileRows ? a.M - m0 : kTileRows);
    t.x = a.x + static_cast<int64_t>(m0) * a.K;
    t.y = a.y + static_cast<int64_t>(m0) * a.N;
    const bool last = m0 + kTileRows >= a.M;
    const dim3 grid((a.N + kMaxWaves - 1) / kMaxWaves), block(kMaxWaves * kWave);
    switch (pick_mt(t.M)) {
      case 1: lsh::launch(gemv_generic<1, INT4>, grid, block, 0, st, last, t); break;
      case 2: lsh::launch(gemv_generic<2, INT4>, grid, block, 0, st, last, t); break;
      case 4: lsh::launch(gemv_generic<4, INT4>, grid, block, 0, st, last, t); break;
      case 8: lsh::launch(gemv_generic<8, INT4>, grid, block, 0, st, last, t); break;
      default: lsh::launch(gemv_generic<16, INT4>, grid, block, 0, st, last, t); break;
    }
  }
}

template <int MT, int LPR, int NSEG, bool INT4>
void launch_lat(const GemvArgs& a, int wpb, hipStream_t st) {
  constexpr int rpw = kWave / LPR;
  // staged x, and for int4 the channel sum of each 32-channel slice per row
  const size_t lds = static_cast<size_t>(MT) * (a.K + (INT4 ? a.K / 32 : 0)) * sizeof(float);
  const int rows_per_block = wpb * rpw;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block);
  constexpr int kSmallWpb = MT > 2 ? 4 : 2;  // MT > 2 always runs 4 wavefronts
  if (MT > 2 || wpb == 4)
    lsh::launch(gemv_lat<MT, LPR, NSEG, 4, INT4>, grid, dim3(4 * kWave), lds, st, true, a);
  else
    lsh::launch(gemv_lat<MT, LPR, NSEG, kSmallWpb, INT4>, grid, dim3(kSmallWpb * kWave), lds, st,
                true, a);
}

// K split over KS wavefronts (one segment each), two row groups per workgroup.
template <int MT, int LPR, int KS, bool INT4>
void launch_lat_split(const GemvArgs& a, hipStream_t st) {
  constexpr int rpw = kWave / LPR, WPB = 2 * KS;
  const size_t lds = (static_cast<size_t>(MT) * (a.K + (INT4 ? a.K / 32 : 0)) +
                      static_cast<size_t>(WPB / KS) * rpw * MT * KS) * sizeof(float);
  const int rows_per_block = (WPB / KS) * rpw;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block);
  lsh::launch(gemv_lat<MT, LPR, 1, WPB, INT4, KS>, grid, dim3(WPB * kWave), lds, st, true, a);
}

template <int MT, int LPR, bool INT4>
void launch_lat_lpr(const GemvArgs& a, int nseg, int wpb, hipStream_t st) {
  if constexpr (MT <= 4) {
    switch (nseg) {  // several segments per lane: split them over wavefronts instead
      case 2: return launch_lat_split<MT, LPR, 2, INT4>(a, st);
      case 3: return launch_lat_split<MT, LPR, 3, INT4>(a, st);
      case 4: return launch_lat_split<MT, LPR, 4, INT4>(a, st);
      default: break;
    }
  }
  switch (nseg) {
    case 1: launch_lat<MT, LPR, 1, INT4>(a, wpb, st); break;
    case 2: launch_lat<MT, LPR, 2, INT4>(a, wpb, st); break;
    case 3: launch_lat<MT, LPR, 3, INT4>(a, wpb, st); break;
    default: launch_lat<MT, LPR, 4, INT4>(a, wpb, st); break;
  }
}

// The straight-line decode kernel for M <= 4, K <= kLatMaxK: the widest LPR (32 or 64)
// whose segment divides the row into at most 4 segments. One segment per lane: workgroups of
// 2 wavefronts when there are fewer than 1024 wavefronts, so that the launch covers every CU;
// several: the segments go to as many wavefronts (launch_lat_split). Returns false when it
// does not apply.
template <bool INT4>
bool try_lat(GemvArgs a, bool aligned, hipStream_t st) {
  if (a.M > 4 || a.K > kLatMaxK || !aligned || (INT4 && a.group % 32 != 0)) return false;
  const int cpl = INT4 ? 32 : 16;
  int lpr = 0;
  for (int l : {64, 32})
    if (a.K % (l * cpl) == 0 && a.K / (l * cpl) <= 4) {
      lpr = l;
      break;
    }
  if (lpr == 0) return false;
  const int nseg = a.K / (lpr * cpl);
  const int waves = (a.N + kWave / lpr - 1) / (kWave / lpr);
  const int wpb = waves >= 1024 || a.M > 2 ? 4 : 2;  // M > 2: x registers bound the stage
  if constexpr (INT4) {
    a.G = a.K / a.group;
    const int spg = a.group / cpl;
    a.spg_log2 = static_cast<int16_t>((spg & (spg - 1)) == 0 ? __builtin_ctz(spg) : -1);
  }
  if (a.M == 1) {
    if (lpr == 64) launch_lat_lpr<1, 64, INT4>(a, nseg, wpb, st);
    else launch_lat_lpr<1, 32, INT4>(a, nseg, wpb, st);
  } else if (a.M == 2) {
    if (lpr == 64) launch_lat_lpr<2, 64, INT4>(a, nseg, wpb, st);
    else launch_lat_lpr<2, 32, INT4>(a, nseg, wpb, st);
  } else {
    if (lpr == 64) launch_lat_lpr<4, 64, INT4>(a, nseg, wpb, st);
    else launch_lat_lpr<4, 32, INT4>(a, nseg, wpb, st);
  }
  return true;
}

template <bool INT4>
int run_gemv(GemvArgs a, bool aligned, hipStream_t st, const char* what) {
  if (try_lat<INT4>(a, aligned, st)) return lsh::launch_status(what);
  const int MT = pick_mt(a.M < kTileRows ? a.M : kTileRows);
  const Config c = choose(INT4, MT, a.N, a.K, a.group, aligned);
  int rc = LLMSERVE_OK;
  if (c.lpr == 0) {
    run_generic<INT4>(a, st);
  } else {
    switch (MT) {
      case 1: rc = launch_mt<1, INT4>(a, c, st); break;
      case 2: rc = launch_mt<2, INT4>(a, c, st); break;
      case 4: rc = launch_mt<4, INT4>(a, c, st); break;
      case 8: rc = launch_mt<8, INT4>(a, c, st); break;
      default: rc = launch_mt<16, INT4>(a, c, st); break;
    }
  }
  return rc ? rc : lsh::launch_status(what);
}

}  // namespace

extern "C" int llmserve_int8_linear(const float* x, const int8_t* q, const float* scale, float* y,
                                    int64_t M, int64_t N, int64_t K, void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 1, "int8_linear: bad shape M=%lld N=%lld K=%lld",
            (long long)M, (long long)N, (long long)K);
  LSH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int8_linear: meant for small batches (M <= 64)");
  LSH_CHECK(N < (1LL << 31) && K < (1LL << 31) && N * K < (1LL << 40),
            "int8_linear: shape too large");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(x && q && scale && y, "int8_linear: null pointer");
  GemvArgs a{};
  a.x = x;
  a.w = reinterpret_cast<const uint8_t*>(q);
  a.s = scale;
  a.y = y;
  a.M = static_cast<int16_t>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.group = 1;
  const bool aligned = lsh::aligned16(x) && lsh::aligned16(q) && K % 16 == 0;
  return run_gemv<false>(a, aligned, lsh::as_stream(stream), "int8_linear");
}

extern "C" int llmserve_int4_linear(const float* x, const float* inv_act_scale,
                                    const uint8_t* nibbles, const float* g_scale,
                                    const float* g_zero, float* y, int64_t M, int64_t N, int64_t K,
                                    int64_t group_size, void* stream) {
  LSH_CHECK(M >= 0 && N >= 0 && K >= 1 && group_size >= 2, "int4: shapes");
  LSH_CHECK(K % group_size == 0 && group_size % 2 == 0, "int4: shapes");
  LSH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int4_linear: meant for small batches (M <= 64)");
  LSH_CHECK(N < (1LL << 31) && K < (1LL << 31) && N * K < (1LL << 41),
            "int4_linear: shape too large");
  if (M == 0 || N == 0) return LLMSERVE_OK;
  LSH_CHECK(x && nibbles && g_scale && g_zero && y, "int4_linear: null pointer");
  GemvArgs a{};
  a.x = x;
  a.inv = inv_act_scale;
  a.w = nibbles;
  a.s = g_scale;
  a.z = g_zero;
  a.y = y;
  a.M = static_cast<int16_t>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.group = static_cast<int>(group_size);
  const bool aligned = lsh::aligned16(x) && lsh::aligned16(nibbles) && K % 32 == 0 &&
                       (inv_act_scale == nullptr || lsh::aligned16(inv_act_scale));
  return run_gemv<true>(a, aligned, lsh::as_stream(stream), "int4_linear");
}
