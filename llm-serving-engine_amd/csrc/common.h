// Shared helpers of the gfx950 kernels: error reporting for the C ABI, launch checks and
// wavefront (64-lane) reductions.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "llmserve_hip.h"

namespace lsh {

// Records the calling thread's last error message (read by llmserve_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks the status of the launch just enqueued.
int launch_status(const char* what);

// Events armed by llmserve_time_next_call() for the calling thread.
struct TimingEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
TimingEvents& timing_events();

// Enqueues `kernel`. When events are armed, the first launch of the call records the start
// event at its dispatch start and the launch marked `last` records the stop event at its
// completion (hipExtLaunchKernelGGL: the kernel's own execution interval).
template <typename F, typename... Args>
void launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, bool last, Args... args) {
  TimingEvents& t = timing_events();
  if (t.start == nullptr && t.stop == nullptr) {
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    return;
  }
  hipEvent_t start = t.start, stop = last ? t.stop : nullptr;
  t.start = nullptr;
  if (last) t.stop = nullptr;
  hipExtLaunchKernelGGL(kernel, grid, block, static_cast<std::uint32_t>(lds), st, start, stop, 0u,
                        args...);
}

constexpr int kWave = 64;

// ---- cross-lane reductions --------------------------------------------------------------
// Within a row of 16 lanes: DPP (quad_perm, row_half_mirror, row_mirror, row_ror), which the
// compiler fuses into the VALU op. Across rows (xor 16 / 32) the steps use ds_bpermute
// (__shfl_xor); the hot loops only reduce within rows, the crossings run once per row or
// partition at the end. (gfx950's v_permlane16/32_swap builtins would avoid the LDS
// crossbar, but this compiler returns the same register for both of their results.)

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

constexpr int kQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;

// Sum over each aligned group of W consecutive lanes (W a power of two <= 64); every lane
// of the group gets the sum.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 2) v += dpp<kQuadXor1>(v);
  if constexpr (W >= 4) v += dpp<kQuadXor2>(v);
  if constexpr (W >= 8) v += dpp<kRowHalfMirror>(v);
  if constexpr (W >= 16) v += dpp<kRowMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// Writes `v` from a DPP source into the rows of ROWMASK; lanes of the other rows get 0.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_rows(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROWMASK, 0xF, false));
}

constexpr int kRowBcast15 = 0x142;  // lane 15 of each row -> every lane of the next row
constexpr int kRowBcast31 = 0x143;  // lane 31 -> every lane of rows 2 and 3

// Sum over each aligned group of W consecutive lanes (W a power of two <= 64), valid in the
// group's last lane (lane % W == W - 1). Rows of 16 lanes reduce with DPP butterflies; rows
// are joined by DPP row broadcasts, so no step goes through the LDS crossbar.
template <int W>
__device__ __forceinline__ float group_total(float v) {
  if constexpr (W <= 16) {
    return group_sum<W>(v);
  } else {
    v = group_sum<16>(v);
    v += dpp_rows<kRowBcast15, 0xA>(v);  // rows 1 and 3 hold the sums of lanes 0-31, 32-63
    if constexpr (W == 64) v += dpp_rows<kRowBcast31, 0xC>(v);  // row 3 holds all 64
    return v;
  }
}

// Max over each aligned group of W consecutive lanes (W a power of two <= 16: DPP only).
template <int W>
__device__ __forceinline__ float group_max(float v) {
  static_assert(W <= 16, "group_max: DPP rows of 16 lanes");
  if constexpr (W >= 2) v = fmaxf(v, dpp<kQuadXor1>(v));
  if constexpr (W >= 4) v = fmaxf(v, dpp<kQuadXor2>(v));
  if constexpr (W >= 8) v = fmaxf(v, dpp<kRowHalfMirror>(v));
  if constexpr (W >= 16) v = fmaxf(v, dpp<kRowMirror>(v));
  return v;
}

// Sum / max over the lanes that share lane % LO (LO a power of two <= 64): the "columns"
// of a wave laid out as rows of LO lanes. Every lane gets its column's result; for LO <= 4
// the two row rotations pair the partial sums differently in different lanes, so the sum may
// differ in its last bit between lanes (group_sum<64> gives every lane the same bits).
template <int LO>
__device__ __forceinline__ float wave_sum_from(float v) {
  if constexpr (LO <= 1) v += dpp<kQuadXor1>(v);
  if constexpr (LO <= 2) v += dpp<kQuadXor2>(v);
  if constexpr (LO <= 4) v += dpp<kRowRor4>(v);
  if constexpr (LO <= 8) v += dpp<kRowRor8>(v);
  if constexpr (LO <= 16) v += __shfl_xor(v, 16, kWave);
  if constexpr (LO <= 32) v += __shfl_xor(v, 32, kWave);
  return v;
}

template <int LO>
__device__ __forceinline__ float wave_max_from(float v) {
  if constexpr (LO <= 1) v = fmaxf(v, dpp<kQuadXor1>(v));
  if constexpr (LO <= 2) v = fmaxf(v, dpp<kQuadXor2>(v));
  if constexpr (LO <= 4) v = fmaxf(v, dpp<kRowRor4>(v));
  if constexpr (LO <= 8) v = fmaxf(v, dpp<kRowRor8>(v));
  if constexpr (LO <= 16) v = fmaxf(v, __shfl_xor(v, 16, kWave));
  if constexpr (LO <= 32) v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

}  // namespace lsh

#define LSH_CHECK(cond, ...)                 \
  do {                                       \
    if (!(cond)) {                           \
      ::lsh::set_error(__VA_ARGS__);         \
      return LLMSERVE_ERR_INVALID;           \
    }                                        \
  } while (0)
