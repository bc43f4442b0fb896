// Per-step attention metadata on the device (replaces the per-sequence host loops of
// AttentionMetadata.build, attention.py:61-112 of the reference).
//
// A step's batch is S sequences whose new tokens are laid end to end in a flat [T] stream:
// sequence s owns tokens [q_start[s], q_start[s] + q_lens[s]), the last q_lens[s] positions of
// its ctx_lens[s]-token context, whose blocks are row s of the [S, max_blocks] block table.
// One thread per token t finds its sequence (binary search over q_start) and writes
//   slot_mapping[t] = table[s, p / bs] * bs + p % bs     (p = ctx - q_len + j, j = t - q_start)
//   row_table[t]    = s                                  (the block-table row it attends over)
//   row_context[t]  = p + 1                              (causal: the tokens up to and
//                                                         including its own position)
// so that the new K/V rows go to slot_mapping and every token, decode or prefill, is one
// query row of the paged attention kernel (llmserve_paged_attention_rows_*). A position whose
// block lies past the table, or a table entry below 0, gets slot -1, which the cache writers
// skip.
#include "common.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void attention_metadata_kernel(
    const int64_t* __restrict__ q_lens, const int64_t* __restrict__ ctx_lens,
    const int64_t* __restrict__ q_start, const int64_t* __restrict__ tables, int S,
    int max_blocks, int64_t bs, int64_t T, int64_t* __restrict__ slot_mapping,
    int64_t* __restrict__ row_table, int64_t* __restrict__ row_context) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= T) return;
  // last s with q_start[s] <= t (q_start is non-decreasing, q_start[0] = 0)
  int lo = 0, hi = S - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (q_start[mid] <= t)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int s = lo;
  const int64_t pos = ctx_lens[s] - q_lens[s] + (t - q_start[s]);
  const int64_t blk = pos >= 0 ? pos / bs : -1;
  int64_t slot = -1;
  if (blk >= 0 && blk < max_blocks) {
    const int64_t id = tables[static_cast<int64_t>(s) * max_blocks + blk];
    if (id >= 0) slot = id * bs + pos % bs;
  }
  slot_mapping[t] = slot;
  row_table[t] = s;
  row_context[t] = pos + 1;
}

}  // namespace

extern "C" int llmserve_attention_metadata(const int64_t* seq_info, const int64_t* block_tables,
                                           int64_t S, int64_t max_blocks, int64_t block_size,
                                           int64_t T, int64_t* slot_mapping, int64_t* row_table,
                                           int64_t* row_context, void* stream) {
  LSH_CHECK(S >= 0 && T >= 0 && max_blocks >= 0 && block_size >= 1,
            "attention_metadata: bad sizes (S=%lld, T=%lld, max_blocks=%lld, block_size=%lld)",
            (long long)S, (long long)T, (long long)max_blocks, (long long)block_size);
  if (T == 0) return LLMSERVE_OK;
  LSH_CHECK(S >= 1 && max_blocks >= 1, "attention_metadata: tokens without sequences or blocks");
  LSH_CHECK(S < (1LL << 31) && max_blocks < (1LL << 31) && T < (1LL << 40),
            "attention_metadata: batch too large");
  LSH_CHECK(seq_info && block_tables && slot_mapping && row_table && row_context,
            "attention_metadata: null pointer");
  const int64_t grid = (T + kThreads - 1) / kThreads;
  lsh::launch(attention_metadata_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,
              lsh::as_stream(stream), true, seq_info, seq_info + S, seq_info + 2 * S, block_tables,
              static_cast<int>(S), static_cast<int>(max_blocks), block_size, T, slot_mapping,
              row_table, row_context);
  return lsh::launch_status("attention_metadata");
}
