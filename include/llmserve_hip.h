/*
 * llmserve_hip.h - C ABI of the MI355X (gfx950) quantized decode path.
 *
 * Every entry point takes plain device pointers, int64 sizes and a HIP stream passed as
 * `void*` (NULL = the default stream). Work is enqueued on that stream and the call returns
 * without synchronising. A nonzero status means nothing was launched (LLMSERVE_ERR_INVALID:
 * an argument check failed, the same checks the reference makes with TORCH_CHECK) or the
 * launch failed (LLMSERVE_ERR_HIP). `llmserve_last_error()` returns the calling thread's
 * message for the last failure.
 *
 * The reference binds its CPU kernels through pybind11 (kernels/__init__.py:19-72 of
 * Buland-Choudhary/llm-serving-engine, src/llmserve/); each function below names the
 * reference interface it replaces. Tensors are row-major and contiguous. Device pointers for
 * vector loads must be 16-byte aligned; the library checks and falls back to a scalar-load
 * kernel where a shape or pointer does not allow them.
 */
#ifndef LLMSERVE_HIP_H
#define LLMSERVE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMSERVE_OK 0
#define LLMSERVE_ERR_INVALID 1
#define LLMSERVE_ERR_HIP 2

/* Largest number of activation rows a GEMV call accepts. Replaces the reference's
 * TORCH_CHECK(M <= 64) in int8_gemv.cpp:22 and int8_gemv.cpp:64. */
#define LLMSERVE_GEMV_MAX_ROWS 64

/* Message of the last failed call on this thread ("" if none). */
const char* llmserve_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int llmserve_abi_version(void);

/*
 * Measurement hook (no counterpart in the reference): arms two hipEvent_t for the calling
 * thread's next kernel-launching call. Its first kernel records `start_event` when the
 * dispatch starts and its last kernel records `stop_event` when it completes
 * (hipExtLaunchKernelGGL), so hipEventElapsedTime gives the kernels' own execution time,
 * the interval a kernel-trace profiler reports. Either event may be NULL.
 */
int llmserve_time_next_call(void* start_event, void* stop_event);

/* ---- quantize + pack (load time) ------------------------------------------------------ */

/*
 * Symmetric per-output-channel int8 (Int8Linear.__init__, quant.py:41-43):
 *   scale[n] = max(amax_k |w[n,k]| / 127, 1e-8)
 *   q[n,k]   = clamp(round_half_even(w[n,k] / scale[n]), -127, 127)
 * w fp32 [N,K] -> q int8 [N,K], scale fp32 [N]. IEEE division, no contraction: bit-exact
 * with the reference's torch CPU ops.
 */
int llmserve_int8_quantize(const float* w, int8_t* q, float* scale, int64_t N, int64_t K,
                           void* stream);

/*
 * Asymmetric group-wise int4 with optional AWQ fold and nibble packing
 * (Int4Linear.__init__ quant.py:94-121, _int4_quantize quant.py:82-90):
 *   w'       = act_scale ? w * act_scale[None,:] : w
 *   per group of `group_size` input channels: mn, mx of w'
 *   scale    = max((mx - mn) / 15, 1e-8);  q = clamp(round_half_even((w' - mn) / scale), 0, 15)
 *   zero     = mn + 8 * scale               (kernel convention w = (q - 8) * scale + zero)
 *   nibbles[n, j] = q[n, 2j] | q[n, 2j+1] << 4
 *   inv_act_scale[k] = 1 / act_scale[k]     (written when both pointers are non-NULL)
 * w fp32 [N,K] -> nibbles uint8 [N,K/2], g_scale/g_zero fp32 [N,K/group_size].
 * Requires K % group_size == 0 and group_size even (the reference raises ValueError /
 * TORCH_CHECK otherwise, quant.py:100-101, int8_gemv.cpp:63).
 */
int llmserve_int4_quantize(const float* w, const float* act_scale /* nullable [K] */,
                           uint8_t* nibbles, float* g_scale, float* g_zero,
                           float* inv_act_scale /* nullable [K] */, int64_t N, int64_t K,
                           int64_t group_size, void* stream);

/*
 * int8 KV-cache quantize + scatter (QuantizedKV.quantize/write, attention.py:153-162, with
 * the key smoothing division of attention.py:243-245 fused when `smooth` is non-NULL):
 *   x'          = smooth ? x / smooth[h, :] : x
 *   s           = max(amax_d |x'[t,h,d]|, 1e-8) / 127
 *   data[slot]  = clamp(round_half_even(x' / s), -127, 127);  scale[slot, h] = s
 * x fp32 [T,Hk,D], slots int64 [T] -> data int8 [num_slots,Hk,D], scale fp32 [num_slots,Hk].
 * Slots outside [0, num_slots) are skipped (torch.index_copy_ raises for them; the host
 * wrappers check before calling). Duplicate slots race, as index_copy_ leaves them undefined.
 */
int llmserve_kv_quantize_write(const float* x, const int64_t* slots, const float* smooth,
                               int8_t* data, float* scale, int64_t T, int64_t Hk, int64_t D,
                               int64_t num_slots, void* stream);

/* ---- weight-only quantized linears ------------------------------------------------------ */

/*
 * int8 weight-only GEMV for decode (replaces int8_linear, int8_gemv.cpp:13-46):
 *   y[m,n] = scale[n] * sum_k x[m,k] * q[n,k]      (fp32 accumulate)
 * x fp32 [M,K], q int8 [N,K], scale fp32 [N] -> y fp32 [M,N]; 1 <= M <= 64.
 */
int llmserve_int8_linear(const float* x, const int8_t* q, const float* scale, float* y,
                         int64_t M, int64_t N, int64_t K, void* stream);

/*
 * int4 weight-only GEMV for decode (replaces int4_linear, int8_gemv.cpp:53-107, and fuses
 * the AWQ activation pre-scale x * inv_act_scale of Int4Linear.forward, quant.py:137-138):
 *   y[m,n] = sum_g s[n,g] * sum_{k in g} x'[m,k] q[n,k] + (z[n,g] - 8 s[n,g]) * sum_{k in g} x'[m,k]
 *   x' = inv_act_scale ? x * inv_act_scale[None,:] : x
 * x fp32 [M,K], nibbles uint8 [N,K/2], g_scale/g_zero fp32 [N,K/group] -> y fp32 [M,N].
 */
int llmserve_int4_linear(const float* x, const float* inv_act_scale /* nullable [K] */,
                         const uint8_t* nibbles, const float* g_scale, const float* g_zero,
                         float* y, int64_t M, int64_t N, int64_t K, int64_t group_size,
                         void* stream);

/*
 * int4 weight-only linear for M > 16 activation rows on the bf16 matrix cores (replaces
 * Int4Linear.forward's large-M branch, quant.py:141-142: x * inv_act_scale, then
 * x @ dequantize().T), with the same group decomposition as int4_linear:
 *   y[m,n] = sum_g s[n,g] * sum_{k in g} x'[m,k] q[n,k] + (z[n,g] - 8 s[n,g]) * sum_{k in g} x'[m,k]
 * x' = x * inv_act_scale (fp32) is split into two bf16 terms (xh + xl = x' to 2^-18
 * relative) by a pre-pass into `workspace`, so every matrix-core product is exact and the
 * result is within a few 1e-6 (relative) of fp32 arithmetic. Requires K % 128 == 0,
 * group_size % 128 == 0, N % 16 == 0, 16-byte aligned nibbles, 8-byte aligned x and
 * inv_act_scale, and a 16-byte aligned workspace of
 * llmserve_int4_linear_gemm_workspace_bytes(M, K) bytes.
 */
int64_t llmserve_int4_linear_gemm_workspace_bytes(int64_t M, int64_t K);
int llmserve_int4_linear_gemm(const float* x, const float* inv_act_scale /* nullable [K] */,
                              const uint8_t* nibbles, const float* g_scale, const float* g_zero,
                              float* y, int64_t M, int64_t N, int64_t K, int64_t group_size,
                              void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The weights of llmserve_int4_linear_gemm_packed: nibbles, group scales and zeros of
 * llmserve_int4_quantize rearranged once (per weight, at load time) into the order the
 * matrix-core kernel reads them, so that each of its load instructions reads contiguous bytes
 * (no counterpart in the reference, which keeps only the [N, K/2] buffers of Int4Linear,
 * quant.py:109-121). The buffer holds llmserve_int4_gemm_pack_bytes(N, K, group_size) bytes:
 * the nibbles of each 64-row slab and 128-channel block (rows past N zero), then per group,
 * slab and row the scale and z - 8 * scale. Requires K and group_size multiples of 128;
 * nibbles and the packed buffer 16-byte aligned.
 */
int64_t llmserve_int4_gemm_pack_bytes(int64_t N, int64_t K, int64_t group_size);
int llmserve_int4_gemm_pack(const uint8_t* nibbles, const float* g_scale, const float* g_zero,
                            int64_t N, int64_t K, int64_t group_size, void* packed,
                            int64_t packed_bytes, void* stream);

/*
 * Int4Linear's batched path (replaces quant.py:141-142 like llmserve_int4_linear_gemm) on a
 * packed weight: x' = x * inv_act_scale split into three bf16 pieces (hi + mid + lo equals x'
 * to ~2^-26 relative), exact bf16 products, fp32 accumulation, so the result is that of fp32
 * arithmetic up to summation order, with the decode-batch kernel, whose wavefronts issue all loads of their 1-3 K blocks before the first product.
 * Any M, N >= 1; K and group_size multiples of 128. x, inv_act_scale and the packed weight
 * 16-byte aligned; `workspace` (16-byte aligned) holds
 * llmserve_int4_linear_gemm_packed_workspace_bytes(M, K) bytes. Up to 16 rows, a narrow output
 * (whose tiles alone leave most CUs idle) splits its K blocks across workgroups into
 * llmserve_int4_packed_splits(M, N, K) planes (the first in y, the others in the workspace),
 * added in plane order by a second launch: the planes, and so the result, are those of
 * llmserve_int4_linear_gemm_xfrag_split with that split count on the same x', bit for bit.
 */
int64_t llmserve_int4_linear_gemm_packed_workspace_bytes(int64_t M, int64_t K);
int64_t llmserve_int4_packed_splits(int64_t M, int64_t N, int64_t K);
int llmserve_int4_linear_gemm_packed(const float* x, const float* inv_act_scale /* nullable */,
                                     const void* packed, float* y, int64_t M, int64_t N,
                                     int64_t K, int64_t group_size, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/*
 * Activation fragments: x' = x * inv_act_scale as the packed kernel reads it (bf16 hi / mid /
 * lo pieces in wavefront order, then fp32 sums of x' over every 128-channel block; rows up to M
 * rounded to 16, the extra rows zero). llmserve_int4_xfrag_bytes(M, K) bytes, 16-byte aligned.
 * Written by llmserve_int4_xfrag_split (the split pass of llmserve_int4_linear_gemm_packed
 * above 16 rows; up to 16 rows that entry point builds the same values inside its GEMM launch,
 * using its workspace only for K planes) or by the fused producers below (bit-identical for the same
 * x'); read by llmserve_int4_linear_gemm_xfrag, which is llmserve_int4_linear_gemm_packed on
 * given fragments. No counterpart in the reference: they fuse Int4Linear's
 * `x * inv_act_scale` (quant.py:141) into the producing kernel.
 */
int64_t llmserve_int4_xfrag_bytes(int64_t M, int64_t K);
/* x [M, K] fp32 (times inv_act_scale [K] when given) -> fragments in xfrag
 * (xfrag_bytes >= llmserve_int4_xfrag_bytes(M, K); K a multiple of 128). */
int llmserve_int4_xfrag_split(const float* x, const float* inv_act_scale /* nullable */,
                              void* xfrag, int64_t M, int64_t K, int64_t xfrag_bytes,
                              void* stream);
int llmserve_int4_linear_gemm_xfrag(const void* xfrag, const void* packed, float* y, int64_t M,
                                    int64_t N, int64_t K, int64_t group_size, void* stream);

/*
 * llmserve_int4_linear_gemm_xfrag with K split across workgroups for narrow outputs (o_proj,
 * down_proj at decode batches, whose 64-channel slabs alone occupy a quarter of the GPU): y is
 * [splits, M, N], plane p the sum over the K blocks [p ceil(nb / splits), ...) (nb = K / 128),
 * and the linear's output is the planes added in order (llmserve_add_rmsnorm_split_xfrag does
 * that as it adds the residual). llmserve_int4_xfrag_splits gives the split count used by the
 * decode step (1 when the output fills the GPU without it); splits in [1, 8]. No counterpart
 * in the reference: a work split of Int4Linear.forward (quant.py:141-142).
 */
int64_t llmserve_int4_xfrag_splits(int64_t M, int64_t N, int64_t K);
int llmserve_int4_linear_gemm_xfrag_split(const void* xfrag, const void* packed, float* y,
                                          int64_t M, int64_t N, int64_t K, int64_t group_size,
                                          int64_t splits, void* stream);

/*
 * Prefill-sized int8 weight-only linear on the bf16 matrix cores (replaces Int8Linear's
 * large-M path, quant.py:71-72 with dequantize quant.py:78-79: x @ (q * scale[:, None]).T):
 *   y[m, n] = scale[n] * sum_k bf16(x[m, k]) * q[n, k]      (fp32 accumulate)
 * x is rounded to bf16 (nearest even) once into `workspace`; the int8 weight is exact in
 * bf16. x fp32 [M,K], q int8 [N,K], scale fp32 [N] -> y fp32 [M,N]. K must be a multiple of
 * 64; x, q and the workspace 16-byte aligned; the workspace holds
 * llmserve_int8_linear_prefill_workspace_bytes(M, N, K) bytes: the bf16 copy of x and, when
 * the output has fewer 256 x 256 tiles than the device has CUs, the fp32 partial sums of the
 * K splits (their count depends on the current device).
 */
int64_t llmserve_int8_linear_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K);
int llmserve_int8_linear_prefill(const float* x, const int8_t* qweight, const float* scale,
                                 float* y, int64_t M, int64_t N, int64_t K, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* ---- decoder-layer elementwise ops and decode-step glue ---------------------------------- */

/*
 * out = w * (x * inv), inv = 1 / sqrt(mean_h(x^2) + eps), per row of H (replaces rmsnorm,
 * fused_ops.cpp:23-30 and :39-56). x, out fp32 [T, H]; w fp32 [H].
 */
int llmserve_rmsnorm(const float* x, const float* w, float* out, int64_t T, int64_t H, float eps,
                     void* stream);

/*
 * x += r (in place), then out = rmsnorm(x) * w (replaces add_rmsnorm_, fused_ops.cpp:58-81).
 */
int llmserve_add_rmsnorm(float* x, const float* r, const float* w, float* out, int64_t T,
                         int64_t H, float eps, void* stream);

/*
 * x[t] = embed[ids[t]], then out[t] = rmsnorm(x[t]) * w: the embedding lookup and the first
 * layer's input norm of the fused forward (replaces embed_tokens + fo.rmsnorm,
 * models/transformer.py:151-155). ids int64 [T] in [0, V) (an id outside gives a NaN row);
 * embed fp32 [V, H]; x (the residual stream) and out fp32 [T, H].
 */
int llmserve_embed_rmsnorm(const int64_t* ids, const float* embed, int64_t V, const float* w,
                           float* x, float* out, int64_t T, int64_t H, float eps, void* stream);

/*
 * The norms above writing the next int4 linear's activation fragments instead of fp32 rows
 * (rmsnorm / add_rmsnorm_ / embedding + rmsnorm fused with Int4Linear's x * inv_act_scale,
 * fused_ops.cpp:23-81 and quant.py:141): x' = (w * (x * inv)) * act_inv (act_inv nullable),
 * written to `xfrag` (llmserve_int4_xfrag_bytes(T, H) bytes). The residual x is updated as
 * by the plain kernels. H a multiple of 128.
 */
int llmserve_rmsnorm_xfrag(const float* x, const float* w, const float* act_inv, void* xfrag,
                           int64_t T, int64_t H, float eps, void* stream);
int llmserve_add_rmsnorm_xfrag(float* x, const float* r, const float* w, const float* act_inv,
                               void* xfrag, int64_t T, int64_t H, float eps, void* stream);
/* llmserve_add_rmsnorm_xfrag whose residual r is `planes` partial sums [planes, T, H] (the
 * output planes of llmserve_int4_linear_gemm_xfrag_split): x += (r_0 + r_1 + ... in plane
 * order), then the norm and the fragments as llmserve_add_rmsnorm_xfrag; planes in [1, 64]. */
int llmserve_add_rmsnorm_split_xfrag(float* x, const float* r, int64_t planes, const float* w,
                                     const float* act_inv, void* xfrag, int64_t T, int64_t H,
                                     float eps, void* stream);
int llmserve_embed_rmsnorm_xfrag(const int64_t* ids, const float* embed, int64_t V,
                                 const float* w, const float* act_inv, float* x, void* xfrag,
                                 int64_t T, int64_t H, float eps, void* stream);

/*
 * silu(gate) * up (fused_ops.cpp:83-99) times the down projection's act_inv (nullable), as
 * activation fragments of [T, I] (llmserve_int4_xfrag_bytes(T, I) bytes). I a multiple of 128.
 */
int llmserve_silu_mul_xfrag(const float* gate_up, const float* act_inv, void* xfrag, int64_t T,
                            int64_t I, void* stream);

/*
 * out[t, i] = gate / (1 + exp(-gate)) * up for a fused gate|up row (replaces silu_mul,
 * fused_ops.cpp:83-99). gate_up fp32 [T, 2I] -> out fp32 [T, I].
 */
int llmserve_silu_mul(const float* gate_up, float* out, int64_t T, int64_t I, void* stream);

/*
 * In place on the fused qkv rows (replaces rope_qk_, fused_ops.cpp:101-127): for each of the
 * first n_q (q) and next n_k (k) heads of a row, optional per-head RMSNorm with q_w / k_w
 * (Qwen3), then rotate-half RoPE with cos/sin [T, D]:
 *   out[d] = x[d] c[d] - x[d + D/2] s[d] (d < D/2),  x[d] c[d] + x[d - D/2] s[d] (d >= D/2).
 * qkv fp32 rows of row_stride floats; head_dim D in {16, 32, 64, 128, 256}.
 */
int llmserve_rope_qk(float* qkv, const float* cos, const float* sin, int64_t T,
                     int64_t row_stride, int64_t n_q, int64_t n_k, int64_t D,
                     const float* q_w /* nullable */, const float* k_w /* nullable */, float eps,
                     void* stream);

/*
 * Decode step glue after the qkv projection (one token per sequence; no single reference
 * function: it is rope_qk_ followed by paged_attention's cache write, attention.py:221-228
 * with QuantizedKV.write :159-162 and the key smoothing :243-245). For token t at position
 * p = context_lens[t] - 1 (context_lens counts the new token):
 *   q heads: norm(q_w) + RoPE with row p of cos_table/sin_table [max_pos, D] -> q_out [T, n_q, D]
 *   k heads: norm(k_w) + RoPE, / k_smooth[h], int8 quantized into k_cache/k_scale at slot
 *            block_tables[t, p / block_size] * block_size + p % block_size
 *   v heads: int8 quantized into v_cache/v_scale at the same slot.
 * The quantizer is llmserve_kv_quantize_write's (bit-identical). Tokens whose position or
 * block is outside the tables or the cache are skipped.
 */
int llmserve_decode_qkv_kv(const float* qkv, int64_t row_stride, const float* cos_table,
                           const float* sin_table, int64_t max_pos, const int64_t* context_lens,
                           const int64_t* block_tables, int64_t max_blocks, int64_t block_size,
                           const float* q_w, const float* k_w, float eps,
                           const float* k_smooth /* nullable [n_k, D] */, float* q_out,
                           int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
                           int64_t num_slots, int64_t T, int64_t n_q, int64_t n_k, int64_t D,
                           void* stream);

/*
 * Greedy decoding (sampling.py:151-170 at temperature 0): next_ids[t] = argmax over logits
 * [T, V] of row t (the first index among equal maxima), then context_lens[t] += 1.
 * `workspace` holds llmserve_argmax_advance_workspace_bytes(T) bytes (16-byte aligned).
 */
int64_t llmserve_argmax_advance_workspace_bytes(int64_t T);
int llmserve_argmax_advance(const float* logits, int64_t T, int64_t V, int64_t* next_ids,
                            int64_t* context_lens, void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * fp32 LM head on activation fragments (replaces the tied-embedding lm_head,
 * models/transformer.py:192-193): y[M, V] = x[M, K] . w[V, K]^T with w fp32 row-major and x
 * given as llmserve_int4_xfrag_bytes(M, K) bytes of fragments (written, e.g., by
 * llmserve_add_rmsnorm_xfrag with act_inv = NULL). Split-bf16 matrix-core products (the hi,
 * mid and lo pieces of x and of w, the six products down to 2^-16 of the leading one, fp32
 * accumulation): each product is the fp32 product up to fp32's rounding. K a multiple of 128;
 * xfrag, w and y 16-byte aligned.
 */
int llmserve_lm_head_f32_xfrag(const void* xfrag, const float* w, float* y, int64_t M, int64_t V,
                               int64_t K, void* stream);

/*
 * The same fp32 LM head for a decode batch of 1-4 rows (models/transformer.py:192-193 at batch
 * 1-4, where the reference's F.linear is a GEMV over the whole matrix): y[M, V] = x[M, K] .
 * w[V, K]^T in exact fp32 arithmetic (up to summation order), streaming w once. K = 256, 512
 * or 1024; x and w 16-byte aligned.
 */
int llmserve_lm_head_f32(const float* x, const float* w, float* y, int64_t M, int64_t V, int64_t K,
                         void* stream);

/* ---- int8-KV paged decode attention ------------------------------------------------------ */

/*
 * Split-context paged decode over an int8 KV cache (replaces paged_attention_decode_int8 ->
 * pa2::decode<int8_t>, paged_attention.cpp:141-346 and :361-376). For each sequence b, kv
 * head h and the G = Hq/Hk query heads sharing it:
 *   s_t   = scale * k_scale[slot_t,h] * (q'_g . k_cache[slot_t,h,:])
 *   out_g = sum_t softmax(s)_t * v_scale[slot_t,h] * v_cache[slot_t,h,:]
 *   q'    = q_mult ? q * q_mult : q            (key smoothing, attention.py:243-244)
 *   slot_t = block_tables[b, t / block_size] * block_size + t % block_size
 * q fp32 [B,Hq,D]; k/v_cache int8 [num_slots,Hk,D]; k/v_scale fp32 [num_slots,Hk];
 * block_tables int64 [B,max_blocks]; context_lens int64 [B] -> out fp32 [B,Hq,D].
 * The context is split, as the reference's partitions are, into work ranges whose partial
 * (max, sum, acc) are merged: partition_size = tokens per range; 0 picks the range size
 * itself, the smallest multiple of 64 tokens whose ranges fit the GPU's resident workgroups
 * once, and cuts each (sequence, kv head group) into ranges of that size, the last one the
 * rest (ranges never straddle two sequences; a sequence more than a few
 * times the batch's mean context gets wider ranges, so that its partials fit a workspace
 * bounded by the grid rather than by max_blocks). Block ids outside [0, num_slots/block_size) contribute nothing;
 * context lengths are clamped to max_blocks*block_size. A zero context yields NaN, as the
 * reference's 0 * (1/0) does. `workspace` holds the partials: at least
 * llmserve_paged_attention_workspace_bytes(...) bytes (non-zero whenever B > 0; the size of
 * the balanced split depends on the current device).
 */
int64_t llmserve_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                                 int64_t max_blocks, int64_t block_size,
                                                 int64_t partition_size);
int llmserve_paged_attention_decode_int8(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, int64_t partition_size, const float* q_mult /* nullable */,
    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * llmserve_paged_attention_decode_int8 whose merge also writes the next linear's input: the
 * attention output [B, Hq*D] times act_inv (nullable; the o_proj's inv_act_scale) as
 * activation fragments (llmserve_int4_xfrag_bytes(B, Hq*D) bytes at xfrag, 16-byte aligned)
 * for llmserve_int4_linear_gemm_xfrag. `out` is written as by the plain entry; the fragments
 * equal what llmserve_rmsnorm_xfrag-style producers write for the same x' (same rounding and
 * block-sum order). D = 128 or 256. No counterpart in the reference: it fuses Int4Linear's
 * `x * inv_act_scale` (quant.py:141) of o_proj into the attention's last kernel.
 */
int llmserve_paged_attention_decode_int8_xfrag(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    const float* act_inv /* nullable */, void* xfrag, int64_t B, int64_t Hq, int64_t Hk, int64_t D,
    int64_t num_slots, int64_t max_blocks, int64_t block_size, float scale,
    int64_t partition_size, const float* q_mult /* nullable */, void* workspace,
    int64_t workspace_bytes, void* stream);

/*
 * The same split-context paged decode over a float32 KV cache (replaces
 * paged_attention_decode -> pa2::decode<float>, paged_attention.cpp:350-359, :141-346):
 *   s_t = scale * (q_g . k_cache[slot_t,h,:]);  out_g = sum_t softmax(s)_t * v_cache[slot_t,h,:]
 * k/v_cache fp32 [num_slots,Hk,D]; everything else, the split and the workspace
 * (llmserve_paged_attention_workspace_bytes) as llmserve_paged_attention_decode_int8.
 */
int llmserve_paged_attention_decode(const float* q, const float* k_cache, const float* v_cache,
                                    const int64_t* block_tables, const int64_t* context_lens,
                                    float* out, int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                    int64_t num_slots, int64_t max_blocks, int64_t block_size,
                                    float scale, int64_t partition_size, void* workspace,
                                    int64_t workspace_bytes, void* stream);

/*
 * Paged attention for the query rows of a ragged batch, decode and prefill alike (replaces
 * paged_attention's prefill loop and decode branch, attention.py:249-307, over the cache of
 * attention.py:241-246): query row r attends, with the paged decode's split and merge, to the
 * first row_context[r] tokens of block-table row row_table[r] (0 <= row_table[r] < table_rows;
 * a row outside gives NaN, as a zero context does). A prefill token at position p is a row
 * with context p + 1, which is the causal mask of the reference's SDPA call
 * (attention.py:114-124). llmserve_attention_metadata writes row_table / row_context for a
 * step. q fp32 [R,Hq,D] (times q_mult [Hq,D] when non-NULL: key smoothing); block_tables int64
 * [table_rows,max_blocks]; out fp32 [R,Hq,D]; the workspace holds
 * llmserve_paged_attention_workspace_bytes(R, Hq, Hk, D, max_blocks, block_size, 0) bytes.
 */
int llmserve_paged_attention_rows_int8(const float* q, const int8_t* k_cache,
                                       const int8_t* v_cache, const float* k_scale,
                                       const float* v_scale, const int64_t* block_tables,
                                       int64_t table_rows, const int64_t* row_table,
                                       const int64_t* row_context, float* out, int64_t R,
                                       int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots,
                                       int64_t max_blocks, int64_t block_size, float scale,
                                       const float* q_mult /* nullable */, void* workspace,
                                       int64_t workspace_bytes, void* stream);
int llmserve_paged_attention_rows_f32(const float* q, const float* k_cache, const float* v_cache,
                                      const int64_t* block_tables, int64_t table_rows,
                                      const int64_t* row_table, const int64_t* row_context,
                                      float* out, int64_t R, int64_t Hq, int64_t Hk, int64_t D,
                                      int64_t num_slots, int64_t max_blocks, int64_t block_size,
                                      float scale, const float* q_mult /* nullable */,
                                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Attention metadata of one step on the device (replaces the host loops of
 * AttentionMetadata.build, attention.py:61-112): S sequences, sequence s with q_len new tokens
 * at the end of its ctx_len-token context, its blocks in row s of block_tables int64
 * [S,max_blocks]. seq_info int64 [3,S] holds q_lens, ctx_lens and q_start (the exclusive
 * prefix sums of q_lens); T = sum of q_lens. For token t of sequence s at position p:
 *   slot_mapping[t] = block_tables[s, p / block_size] * block_size + p % block_size
 *                     (-1 when the block is past the table or its id is negative)
 *   row_table[t] = s;  row_context[t] = p + 1.
 */
int llmserve_attention_metadata(const int64_t* seq_info, const int64_t* block_tables, int64_t S,
                                int64_t max_blocks, int64_t block_size, int64_t T,
                                int64_t* slot_mapping, int64_t* row_table, int64_t* row_context,
                                void* stream);

/*
 * One decoder layer for a decode batch of M <= 4 sequences as one persistent launch:
 * this layer's attention, its linear chain and the next layer's qkv (replaces, for small
 * batches, the reference's per-op sequence of _forward_fused, models/transformer.py:157-189,
 * with the decode attention of paged_attention_decode_int8, paged_attention.cpp:191-420,
 * Int4Linear.forward, quant.py:134-151, and the cache write of paged_attention,
 * attention.py:241-246):
 *   attn = paged decode attention of q_in [M, n_q, 128] (times q_mult [n_q, 128] when given)
 *          over this layer's int8 caches attn_k_cache / attn_v_cache [num_slots, n_k, 128]
 *          with scales attn_k_scale / attn_v_scale [num_slots, n_k], the first
 *          context_lens[m] tokens of row m (softmax scale `scale`; a row with no context
 *          gives NaN)
 *   x1 = x_in + o_proj(attn);  h = rmsnorm(x1) * post_w;  a = silu(gate(h)) * up(h)
 *   x_out = x1 + down(a);      h2 = rmsnorm(x_out) * next_w
 *   then, when qkv_nib is given (not the last layer): the next layer's qkv = qkv_proj(h2),
 *   per-head RMSNorm (q_w / k_w, nullable) and rotate-half RoPE of q and k at position
 *   p = context_lens[m] - 1 (rows p of cos_t / sin_t [max_pos, 128]), q -> q_out [M, n_q, 128],
 *   k / k_smooth (nullable) and v int8-quantized into the caches k_cache / v_cache (the next
 *   layer's) at slot block_tables[m, p / block_size] * block_size + p % block_size (the
 *   quantizer of llmserve_kv_quantize_write; a position outside the tables leaves the cache
 *   and gives a NaN q row); otherwise h_out (nullable) = h2, the final norm's output.
 * Embedding mode (q_in == NULL): x_out = embed[ids] (an id outside [0, vocab) gives a NaN
 * row), then the qkv part for layer 0 with next_w = its input norm.
 * int4 weights are the Int4Linear buffers (nibbles [N, K/2], g_scale / g_zero [N, K/128],
 * inv_act_scale [K] nullable); o_proj [H, n_q*128], gate_up [2I, H], down [H, I], qkv
 * [(n_q + 2 n_k) * 128, H]. Requires head_dim = group_size = 128, H a multiple of 128 in
 * [256, 1024] and of 2 (n_q + 2 n_k), n_q * 128 <= 2048, I a multiple of 512 and of H / 8,
 * at most 4096, with I / (H / 8) a multiple of 8 and at most 32, 16-byte aligned weights,
 * activations and norm weights; x_out must not alias x_in and q_out must not alias q_in.
 * The attention needs n_q = 2 n_k, n_k <= 8, block_size a power of two >= 8, caches of under
 * 2^32 bytes and M n_q <= the grid. The H / 8 [+ n_q + 2 n_k] workgroups hand data to each
 * other through `workspace` (llmserve_decode_chain_workspace_bytes(H, I) bytes, 16-byte
 * aligned, zero before its first use and then owned by the chain: launches that overlap on
 * one workspace race) and must all be resident at once (checked). Each hand-off wait gives up
 * after `spin_limit` polls, sets the workspace's error word (llmserve_decode_chain_error) and
 * lets the grid finish. No counterpart in the reference.
 */
int64_t llmserve_decode_chain_workspace_bytes(int64_t H, int64_t I);
int llmserve_decode_chain(
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
    int64_t workspace_bytes, int64_t spin_limit, void* stream);
/* The chain workspace's error word (nonzero: a hand-off wait ran out of polls). Synchronizes. */
int llmserve_decode_chain_error(const void* workspace, int* error);

/*
 * llmserve_paged_attention_decode_int8 without a workspace argument, for callers that cannot
 * allocate device memory (HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The split-context partials go to a scratch
 * array of llmserve_paged_attention_noalloc_scratch_bytes() bytes (32 MiB) that the library
 * holds on each device it runs on until the process ends; a call whose partials
 * (llmserve_paged_attention_workspace_bytes(...)) exceed it fails with LLMSERVE_ERR_INVALID
 * before anything runs. Calls on one device share the array: calls that overlap on a device
 * race. Arguments and results otherwise as llmserve_paged_attention_decode_int8 (same kernels,
 * same bits). Allocates nothing.
 */
int64_t llmserve_paged_attention_noalloc_scratch_bytes(void);
int llmserve_paged_attention_decode_int8_noalloc(
    const float* q, const int8_t* k_cache, const int8_t* v_cache, const float* k_scale,
    const float* v_scale, const int64_t* block_tables, const int64_t* context_lens, float* out,
    int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t num_slots, int64_t max_blocks,
    int64_t block_size, float scale, int64_t partition_size, const float* q_mult /* nullable */,
    void* stream);

/*
 * Batched token sampler (replaces the body of sampling.sample, sampling.py:151-189, for a
 * logits batch on the GPU): one workgroup per row of logits [B, V] (float32, row-major,
 * V < 2^24). Per row, in the reference's order: presence / frequency penalties over the
 * row's generated tokens (CSR out_ptr [B + 1] / out_ids / out_cnt: distinct ids and their
 * counts), then the repetition penalty over its prompt + generated tokens (seen_ptr /
 * seen_ids, distinct), both written into `logits` (apply_penalties, sampling.py:100-120); the
 * allowed set when has_allow[b] (allow_ptr / allow_ids: every other token -inf) and the
 * banned tokens (ban_ptr / ban_ids: -inf), also in place (sampling.py:165-170). A row with
 * temperature < 1e-5 takes the first index of its maximum (NaN above every number). Any other
 * row samples argmax p / E: p the softmax of logits / temperature after the top-k / top-p
 * cut (when use_topkp, the batch-wide switch of _top_k_top_p_min_p, sampling.py:123-143;
 * top_k -1 is off; the cut is the reference's up to the rounding of the mass before a token
 * at top_p) and the min-p cut (when use_minp), E its Exp(1) noise row noise[noise_row[b]]
 * (sampling.py:183-187). Writes tokens [B] (int64). Greedy-only batches still pass a valid
 * noise buffer (it is not read).
 */
int llmserve_sample(float* logits, int64_t B, int64_t V, const float* temperature,
                    const int* top_k, const float* top_p, const float* min_p,
                    const float* presence, const float* frequency, const float* repetition,
                    const int64_t* out_ptr, const int64_t* out_ids, const int* out_cnt,
                    const int64_t* seen_ptr, const int64_t* seen_ids, const int64_t* allow_ptr,
                    const int64_t* allow_ids, const uint8_t* has_allow, const int64_t* ban_ptr,
                    const int64_t* ban_ids, const float* noise, const int64_t* noise_row,
                    int use_topkp, int use_minp, int64_t* tokens, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLMSERVE_HIP_H */
