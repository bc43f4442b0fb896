// Thin PyTorch binding of the C ABI (include/llmserve_hip.h) as torch.ops.llmserve_hip.*.
//
// Each op keeps the reference's Python-visible signature (int8_gemv.cpp:109-112,
// paged_attention.cpp:386-399 of the reference) and argument checks, takes ROCm tensors,
// allocates its outputs and workspaces with PyTorch's caching allocator and enqueues the
// kernels on the current HIP stream of the input's device without synchronising.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "llmserve_hip.h"

namespace {

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

void check_status(int rc) {
  TORCH_CHECK(rc == LLMSERVE_OK, llmserve_last_error());
}

void check_device(const at::Tensor& ref, std::initializer_list<const at::Tensor*> ts,
                  const char* what) {
  TORCH_CHECK(ref.is_cuda(), what, ": tensors must be on a ROCm device (got ", ref.device(), ")");
  for (const at::Tensor* t : ts)
    TORCH_CHECK(t->device() == ref.device(), what, ": all tensors must be on ", ref.device());
}

template <typename T>
const T* opt_ptr(const std::optional<at::Tensor>& t) {
  return t.has_value() ? t->data_ptr<T>() : nullptr;
}

// ---- quantize + pack ---------------------------------------------------------------------

std::tuple<at::Tensor, at::Tensor> int8_quantize(const at::Tensor& w) {
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kFloat && w.is_contiguous(),
              "int8_quantize: weight must be a contiguous float32 [out, in] tensor");
  check_device(w, {}, "int8_quantize");
  const c10::DeviceGuard guard(w.device());
  const int64_t N = w.size(0), K = w.size(1);
  auto q = at::empty({N, K}, w.options().dtype(at::kChar));
  auto s = at::empty({N}, w.options());
  check_status(llmserve_int8_quantize(w.data_ptr<float>(), q.data_ptr<int8_t>(), s.data_ptr<float>(),
                                      N, K, stream_of(w)));
  return {q, s};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> int4_quantize(
    const at::Tensor& w, int64_t group_size, const std::optional<at::Tensor>& act_scale) {
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kFloat && w.is_contiguous(),
              "int4_quantize: weight must be a contiguous float32 [out, in] tensor");
  check_device(w, {}, "int4_quantize");
  const int64_t N = w.size(0), K = w.size(1);
  if (act_scale.has_value()) {
    check_device(w, {&*act_scale}, "int4_quantize");
    TORCH_CHECK(act_scale->scalar_type() == at::kFloat && act_scale->is_contiguous() &&
                    act_scale->numel() == K,
                "int4_quantize: act_scale must be a contiguous float32 [in] tensor");
  }
  TORCH_CHECK(group_size > 0 && K % group_size == 0, "in_features ", K,
              " not divisible by group ", group_size);
  const c10::DeviceGuard guard(w.device());
  auto nib = at::empty({N, K / 2}, w.options().dtype(at::kByte));
  auto gs = at::empty({N, K / group_size}, w.options());
  auto gz = at::empty({N, K / group_size}, w.options());
  auto inv = at::empty({act_scale.has_value() ? K : 0}, w.options());
  check_status(llmserve_int4_quantize(w.data_ptr<float>(), opt_ptr<float>(act_scale),
                                      nib.data_ptr<uint8_t>(), gs.data_ptr<float>(),
                                      gz.data_ptr<float>(),
                                      act_scale.has_value() ? inv.data_ptr<float>() : nullptr, N,
                                      K, group_size, stream_of(w)));
  return {nib, gs, gz, inv};
}

void kv_quantize_write(const at::Tensor& x, const at::Tensor& slots, at::Tensor& data,
                       at::Tensor& scale, const std::optional<at::Tensor>& smooth) {
  TORCH_CHECK(x.dim() == 3 && x.scalar_type() == at::kFloat && x.is_contiguous(),
              "kv_quantize_write: x must be a contiguous float32 [T, Hk, D] tensor");
  TORCH_CHECK(slots.dim() == 1 && slots.scalar_type() == at::kLong && slots.is_contiguous() &&
                  slots.size(0) == x.size(0),
              "kv_quantize_write: slots must be a contiguous int64 [T] tensor");
  TORCH_CHECK(data.dim() == 3 && data.scalar_type() == at::kChar && data.is_contiguous() &&
                  data.size(1) == x.size(1) && data.size(2) == x.size(2),
              "kv_quantize_write: data must be a contiguous int8 [slots, Hk, D] tensor");
  TORCH_CHECK(scale.dim() == 2 && scale.scalar_type() == at::kFloat && scale.is_contiguous() &&
                  scale.size(0) == data.size(0) && scale.size(1) == x.size(1),
              "kv_quantize_write: scale must be a contiguous float32 [slots, Hk] tensor");
  check_device(x, {&slots, &data, &scale}, "kv_quantize_write");
  if (smooth.has_value()) {
    check_device(x, {&*smooth}, "kv_quantize_write");
    TORCH_CHECK(smooth->scalar_type() == at::kFloat && smooth->is_contiguous() &&
                    smooth->numel() == x.size(1) * x.size(2),
                "kv_quantize_write: smooth must be a contiguous float32 [Hk, D] tensor");
  }
  const c10::DeviceGuard guard(x.device());
  check_status(llmserve_kv_quantize_write(x.data_ptr<float>(), slots.data_ptr<int64_t>(),
                                          opt_ptr<float>(smooth), data.data_ptr<int8_t>(),
                                          scale.data_ptr<float>(), x.size(0), x.size(1),
                                          x.size(2), data.size(0), stream_of(x)));
}

// ---- linears -------------------------------------------------------------------------------

at::Tensor int8_linear(const at::Tensor& x, const at::Tensor& qweight, const at::Tensor& scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat && qweight.scalar_type() == at::kChar &&
                  scale.scalar_type() == at::kFloat,
              "int8_linear: dtypes");
  TORCH_CHECK(x.is_contiguous() && qweight.is_contiguous() && scale.is_contiguous(),
              "int8_linear: contiguous inputs");
  TORCH_CHECK(x.dim() == 2 && qweight.dim() == 2, "int8_linear: 2-D x and qweight");
  check_device(x, {&qweight, &scale}, "int8_linear");
  const int64_t M = x.size(0), K = x.size(1), N = qweight.size(0);
  TORCH_CHECK(qweight.size(1) == K, "int8_linear: K mismatch");
  TORCH_CHECK(scale.numel() == N, "int8_linear: scale must have one entry per output channel");
  TORCH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int8_linear: meant for small batches (M <= 64)");
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({M, N}, x.options());
  check_status(llmserve_int8_linear(x.data_ptr<float>(), qweight.data_ptr<int8_t>(),
                                    scale.data_ptr<float>(), y.data_ptr<float>(), M, N, K,
                                    stream_of(x)));
  return y;
}

at::Tensor int8_linear_prefill(const at::Tensor& x, const at::Tensor& qweight,
                               const at::Tensor& scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat && qweight.scalar_type() == at::kChar &&
                  scale.scalar_type() == at::kFloat,
              "int8_linear_prefill: dtypes");
  TORCH_CHECK(x.is_contiguous() && qweight.is_contiguous() && scale.is_contiguous(),
              "int8_linear_prefill: contiguous inputs");
  TORCH_CHECK(x.dim() == 2 && qweight.dim() == 2, "int8_linear_prefill: 2-D x and qweight");
  check_device(x, {&qweight, &scale}, "int8_linear_prefill");
  const int64_t M = x.size(0), K = x.size(1), N = qweight.size(0);
  TORCH_CHECK(qweight.size(1) == K, "int8_linear_prefill: K mismatch");
  TORCH_CHECK(scale.numel() == N,
              "int8_linear_prefill: scale must have one entry per output channel");
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({M, N}, x.options());
  const int64_t ws_bytes = llmserve_int8_linear_prefill_workspace_bytes(M, N, K);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(ws_bytes + 15) / 16 * 4}, x.options());
  check_status(llmserve_int8_linear_prefill(
      x.data_ptr<float>(), qweight.data_ptr<int8_t>(), scale.data_ptr<float>(), y.data_ptr<float>(),
      M, N, K, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(x)));
  return y;
}

at::Tensor int4_linear(const at::Tensor& x, const at::Tensor& nibbles, const at::Tensor& scale,
                       const at::Tensor& zero, int64_t group_size,
                       const std::optional<at::Tensor>& inv_act_scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat && nibbles.scalar_type() == at::kByte, "int4: dtypes");
  TORCH_CHECK(scale.scalar_type() == at::kFloat && zero.scalar_type() == at::kFloat, "int4: dtypes");
  TORCH_CHECK(x.is_contiguous() && nibbles.is_contiguous() && scale.is_contiguous() &&
                  zero.is_contiguous(),
              "int4: contiguous inputs");
  TORCH_CHECK(x.dim() == 2 && nibbles.dim() == 2, "int4: 2-D x and nibbles");
  check_device(x, {&nibbles, &scale, &zero}, "int4_linear");
  const int64_t M = x.size(0), K = x.size(1), N = nibbles.size(0);
  TORCH_CHECK(group_size > 0, "int4: shapes");
  const int64_t G = K / group_size;
  TORCH_CHECK(nibbles.size(1) * 2 == K && G * group_size == K && group_size % 2 == 0, "int4: shapes");
  TORCH_CHECK(scale.numel() == N * G && zero.numel() == N * G, "int4: scale/zero must be [N, G]");
  TORCH_CHECK(M <= LLMSERVE_GEMV_MAX_ROWS, "int4_linear: meant for small batches (M <= 64)");
  if (inv_act_scale.has_value()) {
    check_device(x, {&*inv_act_scale}, "int4_linear");
    TORCH_CHECK(inv_act_scale->scalar_type() == at::kFloat && inv_act_scale->is_contiguous() &&
                    inv_act_scale->numel() == K,
                "int4_linear: inv_act_scale must be a contiguous float32 [K] tensor");
  }
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({M, N}, x.options());
  check_status(llmserve_int4_linear(x.data_ptr<float>(), opt_ptr<float>(inv_act_scale),
                                    nibbles.data_ptr<uint8_t>(), scale.data_ptr<float>(),
                                    zero.data_ptr<float>(), y.data_ptr<float>(), M, N, K,
                                    group_size, stream_of(x)));
  return y;
}

at::Tensor int4_linear_gemm(const at::Tensor& x, const at::Tensor& nibbles, const at::Tensor& scale,
                            const at::Tensor& zero, int64_t group_size,
                            const std::optional<at::Tensor>& inv_act_scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat && nibbles.scalar_type() == at::kByte, "int4: dtypes");
  TORCH_CHECK(scale.scalar_type() == at::kFloat && zero.scalar_type() == at::kFloat, "int4: dtypes");
  TORCH_CHECK(x.is_contiguous() && nibbles.is_contiguous() && scale.is_contiguous() &&
                  zero.is_contiguous(),
              "int4: contiguous inputs");
  TORCH_CHECK(x.dim() == 2 && nibbles.dim() == 2, "int4: 2-D x and nibbles");
  check_device(x, {&nibbles, &scale, &zero}, "int4_linear_gemm");
  const int64_t M = x.size(0), K = x.size(1), N = nibbles.size(0);
  TORCH_CHECK(group_size > 0, "int4: shapes");
  const int64_t G = K / group_size;
  TORCH_CHECK(nibbles.size(1) * 2 == K && G * group_size == K, "int4: shapes");
  TORCH_CHECK(scale.numel() == N * G && zero.numel() == N * G, "int4: scale/zero must be [N, G]");
  if (inv_act_scale.has_value()) {
    check_device(x, {&*inv_act_scale}, "int4_linear_gemm");
    TORCH_CHECK(inv_act_scale->scalar_type() == at::kFloat && inv_act_scale->is_contiguous() &&
                    inv_act_scale->numel() == K,
                "int4_linear_gemm: inv_act_scale must be a contiguous float32 [K] tensor");
  }
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({M, N}, x.options());
  const int64_t ws_bytes = llmserve_int4_linear_gemm_workspace_bytes(M, K);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(ws_bytes + 15) / 16 * 4}, x.options());
  check_status(llmserve_int4_linear_gemm(
      x.data_ptr<float>(), opt_ptr<float>(inv_act_scale), nibbles.data_ptr<uint8_t>(),
      scale.data_ptr<float>(), zero.data_ptr<float>(), y.data_ptr<float>(), M, N, K, group_size,
      ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(x)));
  return y;
}

at::Tensor int4_gemm_pack(const at::Tensor& nibbles, const at::Tensor& scale,
                          const at::Tensor& zero, int64_t group_size) {
  TORCH_CHECK(nibbles.scalar_type() == at::kByte && scale.scalar_type() == at::kFloat &&
                  zero.scalar_type() == at::kFloat,
              "int4_gemm_pack: uint8 nibbles, float32 scale / zero");
  TORCH_CHECK(nibbles.is_contiguous() && scale.is_contiguous() && zero.is_contiguous() &&
                  nibbles.dim() == 2,
              "int4_gemm_pack: contiguous [N, K/2] nibbles and [N, G] scale / zero");
  check_device(nibbles, {&scale, &zero}, "int4_gemm_pack");
  const int64_t N = nibbles.size(0), K = nibbles.size(1) * 2;
  TORCH_CHECK(group_size > 0 && K % group_size == 0 && scale.numel() == N * (K / group_size) &&
                  zero.numel() == scale.numel(),
              "int4_gemm_pack: scale / zero must be [N, K / group_size]");
  const c10::DeviceGuard guard(nibbles.device());
  const int64_t bytes = llmserve_int4_gemm_pack_bytes(N, K, group_size);
  TORCH_CHECK(bytes > 0, "int4_gemm_pack: K and group_size must be multiples of 128");
  auto packed = at::empty({bytes}, nibbles.options());
  check_status(llmserve_int4_gemm_pack(nibbles.data_ptr<uint8_t>(), scale.data_ptr<float>(),
                                       zero.data_ptr<float>(), N, K, group_size, packed.data_ptr(),
                                       bytes, stream_of(nibbles)));
  return packed;
}

at::Tensor int4_linear_gemm_packed(const at::Tensor& x, const at::Tensor& packed, int64_t N,
                                   int64_t group_size,
                                   const std::optional<at::Tensor>& inv_act_scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat && x.is_contiguous() && x.dim() == 2,
              "int4_linear_gemm_packed: contiguous float32 [M, K] x");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.is_contiguous(),
              "int4_linear_gemm_packed: packed must come from int4_gemm_pack");
  check_device(x, {&packed}, "int4_linear_gemm_packed");
  const int64_t M = x.size(0), K = x.size(1);
  TORCH_CHECK(packed.numel() == llmserve_int4_gemm_pack_bytes(N, K, group_size),
              "int4_linear_gemm_packed: packed buffer does not match N, K, group_size");
  if (inv_act_scale.has_value()) {
    check_device(x, {&*inv_act_scale}, "int4_linear_gemm_packed");
    TORCH_CHECK(inv_act_scale->scalar_type() == at::kFloat && inv_act_scale->is_contiguous() &&
                    inv_act_scale->numel() == K,
                "int4_linear_gemm_packed: inv_act_scale must be a contiguous float32 [K] tensor");
  }
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({M, N}, x.options());
  const int64_t ws_bytes = llmserve_int4_linear_gemm_packed_workspace_bytes(M, K);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(ws_bytes + 15) / 16 * 4}, x.options());
  check_status(llmserve_int4_linear_gemm_packed(
      x.data_ptr<float>(), opt_ptr<float>(inv_act_scale), packed.data_ptr(), y.data_ptr<float>(),
      M, N, K, group_size, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(x)));
  return y;
}

// ---- decoder-layer elementwise ops (fused_ops.cpp:39-127) and decode glue --------------------

void check_f32(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat && t.is_contiguous(), name,
              ": contiguous float32 tensor expected");
}

at::Tensor rmsnorm(const at::Tensor& x, const at::Tensor& w, double eps) {
  check_f32(x, "x");
  check_f32(w, "w");
  check_device(x, {&w}, "rmsnorm");
  const int64_t H = x.size(-1), T = x.numel() / H;
  TORCH_CHECK(w.numel() == H, "rmsnorm: weight must have x.size(-1) entries");
  const c10::DeviceGuard guard(x.device());
  auto out = at::empty_like(x);
  check_status(llmserve_rmsnorm(x.data_ptr<float>(), w.data_ptr<float>(), out.data_ptr<float>(), T,
                                H, static_cast<float>(eps), stream_of(x)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> embed_rmsnorm(const at::Tensor& ids, const at::Tensor& embed,
                                                 const at::Tensor& w, double eps) {
  check_f32(embed, "embed");
  check_f32(w, "w");
  TORCH_CHECK(ids.scalar_type() == at::kLong && ids.is_contiguous() && ids.dim() == 1,
              "embed_rmsnorm: ids must be a contiguous int64 [T] tensor");
  check_device(embed, {&ids, &w}, "embed_rmsnorm");
  TORCH_CHECK(embed.dim() == 2, "embed_rmsnorm: embed must be [V, H]");
  const int64_t T = ids.numel(), V = embed.size(0), H = embed.size(1);
  TORCH_CHECK(w.numel() == H, "embed_rmsnorm: weight must have H entries");
  const c10::DeviceGuard guard(embed.device());
  auto x = at::empty({T, H}, embed.options());
  auto out = at::empty({T, H}, embed.options());
  check_status(llmserve_embed_rmsnorm(ids.data_ptr<int64_t>(), embed.data_ptr<float>(), V,
                                      w.data_ptr<float>(), x.data_ptr<float>(),
                                      out.data_ptr<float>(), T, H, static_cast<float>(eps),
                                      stream_of(embed)));
  return {x, out};
}

at::Tensor add_rmsnorm_(at::Tensor& x, const at::Tensor& r, const at::Tensor& w, double eps) {
  check_f32(x, "x");
  check_f32(r, "r");
  check_f32(w, "w");
  check_device(x, {&r, &w}, "add_rmsnorm_");
  TORCH_CHECK(x.sizes() == r.sizes(), "add_rmsnorm_: shape mismatch");
  const int64_t H = x.size(-1), T = x.numel() / H;
  TORCH_CHECK(w.numel() == H, "add_rmsnorm_: weight must have x.size(-1) entries");
  const c10::DeviceGuard guard(x.device());
  auto out = at::empty_like(x);
  check_status(llmserve_add_rmsnorm(x.data_ptr<float>(), r.data_ptr<float>(), w.data_ptr<float>(),
                                    out.data_ptr<float>(), T, H, static_cast<float>(eps),
                                    stream_of(x)));
  return out;
}

at::Tensor silu_mul(const at::Tensor& gate_up) {
  check_f32(gate_up, "gate_up");
  check_device(gate_up, {}, "silu_mul");
  TORCH_CHECK(gate_up.size(-1) % 2 == 0, "silu_mul: last dimension must be 2 * I");
  const int64_t I = gate_up.size(-1) / 2, T = gate_up.numel() / (2 * I);
  const c10::DeviceGuard guard(gate_up.device());
  auto out = at::empty({T, I}, gate_up.options());
  check_status(llmserve_silu_mul(gate_up.data_ptr<float>(), out.data_ptr<float>(), T, I,
                                 stream_of(gate_up)));
  return out;
}

void rope_qk_(at::Tensor& qkv, const at::Tensor& cos, const at::Tensor& sin, int64_t n_q,
              int64_t n_k, int64_t head_dim, const std::optional<at::Tensor>& q_w,
              const std::optional<at::Tensor>& k_w, double eps) {
  check_f32(qkv, "qkv");
  check_f32(cos, "cos");
  check_f32(sin, "sin");
  check_device(qkv, {&cos, &sin}, "rope_qk_");
  TORCH_CHECK(qkv.dim() == 2, "rope_qk_: qkv must be [T, row]");
  const int64_t T = qkv.size(0), row = qkv.size(1);
  TORCH_CHECK(row >= (n_q + n_k) * head_dim && cos.numel() == T * head_dim &&
                  sin.numel() == T * head_dim,
              "rope_qk_: bad shapes");
  for (const auto* w : {&q_w, &k_w})
    if (w->has_value()) {
      check_f32(**w, "norm weight");
      check_device(qkv, {&**w}, "rope_qk_");
      TORCH_CHECK((*w)->numel() == head_dim, "rope_qk_: norm weights must have head_dim entries");
    }
  const c10::DeviceGuard guard(qkv.device());
  check_status(llmserve_rope_qk(qkv.data_ptr<float>(), cos.data_ptr<float>(), sin.data_ptr<float>(),
                                T, row, n_q, n_k, head_dim, opt_ptr<float>(q_w), opt_ptr<float>(k_w),
                                static_cast<float>(eps), stream_of(qkv)));
}

at::Tensor decode_qkv_kv(const at::Tensor& qkv, const at::Tensor& cos_table,
                         const at::Tensor& sin_table, const at::Tensor& context_lens,
                         const at::Tensor& block_tables, int64_t block_size,
                         const std::optional<at::Tensor>& q_w, const std::optional<at::Tensor>& k_w,
                         double eps, const std::optional<at::Tensor>& k_smooth, at::Tensor& k_cache,
                         at::Tensor& v_cache, at::Tensor& k_scale, at::Tensor& v_scale, int64_t n_q,
                         int64_t n_k, int64_t head_dim) {
  check_f32(qkv, "qkv");
  check_f32(cos_table, "cos_table");
  check_f32(sin_table, "sin_table");
  check_f32(k_scale, "k_scale");
  check_f32(v_scale, "v_scale");
  TORCH_CHECK(context_lens.scalar_type() == at::kLong && block_tables.scalar_type() == at::kLong &&
                  context_lens.is_contiguous() && block_tables.is_contiguous(),
              "decode_qkv_kv: int64 contiguous context_lens / block_tables");
  TORCH_CHECK(k_cache.scalar_type() == at::kChar && v_cache.scalar_type() == at::kChar &&
                  k_cache.is_contiguous() && v_cache.is_contiguous(),
              "decode_qkv_kv: int8 contiguous caches");
  check_device(qkv, {&cos_table, &sin_table, &context_lens, &block_tables, &k_cache, &v_cache,
                     &k_scale, &v_scale},
               "decode_qkv_kv");
  TORCH_CHECK(qkv.dim() == 2 && block_tables.dim() == 2, "decode_qkv_kv: 2-D qkv and block_tables");
  const int64_t T = qkv.size(0);
  TORCH_CHECK(context_lens.numel() == T && block_tables.size(0) == T,
              "decode_qkv_kv: one context length and block-table row per token");
  TORCH_CHECK(cos_table.dim() == 2 && cos_table.size(1) == head_dim &&
                  sin_table.sizes() == cos_table.sizes(),
              "decode_qkv_kv: cos/sin tables must be [max_pos, head_dim]");
  TORCH_CHECK(k_cache.dim() == 3 && k_cache.size(1) == n_k && k_cache.size(2) == head_dim &&
                  v_cache.sizes() == k_cache.sizes() && k_scale.numel() == k_cache.size(0) * n_k &&
                  v_scale.numel() == k_scale.numel(),
              "decode_qkv_kv: caches must be [num_slots, n_k, head_dim], scales [num_slots, n_k]");
  for (const auto* w : {&q_w, &k_w, &k_smooth})
    if (w->has_value()) {
      check_f32(**w, "weight");
      check_device(qkv, {&**w}, "decode_qkv_kv");
    }
  TORCH_CHECK((!q_w.has_value() || q_w->numel() == head_dim) &&
                  (!k_w.has_value() || k_w->numel() == head_dim),
              "decode_qkv_kv: q/k norm weights must have head_dim entries");
  TORCH_CHECK(!k_smooth.has_value() || k_smooth->numel() == n_k * head_dim,
              "decode_qkv_kv: k_smooth must be [n_k, head_dim]");
  TORCH_CHECK(qkv.size(1) >= (n_q + 2 * n_k) * head_dim,
              "decode_qkv_kv: qkv rows hold fewer than (n_q + 2 n_k) * head_dim values");
  const c10::DeviceGuard guard(qkv.device());
  auto q_out = at::empty({T, n_q, head_dim}, qkv.options());
  check_status(llmserve_decode_qkv_kv(
      qkv.data_ptr<float>(), qkv.size(1), cos_table.data_ptr<float>(), sin_table.data_ptr<float>(),
      cos_table.size(0), context_lens.data_ptr<int64_t>(), block_tables.data_ptr<int64_t>(),
      block_tables.size(1), block_size, opt_ptr<float>(q_w), opt_ptr<float>(k_w),
      static_cast<float>(eps), opt_ptr<float>(k_smooth), q_out.data_ptr<float>(),
      k_cache.data_ptr<int8_t>(), v_cache.data_ptr<int8_t>(), k_scale.data_ptr<float>(),
      v_scale.data_ptr<float>(), k_cache.size(0), T, n_q, n_k, head_dim, stream_of(qkv)));
  return q_out;
}

at::Tensor argmax_advance(const at::Tensor& logits, at::Tensor& context_lens) {
  check_f32(logits, "logits");
  TORCH_CHECK(context_lens.scalar_type() == at::kLong && context_lens.is_contiguous(),
              "argmax_advance: int64 contiguous context_lens");
  check_device(logits, {&context_lens}, "argmax_advance");
  TORCH_CHECK(logits.dim() == 2 && context_lens.numel() == logits.size(0),
              "argmax_advance: logits [T, V] and T context lengths");
  const c10::DeviceGuard guard(logits.device());
  const int64_t T = logits.size(0), V = logits.size(1);
  auto ids = at::empty({T}, context_lens.options());
  const int64_t ws_bytes = llmserve_argmax_advance_workspace_bytes(T);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(ws_bytes + 15) / 16 * 4}, logits.options());
  check_status(llmserve_argmax_advance(logits.data_ptr<float>(), T, V, ids.data_ptr<int64_t>(),
                                       context_lens.data_ptr<int64_t>(),
                                       ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                       stream_of(logits)));
  return ids;
}

// ---- activation fragments of the packed int4 linear --------------------------------------------

at::Tensor new_xfrag(const at::Tensor& like, int64_t T, int64_t K, const char* what) {
  const int64_t bytes = llmserve_int4_xfrag_bytes(T, K);
  TORCH_CHECK(bytes > 0, what, ": the channel count must be a multiple of 128");
  return at::empty({bytes}, like.options().dtype(at::kByte));
}

void check_act_inv(const at::Tensor& x, const std::optional<at::Tensor>& act_inv, int64_t K,
                   const char* what) {
  if (!act_inv.has_value()) return;
  check_device(x, {&*act_inv}, what);
  TORCH_CHECK(act_inv->scalar_type() == at::kFloat && act_inv->is_contiguous() &&
                  act_inv->numel() == K,
              what, ": act_inv must be a contiguous float32 tensor with one entry per channel");
}

at::Tensor add_rmsnorm_xfrag_(at::Tensor& x, const at::Tensor& r, const at::Tensor& w,
                              const std::optional<at::Tensor>& act_inv, double eps) {
  check_f32(x, "x");
  check_f32(r, "r");
  check_f32(w, "w");
  check_device(x, {&r, &w}, "add_rmsnorm_xfrag_");
  // r [T, H], or [P, T, H]: the output planes of a K-split linear, added in plane order
  TORCH_CHECK(x.dim() == 2 && ((r.dim() == 2 && r.sizes() == x.sizes()) ||
                               (r.dim() == 3 && r.size(1) == x.size(0) && r.size(2) == x.size(1))),
              "add_rmsnorm_xfrag_: x [T, H], r [T, H] or [P, T, H]");
  const int64_t T = x.size(0), H = x.size(1);
  TORCH_CHECK(w.numel() == H, "add_rmsnorm_xfrag_: weight must have H entries");
  check_act_inv(x, act_inv, H, "add_rmsnorm_xfrag_");
  const c10::DeviceGuard guard(x.device());
  auto xf = new_xfrag(x, T, H, "add_rmsnorm_xfrag_");
  if (r.dim() == 3)
    check_status(llmserve_add_rmsnorm_split_xfrag(
        x.data_ptr<float>(), r.data_ptr<float>(), r.size(0), w.data_ptr<float>(),
        opt_ptr<float>(act_inv), xf.data_ptr(), T, H, static_cast<float>(eps), stream_of(x)));
  else
    check_status(llmserve_add_rmsnorm_xfrag(x.data_ptr<float>(), r.data_ptr<float>(),
                                            w.data_ptr<float>(), opt_ptr<float>(act_inv),
                                            xf.data_ptr(), T, H, static_cast<float>(eps),
                                            stream_of(x)));
  return xf;
}

std::tuple<at::Tensor, at::Tensor> embed_rmsnorm_xfrag(const at::Tensor& ids,
                                                       const at::Tensor& embed, const at::Tensor& w,
                                                       const std::optional<at::Tensor>& act_inv,
                                                       double eps) {
  check_f32(embed, "embed");
  check_f32(w, "w");
  TORCH_CHECK(ids.scalar_type() == at::kLong && ids.is_contiguous() && ids.dim() == 1,
              "embed_rmsnorm_xfrag: ids must be a contiguous int64 [T] tensor");
  check_device(embed, {&ids, &w}, "embed_rmsnorm_xfrag");
  TORCH_CHECK(embed.dim() == 2, "embed_rmsnorm_xfrag: embed must be [V, H]");
  const int64_t T = ids.numel(), V = embed.size(0), H = embed.size(1);
  TORCH_CHECK(w.numel() == H, "embed_rmsnorm_xfrag: weight must have H entries");
  check_act_inv(embed, act_inv, H, "embed_rmsnorm_xfrag");
  const c10::DeviceGuard guard(embed.device());
  auto x = at::empty({T, H}, embed.options());
  auto xf = new_xfrag(embed, T, H, "embed_rmsnorm_xfrag");
  check_status(llmserve_embed_rmsnorm_xfrag(ids.data_ptr<int64_t>(), embed.data_ptr<float>(), V,
                                            w.data_ptr<float>(), opt_ptr<float>(act_inv),
                                            x.data_ptr<float>(), xf.data_ptr(), T, H,
                                            static_cast<float>(eps), stream_of(embed)));
  return {x, xf};
}

at::Tensor silu_mul_xfrag(const at::Tensor& gate_up, const std::optional<at::Tensor>& act_inv) {
  check_f32(gate_up, "gate_up");
  TORCH_CHECK(gate_up.dim() == 2 && gate_up.size(1) % 2 == 0, "silu_mul_xfrag: gate_up [T, 2I]");
  const int64_t T = gate_up.size(0), I = gate_up.size(1) / 2;
  check_act_inv(gate_up, act_inv, I, "silu_mul_xfrag");
  const c10::DeviceGuard guard(gate_up.device());
  auto xf = new_xfrag(gate_up, T, I, "silu_mul_xfrag");
  check_status(llmserve_silu_mul_xfrag(gate_up.data_ptr<float>(), opt_ptr<float>(act_inv),
                                       xf.data_ptr(), T, I, stream_of(gate_up)));
  return xf;
}

at::Tensor int4_linear_gemm_xfrag(const at::Tensor& xfrag, const at::Tensor& packed, int64_t M,
                                  int64_t N, int64_t K, int64_t group_size) {
  TORCH_CHECK(xfrag.scalar_type() == at::kByte && xfrag.is_contiguous() &&
                  xfrag.numel() == llmserve_int4_xfrag_bytes(M, K),
              "int4_linear_gemm_xfrag: xfrag must hold the fragments of [M, K]");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.is_contiguous() &&
                  packed.numel() == llmserve_int4_gemm_pack_bytes(N, K, group_size),
              "int4_linear_gemm_xfrag: packed buffer does not match N, K, group_size");
  check_device(xfrag, {&packed}, "int4_linear_gemm_xfrag");
  const c10::DeviceGuard guard(xfrag.device());
  auto y = at::empty({M, N}, xfrag.options().dtype(at::kFloat));
  check_status(llmserve_int4_linear_gemm_xfrag(xfrag.data_ptr(), packed.data_ptr(),
                                               y.data_ptr<float>(), M, N, K, group_size,
                                               stream_of(xfrag)));
  return y;
}

// The same linear with K split into `splits` output planes [splits, M, N] (their sum, in plane
// order, is the linear's output).
at::Tensor int4_linear_gemm_xfrag_split(const at::Tensor& xfrag, const at::Tensor& packed,
                                        int64_t M, int64_t N, int64_t K, int64_t group_size,
                                        int64_t splits) {
  TORCH_CHECK(xfrag.scalar_type() == at::kByte && xfrag.is_contiguous() &&
                  xfrag.numel() == llmserve_int4_xfrag_bytes(M, K),
              "int4_linear_gemm_xfrag_split: xfrag must hold the fragments of [M, K]");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.is_contiguous() &&
                  packed.numel() == llmserve_int4_gemm_pack_bytes(N, K, group_size),
              "int4_linear_gemm_xfrag_split: packed buffer does not match N, K, group_size");
  check_device(xfrag, {&packed}, "int4_linear_gemm_xfrag_split");
  const c10::DeviceGuard guard(xfrag.device());
  auto y = at::empty({splits, M, N}, xfrag.options().dtype(at::kFloat));
  check_status(llmserve_int4_linear_gemm_xfrag_split(xfrag.data_ptr(), packed.data_ptr(),
                                                     y.data_ptr<float>(), M, N, K, group_size,
                                                     splits, stream_of(xfrag)));
  return y;
}

int64_t int4_xfrag_splits(int64_t M, int64_t N, int64_t K) {
  return llmserve_int4_xfrag_splits(M, N, K);
}

// ---- int8-KV paged decode -------------------------------------------------------------------

at::Tensor lm_head_f32(const at::Tensor& x, const at::Tensor& w) {
  check_f32(x, "x");
  TORCH_CHECK(w.scalar_type() == at::kFloat && w.is_contiguous() && w.dim() == 2,
              "lm_head_f32: w must be a contiguous float32 [V, K] tensor");
  check_device(x, {&w}, "lm_head_f32");
  TORCH_CHECK(x.dim() == 2 && x.size(1) == w.size(1), "lm_head_f32: x [M, K] and w [V, K]");
  const c10::DeviceGuard guard(x.device());
  auto y = at::empty({x.size(0), w.size(0)}, x.options());
  check_status(llmserve_lm_head_f32(x.data_ptr<float>(), w.data_ptr<float>(), y.data_ptr<float>(),
                                    x.size(0), w.size(0), w.size(1), stream_of(x)));
  return y;
}

at::Tensor lm_head_f32_xfrag(const at::Tensor& xfrag, const at::Tensor& w, int64_t M) {
  TORCH_CHECK(xfrag.scalar_type() == at::kByte && xfrag.is_contiguous(),
              "lm_head_f32_xfrag: xfrag must be a contiguous uint8 fragment buffer");
  TORCH_CHECK(w.scalar_type() == at::kFloat && w.is_contiguous() && w.dim() == 2,
              "lm_head_f32_xfrag: w must be a contiguous float32 [V, K] tensor");
  check_device(w, {&xfrag}, "lm_head_f32_xfrag");
  const int64_t V = w.size(0), K = w.size(1);
  TORCH_CHECK(M >= 0 && xfrag.numel() >= llmserve_int4_xfrag_bytes(M, K),
              "lm_head_f32_xfrag: xfrag holds fewer than M rows of K channels");
  const c10::DeviceGuard guard(w.device());
  auto y = at::empty({M, V}, w.options());
  check_status(llmserve_lm_head_f32_xfrag(xfrag.data_ptr(), w.data_ptr<float>(),
                                          y.data_ptr<float>(), M, V, K, stream_of(w)));
  return y;
}

// Checks of the paged decode's tensors (dtypes, shapes, devices, contiguity).
void check_paged(const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                 const at::Tensor& k_scale, const at::Tensor& v_scale,
                 const at::Tensor& block_tables, const at::Tensor& context_lens,
                 const std::optional<at::Tensor>& q_mult) {
  TORCH_CHECK(k_cache.scalar_type() == at::kChar && v_cache.scalar_type() == at::kChar,
              "paged_attention_decode_int8: int8 cache");
  TORCH_CHECK(k_scale.scalar_type() == at::kFloat && v_scale.scalar_type() == at::kFloat &&
                  k_scale.is_contiguous() && v_scale.is_contiguous(),
              "paged_attention_decode_int8: float32 contiguous scales [num_slots, Hk]");
  TORCH_CHECK(q.scalar_type() == at::kFloat, "paged_attention: q must be float32");
  TORCH_CHECK(block_tables.scalar_type() == at::kLong && context_lens.scalar_type() == at::kLong,
              "paged_attention: int64 block tables / context lens");
  TORCH_CHECK(q.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous() &&
                  block_tables.is_contiguous() && context_lens.is_contiguous(),
              "paged_attention: inputs must be contiguous");
  TORCH_CHECK(q.dim() == 3 && k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes(),
              "paged_attention: q [B, Hq, D], caches [num_slots, Hk, D]");
  TORCH_CHECK(block_tables.dim() == 2 && context_lens.dim() == 1 &&
                  block_tables.size(0) == q.size(0) && context_lens.size(0) == q.size(0),
              "paged_attention: block_tables [B, max_blocks], context_lens [B]");
  check_device(q, {&k_cache, &v_cache, &k_scale, &v_scale, &block_tables, &context_lens},
               "paged_attention_decode_int8");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t num_slots = k_cache.size(0), Hk = k_cache.size(1);
  TORCH_CHECK(k_cache.size(2) == D, "paged_attention: head_dim mismatch");
  TORCH_CHECK(k_scale.numel() == num_slots * Hk && v_scale.numel() == num_slots * Hk,
              "paged_attention_decode_int8: float32 contiguous scales [num_slots, Hk]");
  if (q_mult.has_value()) {
    check_device(q, {&*q_mult}, "paged_attention_decode_int8");
    TORCH_CHECK(q_mult->scalar_type() == at::kFloat && q_mult->is_contiguous() &&
                    q_mult->numel() == Hq * D,
                "paged_attention_decode_int8: q_mult must be a contiguous float32 [Hq, D] tensor");
  }
}

at::Tensor paged_workspace(const at::Tensor& q, const at::Tensor& k_cache,
                           const at::Tensor& block_tables, int64_t block_size,
                           int64_t partition_size, int64_t& ws_bytes) {
  ws_bytes = llmserve_paged_attention_workspace_bytes(q.size(0), q.size(1), k_cache.size(1),
                                                      q.size(2), block_tables.size(1), block_size,
                                                      partition_size);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes / 4}, q.options());
  return ws;
}

at::Tensor paged_attention_decode_int8(const at::Tensor& q, const at::Tensor& k_cache,
                                       const at::Tensor& v_cache, const at::Tensor& k_scale,
                                       const at::Tensor& v_scale, const at::Tensor& block_tables,
                                       const at::Tensor& context_lens, int64_t block_size,
                                       double scale, int64_t partition_size,
                                       const std::optional<at::Tensor>& q_mult) {
  check_paged(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, q_mult);
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t num_slots = k_cache.size(0), Hk = k_cache.size(1);
  const c10::DeviceGuard guard(q.device());
  auto out = at::empty_like(q);
  if (B == 0) return out;
  const int64_t max_blocks = block_tables.size(1);
  int64_t ws_bytes = 0;
  at::Tensor ws = paged_workspace(q, k_cache, block_tables, block_size, partition_size, ws_bytes);
  check_status(llmserve_paged_attention_decode_int8(
      q.data_ptr<float>(), k_cache.data_ptr<int8_t>(), v_cache.data_ptr<int8_t>(),
      k_scale.data_ptr<float>(), v_scale.data_ptr<float>(), block_tables.data_ptr<int64_t>(),
      context_lens.data_ptr<int64_t>(), out.data_ptr<float>(), B, Hq, Hk, D, num_slots,
      max_blocks, block_size, static_cast<float>(scale), partition_size, opt_ptr<float>(q_mult),
      ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> paged_attention_decode_int8_xfrag(
    const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
    const at::Tensor& k_scale, const at::Tensor& v_scale, const at::Tensor& block_tables,
    const at::Tensor& context_lens, int64_t block_size, double scale, int64_t partition_size,
    const std::optional<at::Tensor>& q_mult, const std::optional<at::Tensor>& act_inv) {
  check_paged(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens, q_mult);
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t num_slots = k_cache.size(0), Hk = k_cache.size(1);
  TORCH_CHECK(D == 128 || D == 256, "paged_attention_decode_int8_xfrag: head_dim 128 or 256");
  check_act_inv(q, act_inv, Hq * D, "paged_attention_decode_int8_xfrag");
  const c10::DeviceGuard guard(q.device());
  auto out = at::empty_like(q);
  auto xf = new_xfrag(q, B, Hq * D, "paged_attention_decode_int8_xfrag");
  if (B == 0) return {out, xf};
  int64_t ws_bytes = 0;
  at::Tensor ws = paged_workspace(q, k_cache, block_tables, block_size, partition_size, ws_bytes);
  check_status(llmserve_paged_attention_decode_int8_xfrag(
      q.data_ptr<float>(), k_cache.data_ptr<int8_t>(), v_cache.data_ptr<int8_t>(),
      k_scale.data_ptr<float>(), v_scale.data_ptr<float>(), block_tables.data_ptr<int64_t>(),
      context_lens.data_ptr<int64_t>(), out.data_ptr<float>(), opt_ptr<float>(act_inv),
      xf.data_ptr(), B, Hq, Hk, D, num_slots, block_tables.size(1), block_size,
      static_cast<float>(scale), partition_size, opt_ptr<float>(q_mult),
      ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
  return {out, xf};
}

// The reference's fp32-cache decode (paged_attention.cpp:350-359, :386-390).
at::Tensor paged_attention_decode(const at::Tensor& q, const at::Tensor& k_cache,
                                  const at::Tensor& v_cache, const at::Tensor& block_tables,
                                  const at::Tensor& context_lens, int64_t block_size, double scale,
                                  int64_t partition_size) {
  TORCH_CHECK(k_cache.scalar_type() == at::kFloat && v_cache.scalar_type() == at::kFloat,
              "paged_attention_decode: float32 cache");
  TORCH_CHECK(q.scalar_type() == at::kFloat, "paged_attention: q must be float32");
  TORCH_CHECK(block_tables.scalar_type() == at::kLong && context_lens.scalar_type() == at::kLong,
              "paged_attention_decode: int64 block tables / context lens");
  TORCH_CHECK(q.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous() &&
                  block_tables.is_contiguous() && context_lens.is_contiguous(),
              "paged_attention_decode: inputs must be contiguous");
  TORCH_CHECK(q.dim() == 3 && k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes() &&
                  k_cache.size(2) == q.size(2),
              "paged_attention: q [B, Hq, D], caches [num_slots, Hk, D]");
  TORCH_CHECK(block_tables.dim() == 2 && context_lens.dim() == 1 &&
                  block_tables.size(0) == q.size(0) && context_lens.size(0) == q.size(0),
              "paged_attention: block_tables [B, max_blocks], context_lens [B]");
  check_device(q, {&k_cache, &v_cache, &block_tables, &context_lens}, "paged_attention_decode");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const c10::DeviceGuard guard(q.device());
  auto out = at::empty_like(q);
  if (B == 0) return out;
  int64_t ws_bytes = 0;
  at::Tensor ws = paged_workspace(q, k_cache, block_tables, block_size, partition_size, ws_bytes);
  check_status(llmserve_paged_attention_decode(
      q.data_ptr<float>(), k_cache.data_ptr<float>(), v_cache.data_ptr<float>(),
      block_tables.data_ptr<int64_t>(), context_lens.data_ptr<int64_t>(), out.data_ptr<float>(),
      B, Hq, k_cache.size(1), D, k_cache.size(0), block_tables.size(1), block_size,
      static_cast<float>(scale), partition_size, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
      stream_of(q)));
  return out;
}

// Attention over the query rows of a ragged batch (decode and prefill rows alike) for an int8
// (k_scale / v_scale given) or float32 (no scales) cache.
at::Tensor paged_attention_rows(const at::Tensor& q, const at::Tensor& k_cache,
                                const at::Tensor& v_cache, const std::optional<at::Tensor>& k_scale,
                                const std::optional<at::Tensor>& v_scale,
                                const at::Tensor& block_tables, const at::Tensor& row_table,
                                const at::Tensor& row_context, int64_t block_size, double scale,
                                const std::optional<at::Tensor>& q_mult) {
  const bool int8 = k_cache.scalar_type() == at::kChar;
  TORCH_CHECK(int8 || k_cache.scalar_type() == at::kFloat,
              "paged_attention_rows: int8 or float32 cache");
  TORCH_CHECK(v_cache.scalar_type() == k_cache.scalar_type() && v_cache.sizes() == k_cache.sizes(),
              "paged_attention_rows: K and V caches of one type and shape");
  TORCH_CHECK(int8 == (k_scale.has_value() && v_scale.has_value()),
              "paged_attention_rows: an int8 cache takes k_scale and v_scale, a float32 one none");
  TORCH_CHECK(q.scalar_type() == at::kFloat && q.dim() == 3 && q.is_contiguous(),
              "paged_attention_rows: q must be a contiguous float32 [R, Hq, D] tensor");
  TORCH_CHECK(k_cache.dim() == 3 && k_cache.size(2) == q.size(2) && k_cache.is_contiguous() &&
                  v_cache.is_contiguous(),
              "paged_attention_rows: caches must be contiguous [num_slots, Hk, D]");
  for (const at::Tensor* t : {&block_tables, &row_table, &row_context})
    TORCH_CHECK(t->scalar_type() == at::kLong && t->is_contiguous(),
                "paged_attention_rows: int64 contiguous tables");
  TORCH_CHECK(block_tables.dim() == 2 && row_table.numel() == q.size(0) &&
                  row_context.numel() == q.size(0),
              "paged_attention_rows: block_tables [S, max_blocks], one table row and context per "
              "query row");
  check_device(q, {&k_cache, &v_cache, &block_tables, &row_table, &row_context},
               "paged_attention_rows");
  const int64_t R = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t num_slots = k_cache.size(0), Hk = k_cache.size(1);
  if (int8) {
    check_device(q, {&*k_scale, &*v_scale}, "paged_attention_rows");
    TORCH_CHECK(k_scale->scalar_type() == at::kFloat && v_scale->scalar_type() == at::kFloat &&
                    k_scale->is_contiguous() && v_scale->is_contiguous() &&
                    k_scale->numel() == num_slots * Hk && v_scale->numel() == num_slots * Hk,
                "paged_attention_rows: float32 contiguous scales [num_slots, Hk]");
  }
  if (q_mult.has_value()) {
    check_device(q, {&*q_mult}, "paged_attention_rows");
    TORCH_CHECK(q_mult->scalar_type() == at::kFloat && q_mult->is_contiguous() &&
                    q_mult->numel() == Hq * D,
                "paged_attention_rows: q_mult must be a contiguous float32 [Hq, D] tensor");
  }
  const c10::DeviceGuard guard(q.device());
  auto out = at::empty_like(q);
  if (R == 0) return out;
  int64_t ws_bytes = 0;
  at::Tensor ws = paged_workspace(q, k_cache, block_tables, block_size, 0, ws_bytes);
  void* wsp = ws_bytes > 0 ? ws.data_ptr() : nullptr;
  if (int8)
    check_status(llmserve_paged_attention_rows_int8(
        q.data_ptr<float>(), k_cache.data_ptr<int8_t>(), v_cache.data_ptr<int8_t>(),
        k_scale->data_ptr<float>(), v_scale->data_ptr<float>(), block_tables.data_ptr<int64_t>(),
        block_tables.size(0), row_table.data_ptr<int64_t>(), row_context.data_ptr<int64_t>(),
        out.data_ptr<float>(), R, Hq, Hk, D, num_slots, block_tables.size(1), block_size,
        static_cast<float>(scale), opt_ptr<float>(q_mult), wsp, ws_bytes, stream_of(q)));
  else
    check_status(llmserve_paged_attention_rows_f32(
        q.data_ptr<float>(), k_cache.data_ptr<float>(), v_cache.data_ptr<float>(),
        block_tables.data_ptr<int64_t>(), block_tables.size(0), row_table.data_ptr<int64_t>(),
        row_context.data_ptr<int64_t>(), out.data_ptr<float>(), R, Hq, Hk, D, num_slots,
        block_tables.size(1), block_size, static_cast<float>(scale), opt_ptr<float>(q_mult), wsp,
        ws_bytes, stream_of(q)));
  return out;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> attention_metadata(const at::Tensor& seq_info,
                                                                  const at::Tensor& block_tables,
                                                                  int64_t block_size, int64_t T) {
  TORCH_CHECK(seq_info.scalar_type() == at::kLong && seq_info.is_contiguous() &&
                  seq_info.dim() == 2 && seq_info.size(0) == 3,
              "attention_metadata: seq_info must be a contiguous int64 [3, S] tensor");
  TORCH_CHECK(block_tables.scalar_type() == at::kLong && block_tables.is_contiguous() &&
                  block_tables.dim() == 2 && block_tables.size(0) == seq_info.size(1),
              "attention_metadata: block_tables must be a contiguous int64 [S, max_blocks] tensor");
  check_device(seq_info, {&block_tables}, "attention_metadata");
  const c10::DeviceGuard guard(seq_info.device());
  auto slots = at::empty({T}, seq_info.options());
  auto rows = at::empty({T}, seq_info.options());
  auto ctx = at::empty({T}, seq_info.options());
  check_status(llmserve_attention_metadata(
      seq_info.data_ptr<int64_t>(), block_tables.data_ptr<int64_t>(), seq_info.size(1),
      block_tables.size(1), block_size, T, slots.data_ptr<int64_t>(), rows.data_ptr<int64_t>(),
      ctx.data_ptr<int64_t>(), stream_of(seq_info)));
  return {slots, rows, ctx};
}

}  // namespace

TORCH_LIBRARY(llmserve_hip, m) {
  m.def("int8_quantize(Tensor w) -> (Tensor, Tensor)");
  m.def("int4_quantize(Tensor w, int group_size, Tensor? act_scale=None)"
        " -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("kv_quantize_write(Tensor x, Tensor slots, Tensor(a!) data, Tensor(b!) scale,"
        " Tensor? smooth=None) -> ()");
  m.def("int8_linear(Tensor x, Tensor qweight, Tensor scale) -> Tensor");
  m.def("int8_linear_prefill(Tensor x, Tensor qweight, Tensor scale) -> Tensor");
  m.def("int4_linear(Tensor x, Tensor nibbles, Tensor scale, Tensor zero, int group_size,"
        " Tensor? inv_act_scale=None) -> Tensor");
  m.def("int4_linear_gemm(Tensor x, Tensor nibbles, Tensor scale, Tensor zero, int group_size,"
        " Tensor? inv_act_scale=None) -> Tensor");
  m.def("int4_gemm_pack(Tensor nibbles, Tensor scale, Tensor zero, int group_size) -> Tensor");
  m.def("int4_linear_gemm_packed(Tensor x, Tensor packed, int out_features, int group_size,"
        " Tensor? inv_act_scale=None) -> Tensor");
  m.def("rmsnorm(Tensor x, Tensor w, float eps) -> Tensor");
  m.def("add_rmsnorm_(Tensor(a!) x, Tensor r, Tensor w, float eps) -> Tensor");
  m.def("embed_rmsnorm(Tensor ids, Tensor embed, Tensor w, float eps) -> (Tensor, Tensor)");
  m.def("add_rmsnorm_xfrag_(Tensor(a!) x, Tensor r, Tensor w, Tensor? act_inv, float eps) -> Tensor");
  m.def("embed_rmsnorm_xfrag(Tensor ids, Tensor embed, Tensor w, Tensor? act_inv, float eps)"
        " -> (Tensor, Tensor)");
  m.def("silu_mul_xfrag(Tensor gate_up, Tensor? act_inv) -> Tensor");
  m.def("int4_linear_gemm_xfrag(Tensor xfrag, Tensor packed, int M, int N, int K, int group_size)"
        " -> Tensor");
  m.def("int4_linear_gemm_xfrag_split(Tensor xfrag, Tensor packed, int M, int N, int K,"
        " int group_size, int splits) -> Tensor");
  m.def("int4_xfrag_splits(int M, int N, int K) -> int", &int4_xfrag_splits);
  m.def("silu_mul(Tensor gate_up) -> Tensor");
  m.def("lm_head_f32_xfrag(Tensor xfrag, Tensor w, int M) -> Tensor");
  m.def("lm_head_f32(Tensor x, Tensor w) -> Tensor");
  m.def("rope_qk_(Tensor(a!) qkv, Tensor cos, Tensor sin, int n_q, int n_k, int head_dim,"
        " Tensor? q_w=None, Tensor? k_w=None, float eps=1e-6) -> ()");
  m.def("decode_qkv_kv(Tensor qkv, Tensor cos_table, Tensor sin_table, Tensor context_lens,"
        " Tensor block_tables, int block_size, Tensor? q_w, Tensor? k_w, float eps,"
        " Tensor? k_smooth, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor(c!) k_scale,"
        " Tensor(d!) v_scale, int n_q, int n_k, int head_dim) -> Tensor");
  m.def("argmax_advance(Tensor logits, Tensor(a!) context_lens) -> Tensor");
  m.def("paged_attention_decode_int8(Tensor q, Tensor k_cache, Tensor v_cache, Tensor k_scale,"
        " Tensor v_scale, Tensor block_tables, Tensor context_lens, int block_size, float scale,"
        " int partition_size=0, Tensor? q_mult=None) -> Tensor");
  m.def("paged_attention_decode_int8_xfrag(Tensor q, Tensor k_cache, Tensor v_cache,"
        " Tensor k_scale, Tensor v_scale, Tensor block_tables, Tensor context_lens,"
        " int block_size, float scale, int partition_size=0, Tensor? q_mult=None,"
        " Tensor? act_inv=None) -> (Tensor, Tensor)");
  m.def("paged_attention_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables,"
        " Tensor context_lens, int block_size, float scale, int partition_size=0) -> Tensor");
  m.def("paged_attention_rows(Tensor q, Tensor k_cache, Tensor v_cache, Tensor? k_scale,"
        " Tensor? v_scale, Tensor block_tables, Tensor row_table, Tensor row_context,"
        " int block_size, float scale, Tensor? q_mult=None) -> Tensor");
  m.def("attention_metadata(Tensor seq_info, Tensor block_tables, int block_size, int T)"
        " -> (Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(llmserve_hip, CUDA, m) {
  m.impl("int8_quantize", &int8_quantize);
  m.impl("int4_quantize", &int4_quantize);
  m.impl("kv_quantize_write", &kv_quantize_write);
  m.impl("int8_linear", &int8_linear);
  m.impl("int8_linear_prefill", &int8_linear_prefill);
  m.impl("int4_linear_gemm", &int4_linear_gemm);
  m.impl("int4_gemm_pack", &int4_gemm_pack);
  m.impl("int4_linear_gemm_packed", &int4_linear_gemm_packed);
  m.impl("int4_linear", &int4_linear);
  m.impl("rmsnorm", &rmsnorm);
  m.impl("add_rmsnorm_", &add_rmsnorm_);
  m.impl("embed_rmsnorm", &embed_rmsnorm);
  m.impl("add_rmsnorm_xfrag_", &add_rmsnorm_xfrag_);
  m.impl("int4_linear_gemm_xfrag_split", &int4_linear_gemm_xfrag_split);
  m.impl("embed_rmsnorm_xfrag", &embed_rmsnorm_xfrag);
  m.impl("silu_mul_xfrag", &silu_mul_xfrag);
  m.impl("int4_linear_gemm_xfrag", &int4_linear_gemm_xfrag);
  m.impl("silu_mul", &silu_mul);
  m.impl("lm_head_f32_xfrag", &lm_head_f32_xfrag);
  m.impl("lm_head_f32", &lm_head_f32);
  m.impl("rope_qk_", &rope_qk_);
  m.impl("decode_qkv_kv", &decode_qkv_kv);
  m.impl("argmax_advance", &argmax_advance);
  m.impl("paged_attention_decode_int8", &paged_attention_decode_int8);
  m.impl("paged_attention_decode_int8_xfrag", &paged_attention_decode_int8_xfrag);
  m.impl("paged_attention_decode", &paged_attention_decode);
  m.impl("paged_attention_rows", &paged_attention_rows);
  m.impl("attention_metadata", &attention_metadata);
}
