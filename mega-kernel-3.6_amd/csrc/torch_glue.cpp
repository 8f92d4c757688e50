// mega_kernel_qwen36._C -- thin PyTorch-ROCm binding over the libmkq C ABI.
//
// Replaces the reference's csrc/bindings.cpp:32-36 (and the host halves of
// persistent_moe_decode.cu:648-860, attention_decode.cu:150-218,
// linear_attention_decode.cu:44-93): validates tensors with the reference's
// TORCH_CHECK messages, allocates outputs on the tensors' device, and calls the
// C entry points on torch's current HIP stream.  No device queries and no
// synchronisation happen here; scratch memory comes from one cached, zeroed
// workspace per (device, stream).
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <map>
#include <tuple>
#include <utility>

#include "../../include/mkq.h"

#define MK_CHECK_CUDA(x) TORCH_CHECK((x).is_cuda(), #x " must be a CUDA tensor")
#define MK_CHECK_CONTIGUOUS(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define MK_CHECK_INPUT(x) \
  MK_CHECK_CUDA(x);       \
  MK_CHECK_CONTIGUOUS(x)

namespace {

int to_mkq_dtype(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kBFloat16:
      return MKQ_DTYPE_BF16;
    case torch::kHalf:
      return MKQ_DTYPE_F16;
    case torch::kFloat:
      return MKQ_DTYPE_F32;
    default:
      TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(), " (expected bfloat16, float16 or float32)");
  }
  return -1;
}

void check_status(int rc, const char* op) {
  TORCH_CHECK(rc == MKQ_OK, op, " failed (status ", rc, "): ", mkq_last_error());
}

hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

// One zero-filled workspace per (entry point, device, stream).  Kernels leave
// the state they keep there (counters, the MoE generation word) ready for the
// next call of the same entry point, so the buffer is cleared only when it is
// first allocated (or grown); entry points do not share one, since another
// entry point's scratch data would overwrite that state.
enum class Ws { kMoe, kDense, kAttention, kLinearStep };
std::map<std::tuple<int, int, hipStream_t>, torch::Tensor>& workspace_cache() {
  static std::map<std::tuple<int, int, hipStream_t>, torch::Tensor> cache;
  return cache;
}
torch::Tensor workspace_for(Ws op, const torch::Tensor& like, size_t bytes) {
  auto& cache = workspace_cache();
  const auto key = std::make_tuple(static_cast<int>(op), static_cast<int>(like.get_device()), current_stream());
  auto it = cache.find(key);
  if (it != cache.end() && static_cast<size_t>(it->second.numel()) >= bytes) return it->second;
  size_t grow = bytes < 4096 ? 4096 : bytes;
  if (it != cache.end()) grow = std::max(grow, static_cast<size_t>(it->second.numel()) * 2);
  auto ws = torch::zeros({static_cast<int64_t>(grow)}, like.options().dtype(torch::kUInt8));
  cache[key] = ws;
  return ws;
}

void check_moe_inputs(const torch::Tensor& x, const torch::Tensor& norm_weight, const torch::Tensor& router_weight,
                      const torch::Tensor& expert_gate, const torch::Tensor& expert_up,
                      const torch::Tensor& expert_down, const torch::Tensor& shared_gate,
                      const torch::Tensor& shared_up, const torch::Tensor& shared_down, int64_t top_k) {
  // Checks and messages as in the reference's check_moe_inputs
  // (persistent_moe_decode.cu:648-697).
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(norm_weight);
  MK_CHECK_INPUT(router_weight);
  MK_CHECK_INPUT(expert_gate);
  MK_CHECK_INPUT(expert_up);
  MK_CHECK_INPUT(expert_down);
  MK_CHECK_INPUT(shared_gate);
  MK_CHECK_INPUT(shared_up);
  MK_CHECK_INPUT(shared_down);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, hidden]");
  TORCH_CHECK(norm_weight.dim() == 1, "norm_weight must be [hidden]");
  TORCH_CHECK(router_weight.dim() == 2, "router_weight must be [experts, hidden]");
  TORCH_CHECK(expert_gate.dim() == 3, "expert_gate must be [experts, intermediate, hidden]");
  TORCH_CHECK(expert_up.sizes() == expert_gate.sizes(), "expert_up shape must match expert_gate");
  TORCH_CHECK(expert_down.dim() == 3, "expert_down must be [experts, hidden, intermediate]");
  TORCH_CHECK(shared_gate.dim() == 2, "shared_gate must be [shared_intermediate, hidden]");
  TORCH_CHECK(shared_up.sizes() == shared_gate.sizes(), "shared_up shape must match shared_gate");
  TORCH_CHECK(shared_down.dim() == 2, "shared_down must be [hidden, shared_intermediate]");
  TORCH_CHECK(x.scalar_type() == norm_weight.scalar_type(), "x and norm_weight dtype mismatch");
  TORCH_CHECK(x.scalar_type() == router_weight.scalar_type(), "x and router_weight dtype mismatch");
  TORCH_CHECK(x.scalar_type() == expert_gate.scalar_type(), "x and expert_gate dtype mismatch");
  TORCH_CHECK(x.scalar_type() == expert_up.scalar_type(), "x and expert_up dtype mismatch");
  TORCH_CHECK(x.scalar_type() == expert_down.scalar_type(), "x and expert_down dtype mismatch");
  TORCH_CHECK(x.scalar_type() == shared_gate.scalar_type(), "x and shared_gate dtype mismatch");
  TORCH_CHECK(x.scalar_type() == shared_up.scalar_type(), "x and shared_up dtype mismatch");
  TORCH_CHECK(x.scalar_type() == shared_down.scalar_type(), "x and shared_down dtype mismatch");
  const int64_t hidden = x.size(1);
  const int64_t experts = router_weight.size(0);
  const int64_t intermediate = expert_gate.size(1);
  const int64_t shared_intermediate = shared_gate.size(0);
  TORCH_CHECK(top_k > 0 && top_k <= experts, "top_k must be in [1, experts]");
  TORCH_CHECK(norm_weight.size(0) == hidden, "norm_weight hidden mismatch");
  TORCH_CHECK(router_weight.size(1) == hidden, "router_weight hidden mismatch");
  TORCH_CHECK(expert_gate.size(0) == experts && expert_gate.size(2) == hidden, "expert_gate shape mismatch");
  TORCH_CHECK(expert_down.size(0) == experts && expert_down.size(1) == hidden && expert_down.size(2) == intermediate,
              "expert_down shape mismatch");
  TORCH_CHECK(shared_gate.size(1) == hidden, "shared_gate hidden mismatch");
  TORCH_CHECK(shared_down.size(0) == hidden && shared_down.size(1) == shared_intermediate,
              "shared_down shape mismatch");
}

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> moe_impl(
    const torch::Tensor& x, const torch::Tensor& norm_weight, const torch::Tensor& router_weight,
    const torch::Tensor& expert_gate, const torch::Tensor& expert_up, const torch::Tensor& expert_down,
    const torch::Tensor& shared_gate, const torch::Tensor& shared_up, const torch::Tensor& shared_down,
    const torch::Tensor* shared_expert_gate, double eps, int64_t top_k, bool add_residual) {
  check_moe_inputs(x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate, shared_up,
                   shared_down, top_k);
  const int batch = static_cast<int>(x.size(0));
  const int hidden = static_cast<int>(x.size(1));
  const int experts = static_cast<int>(router_weight.size(0));
  const int intermediate = static_cast<int>(expert_gate.size(1));
  const int shared_intermediate = static_cast<int>(shared_gate.size(0));
  const void* sg_ptr = nullptr;
  if (shared_expert_gate != nullptr) {
    const torch::Tensor& sg = *shared_expert_gate;
    MK_CHECK_INPUT(sg);
    TORCH_CHECK(sg.numel() == hidden, "shared_expert_gate must be [hidden] or [1, hidden]");
    TORCH_CHECK(x.scalar_type() == sg.scalar_type(), "x and shared_expert_gate dtype mismatch");
    sg_ptr = sg.data_ptr();
  }
  c10::DeviceGuard guard(x.device());
  auto out = torch::empty_like(x);
  auto indices = torch::empty({batch, top_k}, x.options().dtype(torch::kInt64));
  auto weights = torch::empty({batch, top_k}, x.options().dtype(torch::kFloat32));
  const size_t ws_bytes =
      mkq_moe_decode_workspace_bytes(batch, hidden, experts, intermediate, shared_intermediate, static_cast<int>(top_k));
  auto ws = workspace_for(Ws::kMoe, x, ws_bytes);
  const int rc = mkq_moe_decode(to_mkq_dtype(x), x.data_ptr(), norm_weight.data_ptr(), router_weight.data_ptr(),
                                expert_gate.data_ptr(), expert_up.data_ptr(), expert_down.data_ptr(),
                                shared_gate.data_ptr(), shared_up.data_ptr(), shared_down.data_ptr(), sg_ptr,
                                out.data_ptr(), indices.data_ptr<int64_t>(), weights.data_ptr<float>(), batch, hidden,
                                experts, intermediate, shared_intermediate, static_cast<int>(top_k),
                                static_cast<float>(eps), add_residual ? 1 : 0, ws.data_ptr(),
                                static_cast<size_t>(ws.numel()), current_stream());
  check_status(rc, "moe_decode_persistent");
  return std::make_tuple(out, indices, weights);
}

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> moe_decode_persistent(
    torch::Tensor x, torch::Tensor norm_weight, torch::Tensor router_weight, torch::Tensor expert_gate,
    torch::Tensor expert_up, torch::Tensor expert_down, torch::Tensor shared_gate, torch::Tensor shared_up,
    torch::Tensor shared_down, double eps, int64_t top_k, bool add_residual) {
  return moe_impl(x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate, shared_up,
                  shared_down, nullptr, eps, top_k, add_residual);
}

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> moe_decode_persistent_gated(
    torch::Tensor x, torch::Tensor norm_weight, torch::Tensor router_weight, torch::Tensor expert_gate,
    torch::Tensor expert_up, torch::Tensor expert_down, torch::Tensor shared_gate, torch::Tensor shared_up,
    torch::Tensor shared_down, torch::Tensor shared_expert_gate, double eps, int64_t top_k, bool add_residual) {
  return moe_impl(x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate, shared_up,
                  shared_down, &shared_expert_gate, eps, top_k, add_residual);
}

torch::Tensor dense_ffn_decode(torch::Tensor x, torch::Tensor norm_weight, torch::Tensor gate_weight,
                               torch::Tensor up_weight, torch::Tensor down_weight, double eps, bool add_residual) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(norm_weight);
  MK_CHECK_INPUT(gate_weight);
  MK_CHECK_INPUT(up_weight);
  MK_CHECK_INPUT(down_weight);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, hidden]");
  TORCH_CHECK(norm_weight.dim() == 1, "norm_weight must be [hidden]");
  TORCH_CHECK(gate_weight.dim() == 2, "gate_weight must be [intermediate, hidden]");
  TORCH_CHECK(up_weight.sizes() == gate_weight.sizes(), "up_weight shape must match gate_weight");
  TORCH_CHECK(down_weight.dim() == 2, "down_weight must be [hidden, intermediate]");
  TORCH_CHECK(x.scalar_type() == norm_weight.scalar_type(), "x and norm_weight dtype mismatch");
  TORCH_CHECK(x.scalar_type() == gate_weight.scalar_type(), "x and gate_weight dtype mismatch");
  TORCH_CHECK(x.scalar_type() == up_weight.scalar_type(), "x and up_weight dtype mismatch");
  TORCH_CHECK(x.scalar_type() == down_weight.scalar_type(), "x and down_weight dtype mismatch");
  const int batch = static_cast<int>(x.size(0));
  const int hidden = static_cast<int>(x.size(1));
  const int intermediate = static_cast<int>(gate_weight.size(0));
  TORCH_CHECK(norm_weight.size(0) == hidden, "norm_weight hidden mismatch");
  TORCH_CHECK(gate_weight.size(1) == hidden, "gate_weight hidden mismatch");
  TORCH_CHECK(down_weight.size(0) == hidden && down_weight.size(1) == intermediate, "down_weight shape mismatch");
  c10::DeviceGuard guard(x.device());
  auto out = torch::empty_like(x);
  auto ws = workspace_for(Ws::kDense, x, mkq_dense_ffn_decode_workspace_bytes(batch, hidden, intermediate));
  const int rc = mkq_dense_ffn_decode(to_mkq_dtype(x), x.data_ptr(), norm_weight.data_ptr(), gate_weight.data_ptr(),
                                      up_weight.data_ptr(), down_weight.data_ptr(), out.data_ptr(), batch, hidden,
                                      intermediate, static_cast<float>(eps), add_residual ? 1 : 0, ws.data_ptr(),
                                      static_cast<size_t>(ws.numel()), current_stream());
  check_status(rc, "dense_ffn_decode");
  return out;
}

torch::Tensor attention_impl(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, double scale,
                             const torch::Tensor* cos_sin, int64_t rotary_dim) {
  // Checks and messages as in attention_decode.cu:157-175.
  MK_CHECK_INPUT(q);
  MK_CHECK_INPUT(k_cache);
  MK_CHECK_INPUT(v_cache);
  TORCH_CHECK(q.dim() == 3, "q must be [batch, query_heads, head_dim]");
  TORCH_CHECK(k_cache.dim() == 4, "k_cache must be [batch, seq_len, kv_heads, head_dim]");
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "v_cache shape must match k_cache");
  TORCH_CHECK(q.scalar_type() == k_cache.scalar_type(), "q and k_cache dtype mismatch");
  TORCH_CHECK(q.scalar_type() == v_cache.scalar_type(), "q and v_cache dtype mismatch");
  const int batch = static_cast<int>(q.size(0));
  const int query_heads = static_cast<int>(q.size(1));
  const int head_dim = static_cast<int>(q.size(2));
  const int seq_len = static_cast<int>(k_cache.size(1));
  const int kv_heads = static_cast<int>(k_cache.size(2));
  TORCH_CHECK(k_cache.size(0) == batch, "batch mismatch");
  TORCH_CHECK(k_cache.size(3) == head_dim, "head_dim mismatch");
  TORCH_CHECK(kv_heads > 0 && query_heads % kv_heads == 0, "query_heads must be divisible by kv_heads");
  TORCH_CHECK(head_dim <= 256, "head_dim > 256 is not supported by this kernel");
  TORCH_CHECK(seq_len > 0, "seq_len must be positive");
  c10::DeviceGuard guard(q.device());
  auto out = torch::empty_like(q);
  auto ws = workspace_for(Ws::kAttention, q, mkq_full_attention_decode_workspace_bytes(batch, query_heads, kv_heads, head_dim, seq_len));
  int rc;
  if (cos_sin == nullptr) {
    rc = mkq_full_attention_decode(to_mkq_dtype(q), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                   out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq_len,
                                   static_cast<float>(scale), ws.data_ptr(), static_cast<size_t>(ws.numel()),
                                   current_stream());
  } else {
    TORCH_CHECK(cos_sin->is_cuda() && cos_sin->is_contiguous() && cos_sin->scalar_type() == torch::kFloat32,
                "cos_sin must be a contiguous float32 device tensor");
    TORCH_CHECK(cos_sin->numel() == 2 * rotary_dim, "cos_sin must hold 2 * rotary_dim values");
    rc = mkq_full_attention_decode_rope(to_mkq_dtype(q), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                        out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq_len,
                                        static_cast<float>(scale), cos_sin->data_ptr<float>(),
                                        static_cast<int>(rotary_dim), ws.data_ptr(),
                                        static_cast<size_t>(ws.numel()), current_stream());
  }
  check_status(rc, cos_sin == nullptr ? "full_attention_decode" : "full_attention_decode_rope");
  return out;
}

torch::Tensor full_attention_decode(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, double scale) {
  return attention_impl(q, k_cache, v_cache, scale, nullptr, 0);
}

torch::Tensor full_attention_decode_rope(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, double scale,
                                         torch::Tensor cos_sin, int64_t rotary_dim) {
  return attention_impl(q, k_cache, v_cache, scale, &cos_sin, rotary_dim);
}

// Writes k_new/v_new [batch, kv_heads, head_dim] into row seq_len - 1 of the
// caches [batch, capacity, kv_heads, head_dim] (in place) and attends over
// the first seq_len tokens; cos_sin as for full_attention_decode_rope or None.
torch::Tensor full_attention_decode_append(torch::Tensor q, torch::Tensor k_new, torch::Tensor v_new,
                                           torch::Tensor k_cache, torch::Tensor v_cache, int64_t seq_len, double scale,
                                           c10::optional<torch::Tensor> cos_sin, int64_t rotary_dim) {
  MK_CHECK_INPUT(q);
  MK_CHECK_INPUT(k_new);
  MK_CHECK_INPUT(v_new);
  MK_CHECK_INPUT(k_cache);
  MK_CHECK_INPUT(v_cache);
  TORCH_CHECK(q.dim() == 3, "q must be [batch, query_heads, head_dim]");
  TORCH_CHECK(k_cache.dim() == 4, "k_cache must be [batch, capacity, kv_heads, head_dim]");
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "v_cache shape must match k_cache");
  TORCH_CHECK(q.scalar_type() == k_cache.scalar_type() && q.scalar_type() == v_cache.scalar_type() &&
                  q.scalar_type() == k_new.scalar_type() && q.scalar_type() == v_new.scalar_type(),
              "q, k_new, v_new and the caches must share a dtype");
  const int batch = static_cast<int>(q.size(0));
  const int query_heads = static_cast<int>(q.size(1));
  const int head_dim = static_cast<int>(q.size(2));
  const int capacity = static_cast<int>(k_cache.size(1));
  const int kv_heads = static_cast<int>(k_cache.size(2));
  TORCH_CHECK(k_cache.size(0) == batch && k_cache.size(3) == head_dim, "k_cache batch/head_dim mismatch");
  TORCH_CHECK(k_new.dim() == 3 && k_new.size(0) == batch && k_new.size(1) == kv_heads && k_new.size(2) == head_dim,
              "k_new must be [batch, kv_heads, head_dim]");
  TORCH_CHECK(v_new.sizes() == k_new.sizes(), "v_new shape must match k_new");
  TORCH_CHECK(kv_heads > 0 && query_heads % kv_heads == 0, "query_heads must be divisible by kv_heads");
  TORCH_CHECK(seq_len > 0 && seq_len <= capacity, "seq_len must be in [1, capacity]");
  const float* cs = nullptr;
  if (cos_sin.has_value()) {
    TORCH_CHECK(cos_sin->is_cuda() && cos_sin->is_contiguous() && cos_sin->scalar_type() == torch::kFloat32,
                "cos_sin must be a contiguous float32 device tensor");
    TORCH_CHECK(cos_sin->numel() == 2 * rotary_dim, "cos_sin must hold 2 * rotary_dim values");
    cs = cos_sin->data_ptr<float>();
  }
  c10::DeviceGuard guard(q.device());
  auto out = torch::empty_like(q);
  const int seq = static_cast<int>(seq_len);
  auto ws = workspace_for(Ws::kAttention, q,
                          mkq_full_attention_decode_workspace_bytes(batch, query_heads, kv_heads, head_dim, seq));
  const int rc = mkq_full_attention_decode_append(
      to_mkq_dtype(q), q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
      out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq, capacity, static_cast<float>(scale), cs,
      static_cast<int>(rotary_dim), ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream());
  check_status(rc, "full_attention_decode_append");
  return out;
}

// q [B, Hq, D]; k_blocks/v_blocks [num_blocks, block_size, Hkv, D];
// block_table [B, max_blocks] int32; attends over the first seq_len tokens.
torch::Tensor full_attention_decode_paged(torch::Tensor q, torch::Tensor k_blocks, torch::Tensor v_blocks,
                                          torch::Tensor block_table, int64_t seq_len, double scale,
                                          c10::optional<torch::Tensor> k_new, c10::optional<torch::Tensor> v_new,
                                          c10::optional<torch::Tensor> cos_sin, int64_t rotary_dim) {
  MK_CHECK_INPUT(q);
  MK_CHECK_INPUT(k_blocks);
  MK_CHECK_INPUT(v_blocks);
  MK_CHECK_INPUT(block_table);
  TORCH_CHECK(q.dim() == 3, "q must be [batch, query_heads, head_dim]");
  TORCH_CHECK(k_blocks.dim() == 4, "k_blocks must be [num_blocks, block_size, kv_heads, head_dim]");
  TORCH_CHECK(v_blocks.sizes() == k_blocks.sizes(), "v_blocks shape must match k_blocks");
  TORCH_CHECK(q.scalar_type() == k_blocks.scalar_type() && q.scalar_type() == v_blocks.scalar_type(),
              "q and the block pools dtype mismatch");
  TORCH_CHECK(block_table.scalar_type() == torch::kInt32 && block_table.dim() == 2 &&
                  block_table.size(0) == q.size(0),
              "block_table must be int32 [batch, max_blocks]");
  const int batch = static_cast<int>(q.size(0));
  const int query_heads = static_cast<int>(q.size(1));
  const int head_dim = static_cast<int>(q.size(2));
  const int kv_heads = static_cast<int>(k_blocks.size(2));
  TORCH_CHECK(k_blocks.size(3) == head_dim, "head_dim mismatch");
  TORCH_CHECK(kv_heads > 0 && query_heads % kv_heads == 0, "query_heads must be divisible by kv_heads");
  TORCH_CHECK(seq_len > 0, "seq_len must be positive");
  const int seq = static_cast<int>(seq_len);
  c10::DeviceGuard guard(q.device());
  auto out = torch::empty_like(q);
  auto ws = workspace_for(Ws::kAttention, q,
                          mkq_full_attention_decode_workspace_bytes(batch, query_heads, kv_heads, head_dim, seq));
  TORCH_CHECK(k_new.has_value() == v_new.has_value(), "k_new and v_new must be given together");
  int rc;
  if (cos_sin.has_value()) {
    TORCH_CHECK(cos_sin->is_cuda() && cos_sin->is_contiguous() && cos_sin->scalar_type() == torch::kFloat32,
                "cos_sin must be a contiguous float32 device tensor");
    TORCH_CHECK(cos_sin->numel() == 2 * rotary_dim, "cos_sin must hold 2 * rotary_dim values");
  }
  if (k_new.has_value()) {
    MK_CHECK_INPUT((*k_new));
    MK_CHECK_INPUT((*v_new));
    TORCH_CHECK(k_new->dim() == 3 && k_new->size(0) == batch && k_new->size(1) == kv_heads &&
                    k_new->size(2) == head_dim && v_new->sizes() == k_new->sizes(),
                "k_new and v_new must be [batch, kv_heads, head_dim]");
    TORCH_CHECK(k_new->scalar_type() == q.scalar_type() && v_new->scalar_type() == q.scalar_type(),
                "k_new/v_new dtype mismatch");
  }
  if (cos_sin.has_value() && k_new.has_value()) {
    rc = mkq_full_attention_decode_paged_append_rope(
        to_mkq_dtype(q), q.data_ptr(), k_new->data_ptr(), v_new->data_ptr(), k_blocks.data_ptr(), v_blocks.data_ptr(),
        block_table.data_ptr<int>(), out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq,
        static_cast<int>(k_blocks.size(1)), static_cast<int>(block_table.size(1)), static_cast<int>(k_blocks.size(0)),
        static_cast<float>(scale), cos_sin->data_ptr<float>(), static_cast<int>(rotary_dim), ws.data_ptr(),
        static_cast<size_t>(ws.numel()), current_stream());
  } else if (cos_sin.has_value()) {
    rc = mkq_full_attention_decode_paged_rope(
        to_mkq_dtype(q), q.data_ptr(), k_blocks.data_ptr(), v_blocks.data_ptr(), block_table.data_ptr<int>(),
        out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq, static_cast<int>(k_blocks.size(1)),
        static_cast<int>(block_table.size(1)), static_cast<int>(k_blocks.size(0)), static_cast<float>(scale),
        cos_sin->data_ptr<float>(), static_cast<int>(rotary_dim), ws.data_ptr(), static_cast<size_t>(ws.numel()),
        current_stream());
  } else if (k_new.has_value()) {
    rc = mkq_full_attention_decode_paged_append(
        to_mkq_dtype(q), q.data_ptr(), k_new->data_ptr(), v_new->data_ptr(), k_blocks.data_ptr(), v_blocks.data_ptr(),
        block_table.data_ptr<int>(), out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq,
        static_cast<int>(k_blocks.size(1)), static_cast<int>(block_table.size(1)), static_cast<int>(k_blocks.size(0)),
        static_cast<float>(scale), ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream());
  } else {
    rc = mkq_full_attention_decode_paged(
        to_mkq_dtype(q), q.data_ptr(), k_blocks.data_ptr(), v_blocks.data_ptr(), block_table.data_ptr<int>(),
        out.data_ptr(), batch, query_heads, kv_heads, head_dim, seq, static_cast<int>(k_blocks.size(1)),
        static_cast<int>(block_table.size(1)), static_cast<int>(k_blocks.size(0)), static_cast<float>(scale),
        ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream());
  }
  check_status(rc, "full_attention_decode_paged");
  return out;
}

std::tuple<torch::Tensor, torch::Tensor> linear_attention_decode(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                                                 torch::Tensor state, double decay) {
  // Checks and messages as in linear_attention_decode.cu:52-69.
  MK_CHECK_INPUT(q);
  MK_CHECK_INPUT(k);
  MK_CHECK_INPUT(v);
  MK_CHECK_INPUT(state);
  TORCH_CHECK(q.dim() == 3, "q must be [batch, heads, key_dim]");
  TORCH_CHECK(k.sizes() == q.sizes(), "k shape must match q");
  TORCH_CHECK(v.dim() == 3, "v must be [batch, heads, value_dim]");
  TORCH_CHECK(state.dim() == 4, "state must be [batch, heads, key_dim, value_dim]");
  TORCH_CHECK(state.scalar_type() == torch::kFloat32, "state must be float32");
  TORCH_CHECK(q.scalar_type() == k.scalar_type(), "q and k dtype mismatch");
  TORCH_CHECK(q.scalar_type() == v.scalar_type(), "q and v dtype mismatch");
  const int batch = static_cast<int>(q.size(0));
  const int heads = static_cast<int>(q.size(1));
  const int key_dim = static_cast<int>(q.size(2));
  const int value_dim = static_cast<int>(v.size(2));
  TORCH_CHECK(v.size(0) == batch && v.size(1) == heads, "v batch/head mismatch");
  TORCH_CHECK(state.size(0) == batch && state.size(1) == heads && state.size(2) == key_dim &&
                  state.size(3) == value_dim,
              "state shape mismatch");
  c10::DeviceGuard guard(q.device());
  auto out = torch::empty({batch, heads, value_dim}, q.options());
  auto new_state = torch::empty_like(state);
  const int rc = mkq_linear_attention_decode(to_mkq_dtype(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             state.data_ptr<float>(), out.data_ptr(), new_state.data_ptr<float>(),
                                             batch, heads, key_dim, value_dim, static_cast<float>(decay),
                                             current_stream());
  check_status(rc, "linear_attention_decode");
  return std::make_tuple(out, new_state);
}

void check_gated_delta(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                       const torch::Tensor& state, const torch::Tensor& g, const torch::Tensor& beta) {
  MK_CHECK_INPUT(q);
  MK_CHECK_INPUT(k);
  MK_CHECK_INPUT(v);
  MK_CHECK_INPUT(state);
  MK_CHECK_INPUT(g);
  MK_CHECK_INPUT(beta);
  TORCH_CHECK(q.dim() == 3, "q must be [batch, key_heads, key_dim]");
  TORCH_CHECK(k.sizes() == q.sizes(), "k shape must match q");
  TORCH_CHECK(v.dim() == 3, "v must be [batch, value_heads, value_dim]");
  TORCH_CHECK(state.dim() == 4, "state must be [batch, value_heads, key_dim, value_dim]");
  TORCH_CHECK(state.scalar_type() == torch::kFloat32, "state must be float32");
  TORCH_CHECK(g.scalar_type() == torch::kFloat32 && beta.scalar_type() == torch::kFloat32,
              "g and beta must be float32");
  TORCH_CHECK(q.scalar_type() == k.scalar_type(), "q and k dtype mismatch");
  TORCH_CHECK(q.scalar_type() == v.scalar_type(), "q and v dtype mismatch");
  const int64_t batch = q.size(0), hk = q.size(1), dk = q.size(2), hv = v.size(1), dv = v.size(2);
  TORCH_CHECK(v.size(0) == batch, "v batch mismatch");
  TORCH_CHECK(hk > 0 && hv % hk == 0, "value_heads must be a multiple of key_heads");
  TORCH_CHECK(state.size(0) == batch && state.size(1) == hv && state.size(2) == dk && state.size(3) == dv,
              "state shape mismatch");
  TORCH_CHECK(g.numel() == batch * hv && beta.numel() == batch * hv, "g and beta must be [batch, value_heads]");
}

// Runs the gated delta rule with the new state in `new_state` (may be
// `state` itself); with qk_l2norm, q and k are L2-normalised in the kernel and
// q is scaled by q_scale.
torch::Tensor gated_delta_call(const char* fn, torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor state,
                               torch::Tensor g, torch::Tensor beta, torch::Tensor new_state, bool qk_l2norm,
                               double q_scale) {
  check_gated_delta(q, k, v, state, g, beta);
  c10::DeviceGuard guard(q.device());
  auto out = torch::empty({v.size(0), v.size(1), v.size(2)}, q.options());
  const int dtype = to_mkq_dtype(q);
  const int b = static_cast<int>(q.size(0)), hk = static_cast<int>(q.size(1)), hv = static_cast<int>(v.size(1));
  const int dk = static_cast<int>(q.size(2)), dv = static_cast<int>(v.size(2));
  const int rc =
      qk_l2norm ? mkq_gated_delta_decode_qknorm(dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), state.data_ptr<float>(),
                                                g.data_ptr<float>(), beta.data_ptr<float>(), out.data_ptr(),
                                                new_state.data_ptr<float>(), b, hk, hv, dk, dv,
                                                static_cast<float>(q_scale), current_stream())
                : mkq_gated_delta_decode(dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), state.data_ptr<float>(),
                                         g.data_ptr<float>(), beta.data_ptr<float>(), out.data_ptr(),
                                         new_state.data_ptr<float>(), b, hk, hv, dk, dv, current_stream());
  check_status(rc, fn);
  return out;
}

std::tuple<torch::Tensor, torch::Tensor> gated_delta_decode(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                                            torch::Tensor state, torch::Tensor g, torch::Tensor beta,
                                                            bool qk_l2norm, double q_scale) {
  auto new_state = torch::empty_like(state);
  auto out = gated_delta_call("gated_delta_decode", q, k, v, state, g, beta, new_state, qk_l2norm, q_scale);
  return std::make_tuple(out, new_state);
}

// In-place variant: state is updated where it lies; returns out.
torch::Tensor gated_delta_decode_(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor state,
                                  torch::Tensor g, torch::Tensor beta, bool qk_l2norm, double q_scale) {
  return gated_delta_call("gated_delta_decode_", q, k, v, state, g, beta, state, qk_l2norm, q_scale);
}

// x [batch, channels]; conv_state [batch, channels, state_len] updated in
// place; weight [channels, state_len + 1]; returns act(conv) [batch, channels].
torch::Tensor causal_conv1d_update(torch::Tensor x, torch::Tensor conv_state, torch::Tensor weight,
                                   c10::optional<torch::Tensor> bias, bool silu_activation) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(conv_state);
  MK_CHECK_INPUT(weight);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, channels]");
  TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(0) == x.size(0) && conv_state.size(1) == x.size(1),
              "conv_state must be [batch, channels, state_len]");
  TORCH_CHECK(weight.dim() == 2 && weight.size(0) == x.size(1) && weight.size(1) == conv_state.size(2) + 1,
              "weight must be [channels, state_len + 1]");
  TORCH_CHECK(x.scalar_type() == conv_state.scalar_type() && x.scalar_type() == weight.scalar_type(),
              "x, conv_state and weight dtype mismatch");
  const void* b = nullptr;
  if (bias.has_value()) {
    MK_CHECK_INPUT((*bias));
    TORCH_CHECK(bias->numel() == x.size(1) && bias->scalar_type() == x.scalar_type(), "bias must be [channels]");
    b = bias->data_ptr();
  }
  c10::DeviceGuard guard(x.device());
  auto out = torch::empty_like(x);
  const int rc = mkq_causal_conv1d_update(to_mkq_dtype(x), x.data_ptr(), conv_state.data_ptr(), weight.data_ptr(), b,
                                          out.data_ptr(), static_cast<int>(x.size(0)), static_cast<int>(x.size(1)),
                                          static_cast<int>(conv_state.size(2)), silu_activation ? 1 : 0,
                                          current_stream());
  check_status(rc, "causal_conv1d_update");
  return out;
}

// x, gate [..., dim]; weight [dim]: weight * rms_norm(x) * silu(gate).
torch::Tensor gated_rms_norm(torch::Tensor x, torch::Tensor gate, torch::Tensor weight, double eps) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(gate);
  MK_CHECK_INPUT(weight);
  TORCH_CHECK(x.dim() >= 1 && gate.sizes() == x.sizes(), "gate shape must match x");
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == x.size(-1), "weight must be [dim]");
  TORCH_CHECK(x.scalar_type() == gate.scalar_type() && x.scalar_type() == weight.scalar_type(),
              "x, gate and weight dtype mismatch");
  c10::DeviceGuard guard(x.device());
  auto out = torch::empty_like(x);
  const int64_t dim = x.size(-1);
  const int rc = mkq_gated_rms_norm(to_mkq_dtype(x), x.data_ptr(), gate.data_ptr(), weight.data_ptr(), out.data_ptr(),
                                    static_cast<int>(x.numel() / dim), static_cast<int>(dim),
                                    static_cast<float>(eps), current_stream());
  check_status(rc, "gated_rms_norm");
  return out;
}

// One Qwen3.6 linear-attention step: conv update (conv_state in place), the
// gated delta rule with q/k L2 norm (state in place), gated RMS norm.
torch::Tensor linear_attention_step(torch::Tensor x_mixed, torch::Tensor conv_state, torch::Tensor conv_weight,
                                    c10::optional<torch::Tensor> conv_bias, torch::Tensor state, torch::Tensor g,
                                    torch::Tensor beta, torch::Tensor z, torch::Tensor norm_weight, int64_t k_heads,
                                    double q_scale, double eps) {
  MK_CHECK_INPUT(x_mixed);
  MK_CHECK_INPUT(conv_state);
  MK_CHECK_INPUT(conv_weight);
  MK_CHECK_INPUT(state);
  MK_CHECK_INPUT(g);
  MK_CHECK_INPUT(beta);
  MK_CHECK_INPUT(z);
  MK_CHECK_INPUT(norm_weight);
  TORCH_CHECK(x_mixed.dim() == 2, "x_mixed must be [batch, channels]");
  TORCH_CHECK(state.dim() == 4 && state.scalar_type() == torch::kFloat32,
              "state must be float32 [batch, v_heads, key_dim, value_dim]");
  TORCH_CHECK(z.dim() == 3, "z must be [batch, v_heads, value_dim]");
  const int64_t batch = x_mixed.size(0), c = x_mixed.size(1);
  const int64_t hv = state.size(1), dk = state.size(2), dv = state.size(3);
  TORCH_CHECK(state.size(0) == batch && z.size(0) == batch && z.size(1) == hv && z.size(2) == dv,
              "state/z batch or head mismatch");
  TORCH_CHECK(k_heads > 0 && c == 2 * k_heads * dk + hv * dv, "channels must be 2*k_heads*key_dim + v_heads*value_dim");
  TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(0) == batch && conv_state.size(1) == c,
              "conv_state must be [batch, channels, state_len]");
  TORCH_CHECK(conv_weight.dim() == 2 && conv_weight.size(0) == c && conv_weight.size(1) == conv_state.size(2) + 1,
              "conv_weight must be [channels, state_len + 1]");
  TORCH_CHECK(norm_weight.numel() == dv, "norm_weight must be [value_dim]");
  TORCH_CHECK(g.numel() == batch * hv && beta.numel() == batch * hv && g.scalar_type() == torch::kFloat32 &&
                  beta.scalar_type() == torch::kFloat32,
              "g and beta must be float32 [batch, v_heads]");
  const auto dt = x_mixed.scalar_type();
  TORCH_CHECK(conv_state.scalar_type() == dt && conv_weight.scalar_type() == dt && z.scalar_type() == dt &&
                  norm_weight.scalar_type() == dt,
              "x_mixed, conv_state, conv_weight, z and norm_weight must share a dtype");
  const void* bias = nullptr;
  if (conv_bias.has_value()) {
    MK_CHECK_INPUT((*conv_bias));
    TORCH_CHECK(conv_bias->numel() == c && conv_bias->scalar_type() == dt, "conv_bias must be [channels]");
    bias = conv_bias->data_ptr();
  }
  c10::DeviceGuard guard(x_mixed.device());
  auto out = torch::empty_like(z);
  const int dtype = to_mkq_dtype(x_mixed);
  const size_t need = mkq_linear_attention_step_workspace_bytes(dtype, static_cast<int>(batch), static_cast<int>(k_heads),
                                                                static_cast<int>(hv), static_cast<int>(dk),
                                                                static_cast<int>(dv));
  auto ws = workspace_for(Ws::kLinearStep, x_mixed, need);
  const int rc = mkq_linear_attention_step(
      dtype, x_mixed.data_ptr(), conv_state.data_ptr(), conv_weight.data_ptr(), bias,
      static_cast<int>(conv_state.size(2)), state.data_ptr<float>(), g.data_ptr<float>(), beta.data_ptr<float>(),
      z.data_ptr(), norm_weight.data_ptr(), out.data_ptr(), static_cast<int>(batch), static_cast<int>(k_heads),
      static_cast<int>(hv), static_cast<int>(dk), static_cast<int>(dv), static_cast<float>(q_scale),
      static_cast<float>(eps), ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream());
  check_status(rc, "linear_attention_step");
  return out;
}

torch::Tensor gemv(torch::Tensor x, torch::Tensor w, c10::optional<torch::Tensor> residual) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(w);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, in_features]");
  TORCH_CHECK(w.dim() == 2, "w must be [out_features, in_features]");
  TORCH_CHECK(w.size(1) == x.size(1), "in_features mismatch");
  TORCH_CHECK(x.scalar_type() == w.scalar_type(), "x and w dtype mismatch");
  const void* r = nullptr;
  if (residual.has_value()) {
    MK_CHECK_INPUT((*residual));
    TORCH_CHECK(residual->scalar_type() == x.scalar_type(), "x and residual dtype mismatch");
    TORCH_CHECK(residual->dim() == 2 && residual->size(0) == x.size(0) && residual->size(1) == w.size(0),
                "residual must be [batch, out_features]");
    r = residual->data_ptr();
  }
  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({x.size(0), w.size(0)}, x.options());
  const int rc = mkq_gemv(to_mkq_dtype(x), x.data_ptr(), w.data_ptr(), r, y.data_ptr(), static_cast<int>(x.size(0)),
                          static_cast<int>(x.size(1)), static_cast<int>(w.size(0)), current_stream());
  check_status(rc, "gemv");
  return y;
}

std::tuple<torch::Tensor, torch::Tensor> gemv_add(torch::Tensor x, torch::Tensor w, torch::Tensor residual) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(w);
  MK_CHECK_INPUT(residual);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, in_features]");
  TORCH_CHECK(w.dim() == 2, "w must be [out_features, in_features]");
  TORCH_CHECK(w.size(1) == x.size(1), "in_features mismatch");
  TORCH_CHECK(x.scalar_type() == w.scalar_type() && x.scalar_type() == residual.scalar_type(),
              "x, w and residual dtype mismatch");
  TORCH_CHECK(residual.dim() == 2 && residual.size(0) == x.size(0) && residual.size(1) == w.size(0),
              "residual must be [batch, out_features]");
  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({x.size(0), w.size(0)}, x.options());
  auto sum = torch::empty_like(y);
  const int rc = mkq_gemv_add(to_mkq_dtype(x), x.data_ptr(), w.data_ptr(), residual.data_ptr(), y.data_ptr(),
                              sum.data_ptr(), static_cast<int>(x.size(0)), static_cast<int>(x.size(1)),
                              static_cast<int>(w.size(0)), current_stream());
  check_status(rc, "gemv_add");
  return {y, sum};
}

torch::Tensor rms_norm_gemv(torch::Tensor x, torch::Tensor norm_weight, torch::Tensor w, double eps) {
  MK_CHECK_INPUT(x);
  MK_CHECK_INPUT(norm_weight);
  MK_CHECK_INPUT(w);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, in_features]");
  TORCH_CHECK(w.dim() == 2, "w must be [out_features, in_features]");
  TORCH_CHECK(w.size(1) == x.size(1), "in_features mismatch");
  TORCH_CHECK(norm_weight.dim() == 1 && norm_weight.size(0) == x.size(1), "norm_weight must be [in_features]");
  TORCH_CHECK(x.scalar_type() == w.scalar_type() && x.scalar_type() == norm_weight.scalar_type(),
              "x, norm_weight and w dtype mismatch");
  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({x.size(0), w.size(0)}, x.options());
  const int rc = mkq_rms_norm_gemv(to_mkq_dtype(x), x.data_ptr(), norm_weight.data_ptr(), static_cast<float>(eps),
                                   w.data_ptr(), y.data_ptr(), static_cast<int>(x.size(0)),
                                   static_cast<int>(x.size(1)), static_cast<int>(w.size(0)), current_stream());
  check_status(rc, "rms_norm_gemv");
  return y;
}

// Error word of the MoE workspace of the current device and stream (0 if
// that stream has none yet); with reset, a nonzero word clears the workspace.
// Synchronises the stream.
int64_t moe_decode_status(bool reset) {
  int dev = 0;
  TORCH_CHECK(hipGetDevice(&dev) == hipSuccess, "moe_decode_status: no current device");
  auto& cache = workspace_cache();
  auto it = cache.find(std::make_tuple(static_cast<int>(Ws::kMoe), dev, current_stream()));
  if (it == cache.end()) return 0;
  int code = 0;
  const int rc = mkq_moe_decode_status(it->second.data_ptr(), static_cast<size_t>(it->second.numel()), reset ? 1 : 0,
                                       &code, current_stream());
  check_status(rc, "moe_decode_status");
  return code;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MI355X (gfx950) decode kernels for Qwen3.6 behind the mega_kernel_qwen36 API";
  m.def("moe_decode_persistent", &moe_decode_persistent, "Persistent single-launch MoE decode (HIP)");
  m.def("moe_decode_persistent_gated", &moe_decode_persistent_gated,
        "Persistent MoE decode with a sigmoid-gated shared expert (HIP)");
  m.def("dense_ffn_decode", &dense_ffn_decode, "Fused RMSNorm + SwiGLU FFN decode (HIP)");
  m.def("full_attention_decode", &full_attention_decode, "Split-K GQA flash-decode (HIP)");
  m.def("full_attention_decode_rope", &full_attention_decode_rope,
        "Split-K GQA flash-decode with the keys rotated on the fly (HIP)");
  m.def("full_attention_decode_append", &full_attention_decode_append,
        "KV append fused into the split-K GQA flash-decode (HIP)", pybind11::arg("q"), pybind11::arg("k_new"),
        pybind11::arg("v_new"), pybind11::arg("k_cache"), pybind11::arg("v_cache"), pybind11::arg("seq_len"),
        pybind11::arg("scale"), pybind11::arg("cos_sin") = pybind11::none(), pybind11::arg("rotary_dim") = 0);
  m.def("full_attention_decode_paged", &full_attention_decode_paged,
        "Split-K GQA flash-decode over a paged KV pool (HIP)", pybind11::arg("q"), pybind11::arg("k_blocks"),
        pybind11::arg("v_blocks"), pybind11::arg("block_table"), pybind11::arg("seq_len"), pybind11::arg("scale"),
        pybind11::arg("k_new") = pybind11::none(), pybind11::arg("v_new") = pybind11::none(),
        pybind11::arg("cos_sin") = pybind11::none(), pybind11::arg("rotary_dim") = 0);
  m.def("linear_attention_decode", &linear_attention_decode, "Recurrent linear-attention decode (HIP)");
  m.def("gated_delta_decode", &gated_delta_decode, "Gated delta rule decode (HIP)", pybind11::arg("q"),
        pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("state"), pybind11::arg("g"), pybind11::arg("beta"),
        pybind11::arg("qk_l2norm") = false, pybind11::arg("q_scale") = 1.0);
  m.def("gated_delta_decode_", &gated_delta_decode_, "Gated delta rule decode, state updated in place (HIP)",
        pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("state"), pybind11::arg("g"),
        pybind11::arg("beta"), pybind11::arg("qk_l2norm") = false, pybind11::arg("q_scale") = 1.0);
  m.def("causal_conv1d_update", &causal_conv1d_update, "Causal conv1d state update for one token (HIP)",
        pybind11::arg("x"), pybind11::arg("conv_state"), pybind11::arg("weight"),
        pybind11::arg("bias") = pybind11::none(), pybind11::arg("silu_activation") = true);
  m.def("gated_rms_norm", &gated_rms_norm, "Gated RMS norm, norm before gate (HIP)", pybind11::arg("x"),
        pybind11::arg("gate"), pybind11::arg("weight"), pybind11::arg("eps") = 1e-6);
  m.def("linear_attention_step", &linear_attention_step,
        "Qwen3.6 linear-attention step: conv update, gated delta rule with q/k norm, gated norm (HIP)",
        pybind11::arg("x_mixed"), pybind11::arg("conv_state"), pybind11::arg("conv_weight"),
        pybind11::arg("conv_bias"), pybind11::arg("state"), pybind11::arg("g"), pybind11::arg("beta"),
        pybind11::arg("z"), pybind11::arg("norm_weight"), pybind11::arg("k_heads"), pybind11::arg("q_scale"),
        pybind11::arg("eps"));
  m.def("gemv", &gemv, "y = x w^T (+ residual) (HIP)", pybind11::arg("x"), pybind11::arg("w"),
        pybind11::arg("residual") = pybind11::none());
  m.def("gemv_add", &gemv_add, "(y, residual + y) with y = x w^T (HIP)", pybind11::arg("x"), pybind11::arg("w"),
        pybind11::arg("residual"));
  m.def("rms_norm_gemv", &rms_norm_gemv, "y = rms_norm(x, norm_weight) w^T, norm rounded to the dtype (HIP)",
        pybind11::arg("x"), pybind11::arg("norm_weight"), pybind11::arg("w"), pybind11::arg("eps") = 1e-6);
  m.def("moe_decode_status", &moe_decode_status,
        "Error word of the current stream's MoE workspace (1: a cross-workgroup wait timed out); synchronises",
        pybind11::arg("reset") = false);
  m.def("abi_version", &mkq_abi_version);
}
