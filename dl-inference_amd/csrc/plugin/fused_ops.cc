// Fused decode operators (extensions registered next to the reference operators). Each replaces
// a run of nodes of the reference's exported Qwen2 decoder graph
// (python/dli_export/export.py:272-446) and keeps that graph's bf16 rounding points:
//
//   qkv_rope_append        (input_layernorm,) q/k/v_proj, reshapes, rotary_embedding, KV
//                          append
//   qkv_rope_heads         q/k/v_proj, reshapes, [B,S,H,D] -> [B,H,S,D] transposes and
//                          rotary_embedding of a prompt (prefill)
//   paged_attention        attention over the already appended paged KV cache (decode)
//   linear_residual        o_proj + attention_residual, down_proj + mlp_residual
//   linear_residual_norm   the same plus the RMSNorm that follows the residual update
//                          (post_attention_layernorm, the next input_layernorm, model.norm)
//   gate_up_silu           (post_attention_layernorm,) gate_proj, up_proj, act_fn, mul
//   lm_head_argmax         lm_head, greedy argmax
//   decoder_stack          every decoder layer above in one persistent launch
//   argmax                 greedy argmax over the last dim (unfused graphs)
#include <cmath>

#include "common.h"

namespace dli::plugin {
namespace {

void requireBf16(const Tensor& t, const std::string& op, const std::string& what) {
  if (t.dtype() != DType::BFloat16) throw std::invalid_argument(op + " " + what + " must be bfloat16");
}

std::int64_t rowsOf(const Tensor& t) { return product(t.shape(), 0, t.rank() - 1); }

// inputs: hidden [B, H], (norm_weight [H],) w_qkv [N, H], b_qkv [N], cos, sin, positions [B].
// With norm_weight the RMSNorm (input_layernorm) runs inside the kernel; without it hidden is
// the normalized activation.
class QkvRopeAppendOp final : public Operator {
 public:
  std::string type() const override { return "qkv_rope_append"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 6, 7, 1, type());
    requireCudaInputs(in, type());
    const std::size_t o = in.size() == 7 ? 1 : 0;
    const Tensor* nw = o ? in[1] : nullptr;
    const Tensor &x = *in[0], &w = *in[1 + o], &b = *in[2 + o], &cos = *in[3 + o],
                 &sin = *in[4 + o], &pos = *in[5 + o];
    for (const Tensor* t : {&x, &w, &b}) requireBf16(*t, type(), "activations/weights");
    requireFloat(cos, type());
    requireFloat(sin, type());
    requireIndex(pos, type(), "positions");
    const auto hq = attrs.require<std::int64_t>("q_heads");
    const auto hkv = attrs.require<std::int64_t>("kv_heads");
    const auto d = attrs.require<std::int64_t>("head_dim");
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    const std::string& cache_name = attrs.require<std::string>("kv_cache");
    const std::int64_t hidden = x.shape().back();
    const std::int64_t m = rowsOf(x);
    const std::int64_t n = (hq + 2 * hkv) * d;
    if (w.rank() != 2 || w.dim(0) != n || w.dim(1) != hidden || static_cast<std::int64_t>(b.numel()) != n)
      throw std::invalid_argument("qkv_rope_append weight shapes do not match the attributes");
    if (nw != nullptr && (nw->dtype() != DType::BFloat16 || static_cast<std::int64_t>(nw->numel()) != hidden))
      throw std::invalid_argument("qkv_rope_append norm weight must be bfloat16 [hidden]");
    if (cos.rank() != 2 || cos.dim(1) != d / 2 || cos.shape() != sin.shape())
      throw std::invalid_argument("qkv_rope_append cos/sin must be [max_pos, head_dim/2]");
    if (static_cast<std::int64_t>(pos.numel()) != m)
      throw std::invalid_argument("qkv_rope_append positions must have one entry per row");
    if (ctx.kv_cache == nullptr) throw std::invalid_argument("qkv_rope_append missing KV cache");
    KVCacheEntry& e = ctx.kv_cache->reserve(cache_name, DType::BFloat16, m, hkv, d, x.deviceId());
    *out[0] = Tensor::cuda(DType::BFloat16, {m, hq, 1, d}, x.deviceId());
    // hidden sizes above 1024 project through a workspace (K-split parts and one reduce)
    const std::size_t ws_bytes = dli_hip_qkv_rope_append_workspace(m, hidden, hq, hkv, d);
    check(dli_hip_qkv_rope_append_ws(
              ptr(x), nw ? ptr(*nw) : nullptr, ptr(w), ptr(b), static_cast<const float*>(ptr(cos)),
              static_cast<const float*>(ptr(sin)), cos.dim(0), ptr(pos), hipDtype(pos.dtype()),
              ptr(*out[0]), ptr(e.key_pool), ptr(e.value_pool),
              static_cast<const std::int32_t*>(ptr(e.block_table)), e.block_size, e.max_blocks, m,
              hidden, hq, hkv, d, eps,
              ws_bytes ? workspace_.get(ws_bytes, x.deviceId(), ctx.stream) : nullptr, ws_bytes, ctx.stream),
          type());
  }

 private:
  mutable PersistentWorkspace workspace_;
};

// inputs: x [B, S, H] (normalized), w_qkv [N, H], b_qkv [N], cos, sin [max_pos, D / 2];
// attrs q_heads, kv_heads, head_dim, start_pos (0); outputs q [B, Hq, S, D], k and v
// [B, Hkv, S, D] with RoPE on q and k at positions start_pos + s.
class QkvRopeHeadsOp final : public Operator {
 public:
  std::string type() const override { return "qkv_rope_heads"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 5, 5, 3, type());
    requireCudaInputs(in, type());
    const Tensor &x = *in[0], &w = *in[1], &b = *in[2], &cos = *in[3], &sin = *in[4];
    for (const Tensor* t : {&x, &w, &b}) requireBf16(*t, type(), "activations/weights");
    requireFloat(cos, type());
    requireFloat(sin, type());
    const auto hq = attrs.require<std::int64_t>("q_heads");
    const auto hkv = attrs.require<std::int64_t>("kv_heads");
    const auto d = attrs.require<std::int64_t>("head_dim");
    const auto start = attrs.value_or<std::int64_t>("start_pos", 0);
    if (x.rank() != 3) throw std::invalid_argument("qkv_rope_heads x must be [B, S, H]");
    const std::int64_t B = x.dim(0), S = x.dim(1), hidden = x.dim(2);
    const std::int64_t n = (hq + 2 * hkv) * d;
    if (w.rank() != 2 || w.dim(0) != n || w.dim(1) != hidden || static_cast<std::int64_t>(b.numel()) != n)
      throw std::invalid_argument("qkv_rope_heads weight shapes do not match the attributes");
    if (cos.rank() != 2 || cos.dim(1) != d / 2 || cos.shape() != sin.shape())
      throw std::invalid_argument("qkv_rope_heads cos/sin must be [max_pos, head_dim/2]");
    *out[0] = Tensor::cuda(DType::BFloat16, {B, hq, S, d}, x.deviceId());
    *out[1] = Tensor::cuda(DType::BFloat16, {B, hkv, S, d}, x.deviceId());
    *out[2] = Tensor::cuda(DType::BFloat16, {B, hkv, S, d}, x.deviceId());
    check(dli_hip_qkv_rope_heads(ptr(x), ptr(w), ptr(b), static_cast<const float*>(ptr(cos)),
                                 static_cast<const float*>(ptr(sin)), cos.dim(0), ptr(*out[0]),
                                 ptr(*out[1]), ptr(*out[2]), B, S, hidden, hq, hkv, d, start,
                                 ctx.stream),
          type());
  }
};

// Decode attention over a cache entry whose newest token (at positions[b]) is already written.
class PagedAttentionOp final : public Operator {
 public:
  std::string type() const override { return "paged_attention"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireCudaInputs(in, type());
    const Tensor& q = *in[0];
    const Tensor& pos = *in[1];
    requireFloating(q, type());
    requireIndex(pos, type(), "positions");
    if (q.rank() != 4 || q.dim(2) != 1) throw std::invalid_argument("paged_attention expects q [B, H, 1, D]");
    if (ctx.kv_cache == nullptr) throw std::invalid_argument("paged_attention missing KV cache");
    const KVCacheEntry* e = ctx.kv_cache->get(attrs.require<std::string>("kv_cache"));
    if (e == nullptr) throw std::invalid_argument("paged_attention: unknown kv_cache entry");
    if (e->batch != q.dim(0) || e->head_dim != q.dim(3) || e->key_pool.dtype() != q.dtype())
      throw std::invalid_argument("paged_attention: q does not match the cache entry");
    const std::int64_t B = q.dim(0), Hq = q.dim(1), D = q.dim(3);
    const float scale = static_cast<float>(attrDouble(attrs, "scale", 1.0 / std::sqrt(static_cast<double>(D))));
    // key-range splits per (sequence, kv head); 0 = about one workgroup per CU
    const auto splits = static_cast<int>(attrs.value_or<std::int64_t>("attention_splits", 0));
    *out[0] = Tensor::cuda(q.dtype(), q.shape(), q.deviceId());
    const std::size_t ws_bytes = dli_hip_paged_attention_workspace(B, Hq, 1, D, e->capacity());
    check(dli_hip_paged_attention(hipDtype(q.dtype()), ptr(q), ptr(e->key_pool), ptr(e->value_pool),
                                  static_cast<const std::int32_t*>(ptr(e->block_table)), ptr(*out[0]),
                                  B, Hq, e->heads, 1, D, e->block_size, e->max_blocks, 0, ptr(pos),
                                  hipDtype(pos.dtype()), 1, scale, splits,
                                  workspace_.get(ws_bytes, q.deviceId(), ctx.stream), ws_bytes, ctx.stream),
          type());
  }

 private:
  mutable PersistentWorkspace workspace_;
};

// inputs: x [.., K], w [N, K], residual [.., N] (+ bias [N]); out = residual + bf16(x w^T + b)
class LinearResidualOp final : public Operator {
 public:
  std::string type() const override { return "linear_residual"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 3, 4, 1, type());
    requireCudaInputs(in, type());
    for (const Tensor* t : in) requireBf16(*t, type(), "inputs");
    const Tensor &x = *in[0], &w = *in[1], &res = *in[2];
    const std::int64_t k = x.shape().back(), m = rowsOf(x);
    if (w.rank() != 2 || w.dim(1) != k) throw std::invalid_argument("linear_residual weight shape mismatch");
    const std::int64_t n = w.dim(0);
    if (rowsOf(res) != m || res.shape().back() != n)
      throw std::invalid_argument("linear_residual residual shape mismatch");
    if (in.size() == 4 && static_cast<std::int64_t>(in[3]->numel()) != n)
      throw std::invalid_argument("linear_residual bias size mismatch");
    const auto splits = static_cast<int>(attrs.value_or<std::int64_t>("splits", 1));
    *out[0] = Tensor::cuda(DType::BFloat16, res.shape(), x.deviceId());
    const std::size_t ws_bytes = dli_hip_splitk_workspace(n, m, splits);
    check(dli_hip_linear_residual(ptr(x), ptr(w), in.size() == 4 ? ptr(*in[3]) : nullptr, ptr(res),
                                  ptr(*out[0]), m, n, k, splits,
                                  workspace_.get(ws_bytes, x.deviceId(), ctx.stream), ws_bytes, ctx.stream),
          type());
  }

 private:
  mutable PersistentWorkspace workspace_;
};

// inputs: x [.., K], w [N, K], residual [.., N], norm_weight [N] (+ bias [N]);
// outputs: h = residual + bf16(x w^T + b), xn = rms_norm(h) * norm_weight
class LinearResidualNormOp final : public Operator {
 public:
  std::string type() const override { return "linear_residual_norm"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 4, 5, 2, type());
    requireCudaInputs(in, type());
    for (const Tensor* t : in) requireBf16(*t, type(), "inputs");
    const Tensor &x = *in[0], &w = *in[1], &res = *in[2], &nw = *in[3];
    const std::int64_t k = x.shape().back(), m = rowsOf(x);
    if (w.rank() != 2 || w.dim(1) != k) throw std::invalid_argument("linear_residual_norm weight shape mismatch");
    const std::int64_t n = w.dim(0);
    if (rowsOf(res) != m || res.shape().back() != n)
      throw std::invalid_argument("linear_residual_norm residual shape mismatch");
    if (static_cast<std::int64_t>(nw.numel()) != n)
      throw std::invalid_argument("linear_residual_norm norm weight size mismatch");
    if (in.size() == 5 && static_cast<std::int64_t>(in[4]->numel()) != n)
      throw std::invalid_argument("linear_residual_norm bias size mismatch");
    const auto splits = static_cast<int>(attrs.value_or<std::int64_t>("splits", 1));
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    *out[0] = Tensor::cuda(DType::BFloat16, res.shape(), x.deviceId());
    *out[1] = Tensor::cuda(DType::BFloat16, res.shape(), x.deviceId());
    const std::size_t ws_bytes = dli_hip_splitk_workspace(n, m, splits);
    check(dli_hip_linear_residual_norm(ptr(x), ptr(w), in.size() == 5 ? ptr(*in[4]) : nullptr,
                                       ptr(res), ptr(nw), ptr(*out[0]), ptr(*out[1]), m, n, k, eps,
                                       splits, workspace_.get(ws_bytes, x.deviceId(), ctx.stream), ws_bytes,
                                       ctx.stream),
          type());
  }

 private:
  mutable PersistentWorkspace workspace_;
};

// inputs: hidden [.., H], (norm_weight [H],) w_gate_up [2F, H] (16-row interleaved). With
// norm_weight the RMSNorm (post_attention_layernorm) runs inside the kernel.
class GateUpSiluOp final : public Operator {
 public:
  std::string type() const override { return "gate_up_silu"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 3, 1, type());
    requireCudaInputs(in, type());
    for (const Tensor* t : in) requireBf16(*t, type(), "inputs");
    const Tensor& x = *in[0];
    const Tensor* nw = in.size() == 3 ? in[1] : nullptr;
    const Tensor& w = *in.back();
    const std::int64_t hidden = x.shape().back(), m = rowsOf(x);
    if (w.rank() != 2 || w.dim(1) != hidden || w.dim(0) % 2 != 0)
      throw std::invalid_argument("gate_up_silu weight shape mismatch");
    if (nw != nullptr && static_cast<std::int64_t>(nw->numel()) != hidden)
      throw std::invalid_argument("gate_up_silu norm weight size mismatch");
    const std::int64_t f = w.dim(0) / 2;
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    *out[0] = Tensor::cuda(DType::BFloat16, withLast(x.shape(), f), x.deviceId());
    check(dli_hip_gate_up_silu(ptr(x), nw ? ptr(*nw) : nullptr, ptr(w), ptr(*out[0]), m, f, hidden,
                               eps, ctx.stream),
          type());
  }
};

// inputs: xn [B, H], w [V, H] (, model.norm weight [H]: x is then the un-normalized residual
// stream and the final RMSNorm, attr eps, runs in the kernel); outputs: (logits [B, V],)
// next_ids int64 [B]
class LmHeadArgmaxOp final : public Operator {
 public:
  std::string type() const override { return "lm_head_argmax"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    if (out.size() != 1 && out.size() != 2) throw std::invalid_argument("lm_head_argmax arity");
    requireArity(in, out, 2, 3, out.size(), type());
    requireCudaInputs(in, type());
    for (const Tensor* t : in) requireBf16(*t, type(), "inputs");
    const Tensor &x = *in[0], &w = *in[1];
    const std::int64_t hidden = x.shape().back(), m = rowsOf(x);
    if (w.rank() != 2 || w.dim(1) != hidden)
      throw std::invalid_argument("lm_head_argmax weight shape mismatch");
    // optional third input: model.norm's weight, the final RMSNorm applied in the kernel
    const Tensor* norm = in.size() == 3 ? in[2] : nullptr;
    if (norm != nullptr && static_cast<std::int64_t>(norm->numel()) != hidden)
      throw std::invalid_argument("lm_head_argmax norm weight must have hidden elements");
    const float eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    const std::int64_t vocab = w.dim(0);
    const DType logits_dtype = dtypeFromString(attrs.value_or<std::string>("logits_dtype", "float32"));
    Tensor* logits = out.size() == 2 ? out[0] : nullptr;
    Tensor* ids = out.back();
    if (logits != nullptr) *logits = Tensor::cuda(logits_dtype, withLast(x.shape(), vocab), x.deviceId());
    *ids = Tensor::cuda(DType::Int64, {m}, x.deviceId());
    const std::size_t ws_bytes = dli_hip_lm_head_argmax_workspace(m, vocab);
    Tensor ws = Tensor::cuda(DType::Float32, {static_cast<std::int64_t>((ws_bytes + 3) / 4)}, x.deviceId());
    check(dli_hip_lm_head_argmax_norm(ptr(x), norm ? ptr(*norm) : nullptr, eps, ptr(w),
                                      logits ? ptr(*logits) : nullptr, hipDtype(logits_dtype),
                                      static_cast<std::int64_t*>(ptr(*ids)), m, vocab, hidden,
                                      ptr(ws), ws_bytes, ctx.stream),
          type());
  }
};

// All decoder layers in one launch (dli_hip_decoder_stack). inputs: hidden [B, H], positions
// [B], cos, sin, then per layer: input_layernorm.weight, qkv_proj.weight, qkv_proj.bias,
// o_proj.weight, post_attention_layernorm.weight, gate_up_proj.weight, down_proj.weight; then,
// optionally, a stage-timeline buffer (int64, layers x CUs x DLI_STACK_TRACE_EVENTS entries: DliStackOptions.trace).
// With token ids instead of hidden (int64/int32 [B]) the embedding table [vocab, H] follows the
// layer weights (before the timeline buffer) and the launch gathers the first layer's input
// rows itself (the model.embed_tokens node folded in: DliStackOptions.token_ids).
// Attributes: attention_splits (0 = the launch's choice; the paged_attention node's count makes
// the two bit-identical), down_splits, eps, kv_cache_prefix, check_status.
// Layer i appends to and attends over cache entry kv_cache_prefix + i. Computes what the
// five-launch layer (qkv_rope_append, paged_attention, linear_residual, gate_up_silu,
// linear_residual with down_splits) computes, bit for bit.
class DecoderStackOp final : public Operator {
 public:
  std::string type() const override { return "decoder_stack"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    constexpr std::size_t kPerLayer = 7, kHead = 4;
    const auto layers = attrs.require<std::int64_t>("layers");
    const std::size_t n_layer_in = kHead + kPerLayer * static_cast<std::size_t>(layers);
    if (layers < 1 || in.empty())
      throw std::invalid_argument("decoder_stack expects 4 + 7 * layers inputs (+ a trace buffer)");
    const bool from_ids = in[0]->dtype() == DType::Int64 || in[0]->dtype() == DType::Int32;
    const std::size_t n_in = n_layer_in + (from_ids ? 1 : 0);  // + the embedding table
    if (in.size() != n_in && in.size() != n_in + 1)
      throw std::invalid_argument(from_ids ? "decoder_stack expects token ids, 3 + 7 * layers "
                                             "inputs, the embedding table (+ a trace buffer)"
                                           : "decoder_stack expects 4 + 7 * layers inputs (+ a "
                                             "trace buffer)");
    if (out.size() != 1 && out.size() != 2)
      throw std::invalid_argument("decoder_stack outputs: hidden (, status)");
    requireArity(in, out, in.size(), in.size(), out.size(), type());
    requireCudaInputs(in, type());
    const Tensor &x = *in[0], &pos = *in[1], &cos = *in[2], &sin = *in[3];
    const Tensor* embed = from_ids ? in[n_layer_in] : nullptr;
    if (from_ids) {
      requireBf16(*embed, type(), "embedding table");
      if (embed->rank() != 2 || x.rank() != 1)
        throw std::invalid_argument("decoder_stack token ids must be [B], the table [vocab, H]");
    } else {
      requireBf16(x, type(), "hidden");
    }
    requireIndex(pos, type(), "positions");
    requireFloat(cos, type());
    requireFloat(sin, type());
    const auto hq = attrs.require<std::int64_t>("q_heads");
    const auto hkv = attrs.require<std::int64_t>("kv_heads");
    const auto d = attrs.require<std::int64_t>("head_dim");
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    const auto down_splits = attrs.value_or<std::int64_t>("down_splits", 4);
    DliStackOptions options{};
    options.attention_splits =
        static_cast<int>(attrs.value_or<std::int64_t>("attention_splits", 0));
    if (in.size() == n_in + 1) {
      const Tensor& trace = *in[n_in];
      if (trace.dtype() != DType::Int64)
        throw std::invalid_argument("decoder_stack trace buffer must be int64");
      int cus = 0;
      check(dli_hip_compute_units(&cus), type());
      const auto per_layer = static_cast<std::int64_t>(cus) * DLI_STACK_TRACE_EVENTS;
      options.trace_layers = static_cast<int>(static_cast<std::int64_t>(trace.numel()) / per_layer);
      if (options.trace_layers < 1)
        throw std::invalid_argument("decoder_stack trace buffer holds less than one layer");
      options.trace = static_cast<unsigned long long*>(ptr(trace));
    }
    const std::string prefix = attrs.value_or<std::string>("kv_cache_prefix", "layer_");
    const std::int64_t hidden = from_ids ? embed->dim(1) : x.shape().back();
    const std::int64_t m = from_ids ? static_cast<std::int64_t>(x.numel()) : rowsOf(x);
    if (from_ids) {
      options.token_ids = ptr(x);
      options.token_ids_dtype = hipDtype(x.dtype());
      options.embedding = ptr(*embed);
      options.vocab = embed->dim(0);
    }
    const std::int64_t n_qkv = (hq + 2 * hkv) * d;
    if (static_cast<std::int64_t>(pos.numel()) != m)
      throw std::invalid_argument("decoder_stack positions must have one entry per row");
    if (cos.rank() != 2 || cos.dim(1) != d / 2 || cos.shape() != sin.shape())
      throw std::invalid_argument("decoder_stack cos/sin must be [max_pos, head_dim/2]");
    if (ctx.kv_cache == nullptr) throw std::invalid_argument("decoder_stack missing KV cache");
    std::vector<DliDecoderLayer> table(static_cast<std::size_t>(layers));
    std::int64_t ffn = 0, block_size = 0, max_blocks = 0;
    for (std::int64_t i = 0; i < layers; ++i) {
      const Tensor* const* t = &in[kHead + kPerLayer * static_cast<std::size_t>(i)];
      for (std::size_t j = 0; j < kPerLayer; ++j) requireBf16(*t[j], type(), "weights");
      const Tensor &ln1 = *t[0], &wqkv = *t[1], &bqkv = *t[2], &wo = *t[3], &ln2 = *t[4],
                   &wgu = *t[5], &wd = *t[6];
      if (static_cast<std::int64_t>(ln1.numel()) != hidden ||
          static_cast<std::int64_t>(ln2.numel()) != hidden || wqkv.rank() != 2 ||
          wqkv.dim(0) != n_qkv || wqkv.dim(1) != hidden ||
          static_cast<std::int64_t>(bqkv.numel()) != n_qkv || wo.rank() != 2 ||
          wo.dim(0) != hidden || wo.dim(1) != hq * d || wgu.rank() != 2 || wgu.dim(1) != hidden ||
          wd.rank() != 2 || wd.dim(0) != hidden || 2 * wd.dim(1) != wgu.dim(0))
        throw std::invalid_argument("decoder_stack layer " + std::to_string(i) +
                                    " weight shapes do not match the attributes");
      ffn = wd.dim(1);
      KVCacheEntry& e = ctx.kv_cache->reserve(prefix + std::to_string(i), DType::BFloat16, m, hkv,
                                              d, x.deviceId());
      if (i == 0) {
        block_size = e.block_size;
        max_blocks = e.max_blocks;
      } else if (e.block_size != block_size || e.max_blocks != max_blocks) {
        throw std::invalid_argument("decoder_stack cache entries differ in geometry");
      }
      table[static_cast<std::size_t>(i)] =
          DliDecoderLayer{ptr(ln1), ptr(wqkv), ptr(bqkv), ptr(wo), ptr(ln2), ptr(wgu), ptr(wd),
                          ptr(e.key_pool), ptr(e.value_pool),
                          static_cast<const std::int32_t*>(ptr(e.block_table))};
    }
    *out[0] = Tensor::cuda(DType::BFloat16,
                           from_ids ? std::vector<std::int64_t>{m, hidden} : x.shape(),
                           x.deviceId());
    const std::size_t ws_bytes = dli_hip_decoder_stack_workspace(
        static_cast<int>(layers), m, hidden, hq, hkv, d, ffn, max_blocks,
        static_cast<int>(down_splits), options.attention_splits);
    if (ws_bytes == 0) throw std::invalid_argument("decoder_stack: unsupported geometry or splits");
    // The launch status accumulates in one persistent word per operator instance (the same
    // buffer every run, so a captured graph keeps reporting into it); the second output, when
    // the node lists one, is that word. A driver reads it after a synchronization it makes anyway
    // and zeroes it.
    void* status = status_.get(sizeof(unsigned), x.deviceId(), ctx.stream);
    check(dli_hip_decoder_stack(table.data(), static_cast<int>(layers),
                                from_ids ? nullptr : ptr(x), ptr(*out[0]),
                                ptr(pos), hipDtype(pos.dtype()),
                                static_cast<const float*>(ptr(cos)),
                                static_cast<const float*>(ptr(sin)), cos.dim(0), block_size,
                                max_blocks, m, hidden, hq, hkv, d, ffn, eps,
                                static_cast<int>(down_splits),
                                workspace_.get(ws_bytes, x.deviceId(), ctx.stream), ws_bytes,
                                static_cast<unsigned*>(status), &options, ctx.stream),
          type());
    if (out.size() == 2) *out[1] = status_.tensor().withShape({1});
    // check_status (tests): wait for the launch and fail if a wait in it gave up
    if (attrs.value_or<std::int64_t>("check_status", 0) != 0) {
      check(dli_hip_stream_synchronize(ctx.stream), type());
      at::Tensor word = status_.tensor().torchTensor();
      const bool aborted = word.item<std::int32_t>() != 0;
      if (aborted) {
        word.zero_();
        throw std::runtime_error("decoder_stack: a workgroup gave up waiting");
      }
    }
  }

 private:
  mutable PersistentWorkspace workspace_;
  mutable PersistentWorkspace status_;
};

class ArgmaxOp final : public Operator {
 public:
  std::string type() const override { return "argmax"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    const std::int64_t width = in[0]->shape().back();
    const std::int64_t rows = width > 0 ? static_cast<std::int64_t>(in[0]->numel()) / width : 0;
    std::vector<std::int64_t> shape(in[0]->shape().begin(), in[0]->shape().end() - 1);
    *out[0] = Tensor::cuda(DType::Int64, shape.empty() ? std::vector<std::int64_t>{1} : shape,
                           in[0]->deviceId());
    check(dli_hip_argmax(hipDtype(in[0]->dtype()), ptr(*in[0]),
                         static_cast<std::int64_t*>(ptr(*out[0])), rows, width, ctx.stream),
          type());
  }
};

}  // namespace

void registerFusedOps(OperatorRegistry* registry) {
  add<QkvRopeAppendOp>(registry);
  add<QkvRopeHeadsOp>(registry);
  add<PagedAttentionOp>(registry);
  add<LinearResidualOp>(registry);
  add<LinearResidualNormOp>(registry);
  add<GateUpSiluOp>(registry);
  add<LmHeadArgmaxOp>(registry);
  add<DecoderStackOp>(registry);
  add<ArgmaxOp>(registry);
}

}  // namespace dli::plugin
