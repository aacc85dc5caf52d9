// The 16 operators of the reference plugin (python/dli_ops/aot/*/template.cc), with the same
// registry names, arity, attributes and defaults, running on the gfx950 kernels of
// libdli_hip.so. Extensions over the reference (documented per op): bfloat16 / float16 data,
// any shape (no fixed AOT specialisations), grouped KV heads, per-sequence positions.
#include <cmath>

#include "common.h"

namespace dli::plugin {
namespace {

Tensor allocLike(DType dtype, std::vector<std::int64_t> shape, const Tensor& ref) {
  return Tensor::cuda(dtype, std::move(shape), ref.deviceId());
}

// add/template.cc:7-14, mul/template.cc:7-14 — out = a + b (b repeats over a's trailing elements).
template <bool kMul>
class BroadcastOp final : public Operator {
 public:
  std::string type() const override { return kMul ? "mul" : "add"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    *out[0] = allocLike(in[0]->dtype(), in[0]->shape(), *in[0]);
    const auto total = static_cast<std::int64_t>(in[0]->numel());
    const auto width = static_cast<std::int64_t>(in[1]->numel());
    if (total > 0 && width == 0) throw std::invalid_argument(type() + " broadcast operand is empty");
    auto fn = kMul ? dli_hip_mul : dli_hip_add;
    check(fn(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*in[1]), ptr(*out[0]), total, width,
             ctx.stream),
          type());
  }
};

// silu/template.cc, relu/template.cc — elementwise activations.
template <bool kRelu>
class ActivationOp final : public Operator {
 public:
  std::string type() const override { return kRelu ? "relu" : "silu"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    *out[0] = allocLike(in[0]->dtype(), in[0]->shape(), *in[0]);
    auto fn = kRelu ? dli_hip_relu : dli_hip_silu;
    check(fn(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*out[0]),
             static_cast<std::int64_t>(in[0]->numel()), ctx.stream),
          type());
  }
};

// rms_norm/template.cc:18-26 — one row per element of x.shape[:-1]; attr eps (default 1e-6).
class RmsNormOp final : public Operator {
 public:
  std::string type() const override { return "rms_norm"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    const std::int64_t hidden = in[0]->shape().back();
    if (static_cast<std::int64_t>(in[1]->numel()) != hidden)
      throw std::invalid_argument("rms_norm weight size must match the last input dim");
    const std::int64_t rows = hidden > 0 ? static_cast<std::int64_t>(in[0]->numel()) / hidden : 0;
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-6));
    *out[0] = allocLike(in[0]->dtype(), in[0]->shape(), *in[0]);
    check(dli_hip_rms_norm(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*in[1]), ptr(*out[0]), rows,
                           hidden, eps, ctx.stream),
          type());
  }
};

// embedding/template.cc:18-29 — out[..., :] = table[ids[...], :].
class EmbeddingOp final : public Operator {
 public:
  std::string type() const override { return "embedding"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireCudaInputs(in, type());
    requireIndex(*in[0], type(), "ids");
    requireFloating(*in[1], type());
    if (in[1]->rank() != 2) throw std::invalid_argument("embedding table must be 2-D");
    auto shape = in[0]->shape();
    shape.push_back(in[1]->dim(1));
    *out[0] = allocLike(in[1]->dtype(), shape, *in[0]);
    check(dli_hip_embedding(hipDtype(in[1]->dtype()), hipDtype(in[0]->dtype()), ptr(*in[0]),
                            ptr(*in[1]), ptr(*out[0]), static_cast<std::int64_t>(in[0]->numel()),
                            in[1]->dim(1), in[1]->dim(0), ctx.stream),
          type());
  }
};

// Extension attribute of linear and conv2d: activation = "relu" applies ReLU in the GEMM
// epilogue (the reference graph has a separate relu node instead). Absent or "none": no
// activation.
int activationAttr(const Attributes& attrs, const std::string& op) {
  const std::string a = attrs.value_or<std::string>("activation", "none");
  if (a == "none") return DLI_ACT_NONE;
  if (a == "relu") return DLI_ACT_RELU;
  throw std::invalid_argument(op + ": unsupported activation " + a);
}

// linear/template.cc:20-32 — x [..., k] * w[n, k]^T (+ b[n]). Extension: attr
// out_dtype = "float32" keeps an fp32 result for low-precision inputs (e.g. logits); attr
// activation (above).
class LinearOp final : public Operator {
 public:
  std::string type() const override { return "linear"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 3, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    if (in[1]->rank() != 2) throw std::invalid_argument("linear weight must be 2-D");
    const std::int64_t k = in[0]->shape().back();
    if (in[1]->dim(1) != k)
      throw std::invalid_argument("linear weight shape " + formatShape(in[1]->shape()) +
                                  " does not match input " + formatShape(in[0]->shape()));
    const std::int64_t n = in[1]->dim(0);
    const bool has_bias = in.size() == 3;
    if (has_bias) {
      requireSameDType(*in[0], *in[2], type());
      if (static_cast<std::int64_t>(in[2]->numel()) != n)
        throw std::invalid_argument("linear bias size must match the output features");
    }
    const std::int64_t m = product(in[0]->shape(), 0, in[0]->rank() - 1);
    DType out_dtype = in[0]->dtype();
    const std::string requested = attrs.value_or<std::string>("out_dtype", "");
    if (!requested.empty()) out_dtype = dtypeFromString(requested);
    *out[0] = allocLike(out_dtype, withLast(in[0]->shape(), n), *in[0]);
    const int act = activationAttr(attrs, type());
    const int dt = hipDtype(in[0]->dtype());
    // split-K scratch for fp32 shapes with few output tiles (from the caching allocator)
    const std::size_t ws_bytes = dli_hip_linear_workspace(dt, m, n, k);
    Tensor ws;
    if (ws_bytes > 0)
      ws = allocLike(DType::Float32, {static_cast<std::int64_t>(ws_bytes / sizeof(float))}, *in[0]);
    check(dli_hip_linear_act(dt, hipDtype(out_dtype), ptr(*in[0]), ptr(*in[1]),
                             has_bias ? ptr(*in[2]) : nullptr, ptr(*out[0]), m, n, k, act,
                             ws_bytes > 0 ? ptr(ws) : nullptr, ws_bytes, ctx.stream),
          type());
  }
};

// matmul/template.cc:20-28 — a [m, k] @ b [k, n].
class MatmulOp final : public Operator {
 public:
  std::string type() const override { return "matmul"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    if (in[0]->rank() != 2 || in[1]->rank() != 2 || in[0]->dim(1) != in[1]->dim(0))
      throw std::invalid_argument("matmul expects [m,k] @ [k,n]");
    const std::int64_t m = in[0]->dim(0), k = in[0]->dim(1), n = in[1]->dim(1);
    *out[0] = allocLike(in[0]->dtype(), {m, n}, *in[0]);
    check(dli_hip_matmul(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*in[1]), ptr(*out[0]), m, n, k,
                         ctx.stream),
          type());
  }
};

// rotary/template.cc:7-26 — interleaved-pair RoPE on q and k at start_pos + token.
// Extensions: q and k may have different head counts; the optional 5th input (unused by the
// reference) is a per-sequence position offset, int32/int64 [batch].
class RotaryOp final : public Operator {
 public:
  std::string type() const override { return "rotary_embedding"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 4, 5, 2, type());
    requireCudaInputs(in, type());
    const Tensor& q = *in[0];
    const Tensor& k = *in[1];
    requireFloating(q, type());
    requireSameDType(q, k, type());
    if (q.rank() != 4 || k.rank() != 4) throw std::invalid_argument("rotary_embedding expects rank-4 q and k");
    if (q.dim(0) != k.dim(0) || q.dim(2) != k.dim(2) || q.dim(3) != k.dim(3))
      throw std::invalid_argument("rotary_embedding q/k shapes disagree");
    requireFloat(*in[2], type());
    requireFloat(*in[3], type());
    if (in[2]->rank() != 2 || in[2]->shape() != in[3]->shape())
      throw std::invalid_argument("rotary_embedding cos/sin must be [max_pos, pairs]");
    const Tensor* positions = in.size() == 5 ? in[4] : nullptr;
    if (positions != nullptr) {
      requireIndex(*positions, type(), "positions");
      if (static_cast<std::int64_t>(positions->numel()) != q.dim(0))
        throw std::invalid_argument("rotary_embedding positions must have one entry per sequence");
    }
    const std::int64_t start_pos = attrs.value_or<std::int64_t>("start_pos", 0);
    *out[0] = allocLike(q.dtype(), q.shape(), q);
    *out[1] = allocLike(k.dtype(), k.shape(), k);
    check(dli_hip_rotary(hipDtype(q.dtype()), ptr(q), ptr(k),
                         static_cast<const float*>(ptr(*in[2])),
                         static_cast<const float*>(ptr(*in[3])), ptr(*out[0]), ptr(*out[1]),
                         q.dim(0), q.dim(1), k.dim(1), q.dim(2), q.dim(3), in[2]->dim(1),
                         in[2]->dim(0), start_pos, positions ? ptr(*positions) : nullptr,
                         positions ? hipDtype(positions->dtype()) : DLI_I64, ctx.stream),
          type());
  }
};

// attention/template.cc:7-47 — softmax(q k^T / sqrt(D)) v with attrs causal (false) and
// kv_cache (""). With kv_cache the new k/v are appended to the named cache entry first and q
// attends over everything cached. Extensions: grouped KV heads (Hq % Hkv == 0), an optional
// `scale` attr, an optional 4th input `positions` (int32/int64 [batch]: tokens already cached
// per sequence; the new tokens are written at those positions).
class AttentionOp final : public Operator {
 public:
  std::string type() const override { return "attention"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 3, 4, 1, type());
    requireCudaInputs(in, type());
    const Tensor& q = *in[0];
    const Tensor& k = *in[1];
    const Tensor& v = *in[2];
    requireFloating(q, type());
    requireSameDType(q, k, type());
    requireSameDType(q, v, type());
    if (q.rank() != 4 || k.rank() != 4 || v.rank() != 4)
      throw std::invalid_argument("attention expects rank-4 [B,H,S,D] tensors");
    if (k.shape() != v.shape() || q.dim(0) != k.dim(0) || q.dim(3) != k.dim(3))
      throw std::invalid_argument("attention q/k/v shapes disagree");
    const std::int64_t B = q.dim(0), Hq = q.dim(1), Sq = q.dim(2), D = q.dim(3), Hkv = k.dim(1);
    if (Hkv <= 0 || Hq % Hkv != 0)
      throw std::invalid_argument("attention q heads must be a multiple of kv heads");
    const bool causal = attrs.value_or<bool>("causal", false);
    const float scale = static_cast<float>(attrDouble(attrs, "scale", 1.0 / std::sqrt(static_cast<double>(D))));
    const std::string cache_name = attrs.value_or<std::string>("kv_cache", "");
    const Tensor* positions = in.size() == 4 ? in[3] : nullptr;
    if (positions != nullptr) {
      requireIndex(*positions, type(), "positions");
      if (static_cast<std::int64_t>(positions->numel()) != B)
        throw std::invalid_argument("attention positions must have one entry per sequence");
    }
    // extension: output_layout "bshd" returns [B, S, H, D] (the layout a prompt's transpose node
    // after attention makes), written by the flash kernel directly
    const std::string layout = attrs.value_or<std::string>("output_layout", "bhsd");
    if (layout != "bhsd" && layout != "bshd")
      throw std::invalid_argument("attention output_layout must be \"bhsd\" or \"bshd\"");
    const bool bshd = layout == "bshd";
    *out[0] = allocLike(q.dtype(), bshd ? std::vector<std::int64_t>{B, Sq, Hq, D} : q.shape(), q);
    const int dt = hipDtype(q.dtype());
    auto contiguous = [&](const Tensor& kk, const Tensor& vv) {
      auto fn = bshd ? dli_hip_attention_bshd : dli_hip_attention;
      check(fn(dt, ptr(q), ptr(kk), ptr(vv), ptr(*out[0]), B, Hq, Hkv, Sq, kk.dim(2), D,
               causal ? 1 : 0, scale, ctx.stream),
            type());
    };

    if (cache_name.empty()) {
      if (positions != nullptr) throw std::invalid_argument("attention positions require kv_cache");
      contiguous(k, v);
      return;
    }
    if (ctx.kv_cache == nullptr) throw std::invalid_argument("attention missing KV cache");
    KVCache& cache = *ctx.kv_cache;
    std::int64_t past = 0;
    if (positions != nullptr) {
      cache.appendAt(cache_name, k, v, *positions);
    } else {
      const KVCacheEntry* before = cache.get(cache_name);
      past = before ? before->length : 0;
      cache.append(cache_name, k, v);
    }
    if (positions == nullptr && past == 0) {
      // A prompt from an empty cache: the cache now holds exactly k and v, so attending over
      // them directly is the same computation, and runs on the contiguous (flash) kernel.
      contiguous(k, v);
      return;
    }
    if (bshd) throw std::invalid_argument("attention output_layout \"bshd\" needs an empty cache");
    const KVCacheEntry& e = *cache.get(cache_name);
    const std::size_t ws_bytes = dli_hip_paged_attention_workspace(B, Hq, Sq, D, e.capacity());
    check(dli_hip_paged_attention(
              dt, ptr(q), ptr(e.key_pool), ptr(e.value_pool),
              static_cast<const std::int32_t*>(ptr(e.block_table)), ptr(*out[0]), B, Hq, Hkv, Sq,
              D, e.block_size, e.max_blocks, past, positions ? ptr(*positions) : nullptr,
              positions ? hipDtype(positions->dtype()) : DLI_I64, causal ? 1 : 0, scale, 0,
              workspace_.get(ws_bytes, q.deviceId(), ctx.stream), ws_bytes, ctx.stream),
          type());
  }

 private:
  mutable PersistentWorkspace workspace_;
};

// reshape/template.cc:7-9 — a view; one dim may be -1.
class ReshapeOp final : public Operator {
 public:
  std::string type() const override { return "reshape"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    *out[0] = in[0]->withShape(
        reshapeShape(in[0]->shape(), attrs.require<std::vector<std::int64_t>>("shape")));
  }
};

// softmax/template.cc:26-35 — over the last dim (any width here; the reference stops at 512).
class SoftmaxOp final : public Operator {
 public:
  std::string type() const override { return "softmax"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext& ctx) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    const std::int64_t width = in[0]->shape().back();
    const std::int64_t rows = width > 0 ? static_cast<std::int64_t>(in[0]->numel()) / width : 0;
    *out[0] = allocLike(in[0]->dtype(), in[0]->shape(), *in[0]);
    check(dli_hip_softmax(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*out[0]), rows, width,
                          ctx.stream),
          type());
  }
};

// transpose/template.cc:7-18 — 2-D, perm [1, 0]. Extension: rank 4 with perm [0, 2, 1, 3] (the
// [B, S, H, D] <-> [B, H, S, D] change a prefill graph needs around rotary and attention).
class TransposeOp final : public Operator {
 public:
  std::string type() const override { return "transpose"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    const auto perm = attrs.require<std::vector<std::int64_t>>("perm");
    if (in[0]->rank() == 4 && perm == std::vector<std::int64_t>{0, 2, 1, 3}) {
      const Tensor& x = *in[0];
      *out[0] = allocLike(x.dtype(), {x.dim(0), x.dim(2), x.dim(1), x.dim(3)}, x);
      check(dli_hip_permute_0213(hipDtype(x.dtype()), ptr(x), ptr(*out[0]), x.dim(0), x.dim(1),
                                 x.dim(2), x.dim(3), ctx.stream),
            type());
      return;
    }
    if (in[0]->rank() != 2 || perm != std::vector<std::int64_t>{1, 0})
      throw std::invalid_argument("transpose supports 2D perm [1,0] and 4D perm [0,2,1,3]");
    const std::int64_t rows = in[0]->dim(0), cols = in[0]->dim(1);
    *out[0] = allocLike(in[0]->dtype(), {cols, rows}, *in[0]);
    check(dli_hip_transpose2d(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*out[0]), rows, cols,
                              ctx.stream),
          type());
  }
};

std::int64_t pooledExtent(std::int64_t in, std::int64_t k, std::int64_t s, std::int64_t p) {
  return (in + 2 * p - k) / s + 1;
}

// conv2d/template.cc:7-35 — NCHW convolution; attrs stride [1,1], padding [0,0]; extension
// attr activation (above).
class Conv2dOp final : public Operator {
 public:
  std::string type() const override { return "conv2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 2, 3, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    for (const Tensor* t : in) requireSameDType(*in[0], *t, type());
    const Tensor& x = *in[0];
    const Tensor& w = *in[1];
    if (x.rank() != 4 || w.rank() != 4 || x.dim(1) != w.dim(1))
      throw std::invalid_argument("conv2d expects NCHW input and [OC, C, KH, KW] weight");
    const auto stride = attrInts(attrs, "stride", {1, 1});
    const auto pad = attrInts(attrs, "padding", {0, 0});
    if (stride.size() != 2 || pad.size() != 2) throw std::invalid_argument("conv2d stride/padding must have 2 entries");
    const std::int64_t n = x.dim(0), c = x.dim(1), h = x.dim(2), wd = x.dim(3);
    const std::int64_t oc = w.dim(0), kh = w.dim(2), kw = w.dim(3);
    const std::int64_t oh = pooledExtent(h, kh, stride[0], pad[0]);
    const std::int64_t ow = pooledExtent(wd, kw, stride[1], pad[1]);
    if (oh <= 0 || ow <= 0) throw std::invalid_argument("conv2d output would be empty");
    const bool has_bias = in.size() == 3;
    if (has_bias && static_cast<std::int64_t>(in[2]->numel()) != oc)
      throw std::invalid_argument("conv2d bias size must match output channels");
    const int act = activationAttr(attrs, type());
    *out[0] = allocLike(x.dtype(), {n, oc, oh, ow}, x);
    const int dt = hipDtype(x.dtype());
    const std::size_t ws_bytes = dli_hip_conv2d_workspace(dt, n, c, oc, kh, kw, oh, ow);
    Tensor ws;
    if (ws_bytes > 0)
      ws = allocLike(DType::Float32, {static_cast<std::int64_t>(ws_bytes / sizeof(float))}, x);
    check(dli_hip_conv2d_act(dt, ptr(x), ptr(w), has_bias ? ptr(*in[2]) : nullptr, ptr(*out[0]),
                             n, c, h, wd, oc, kh, kw, oh, ow, stride[0], stride[1], pad[0],
                             pad[1], act, ws_bytes > 0 ? ptr(ws) : nullptr, ws_bytes, ctx.stream),
          type());
  }
};

// max_pool2d/template.cc:7-28 — attrs kernel_size [2,2], stride (= kernel_size), padding [0,0].
class MaxPool2dOp final : public Operator {
 public:
  std::string type() const override { return "max_pool2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    const Tensor& x = *in[0];
    if (x.rank() != 4) throw std::invalid_argument("max_pool2d expects NCHW input");
    const auto ks = attrInts(attrs, "kernel_size", {2, 2});
    const auto stride = attrInts(attrs, "stride", ks);
    const auto pad = attrInts(attrs, "padding", {0, 0});
    if (ks.size() != 2 || stride.size() != 2 || pad.size() != 2)
      throw std::invalid_argument("max_pool2d kernel_size/stride/padding must have 2 entries");
    const std::int64_t n = x.dim(0), c = x.dim(1), h = x.dim(2), w = x.dim(3);
    const std::int64_t oh = pooledExtent(h, ks[0], stride[0], pad[0]);
    const std::int64_t ow = pooledExtent(w, ks[1], stride[1], pad[1]);
    if (oh <= 0 || ow <= 0) throw std::invalid_argument("max_pool2d output would be empty");
    *out[0] = allocLike(x.dtype(), {n, c, oh, ow}, x);
    check(dli_hip_max_pool2d(hipDtype(x.dtype()), ptr(x), ptr(*out[0]), n, c, h, w, oh, ow, ks[0],
                             ks[1], stride[0], stride[1], pad[0], pad[1], ctx.stream),
          type());
  }
};

// batch_norm2d/template.cc:7-31 — eval-mode BN; inputs x, weight, bias, mean, var; eps 1e-5.
class BatchNorm2dOp final : public Operator {
 public:
  std::string type() const override { return "batch_norm2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 5, 5, 1, type());
    requireCudaInputs(in, type());
    requireFloating(*in[0], type());
    for (const Tensor* t : in) requireSameDType(*in[0], *t, type());
    if (in[0]->rank() != 4) throw std::invalid_argument("batch_norm2d expects NCHW input");
    const std::int64_t channels = in[0]->dim(1);
    for (std::size_t i = 1; i < in.size(); ++i)
      if (static_cast<std::int64_t>(in[i]->numel()) != channels)
        throw std::invalid_argument("batch_norm2d parameter size must match input channels");
    const auto eps = static_cast<float>(attrDouble(attrs, "eps", 1e-5));
    *out[0] = allocLike(in[0]->dtype(), in[0]->shape(), *in[0]);
    check(dli_hip_batch_norm2d(hipDtype(in[0]->dtype()), ptr(*in[0]), ptr(*in[1]), ptr(*in[2]),
                               ptr(*in[3]), ptr(*in[4]), ptr(*out[0]),
                               static_cast<std::int64_t>(in[0]->numel()), channels,
                               in[0]->dim(2) * in[0]->dim(3), eps, ctx.stream),
          type());
  }
};

}  // namespace

void registerReferenceOps(OperatorRegistry* registry) {
  add<BroadcastOp<false>>(registry);
  add<BroadcastOp<true>>(registry);
  add<ActivationOp<false>>(registry);
  add<ActivationOp<true>>(registry);
  add<RmsNormOp>(registry);
  add<EmbeddingOp>(registry);
  add<LinearOp>(registry);
  add<MatmulOp>(registry);
  add<RotaryOp>(registry);
  add<AttentionOp>(registry);
  add<ReshapeOp>(registry);
  add<SoftmaxOp>(registry);
  add<TransposeOp>(registry);
  add<Conv2dOp>(registry);
  add<MaxPool2dOp>(registry);
  add<BatchNorm2dOp>(registry);
}

}  // namespace dli::plugin
