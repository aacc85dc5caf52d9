// ATen CPU reference plugin (lib/libdli_aten_ops.so): the reference plugin's 16 operator names
// (python/dli_ops/aot/*/template.cc), plus the decode graph's argmax, implemented with ATen on
// host tensors. It runs the same dli.graph.v1 graphs as the gfx950 plugin through the same
// Engine, so the CPU time of a graph is measured on the reference's own runtime path (Engine ->
// registry -> operator), with ATen's CPU kernels in place of the device kernels.
//
// Numerics follow the reference kernels (cited per op) with the gfx950 plugin's extensions
// (bfloat16/float16 data, grouped KV heads, per-sequence positions): every op computes in fp32
// and rounds its output to the input dtype once, the rounding points of the device path. The
// paged KV cache keeps host entries (include/dli/kv_cache.h: one block per sequence).
#include <ATen/ATen.h>

#include <cmath>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "dli/kv_cache.h"
#include "dli/operator.h"
#include "dli/utils.h"

namespace dli::aten_plugin {
namespace {

void requireHost(const std::vector<const Tensor*>& in, const std::string& op) {
  for (const Tensor* t : in) {
    if (t == nullptr) throw std::invalid_argument(op + " received a null input");
    if (!t->isCpu()) throw std::invalid_argument(op + " (ATen CPU plugin) expects host tensors");
  }
}

void requireArity(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
                  std::size_t min_in, std::size_t max_in, std::size_t n_out, const std::string& op) {
  if (in.size() < min_in || in.size() > max_in || out.size() != n_out)
    throw std::invalid_argument(op + " arity");
  for (Tensor* t : out)
    if (t == nullptr) throw std::invalid_argument(op + " received a null output");
  requireHost(in, op);
}

at::Tensor f32(const Tensor& t) { return t.torchTensor().to(at::kFloat); }

// Rounds an fp32 result to the dtype of the node (the graph's rounding point).
Tensor result(const at::Tensor& value, DType dtype) {
  return Tensor(value.to(toTorchDType(dtype)).contiguous());
}

void requireIndex(const Tensor& t, const std::string& op, const std::string& what) {
  if (t.dtype() != DType::Int64 && t.dtype() != DType::Int32)
    throw std::invalid_argument(op + " " + what + " must be int64 or int32");
}

// add/kernel.py:6-11, mul/kernel.py:6-11: out[i] = a[i] op b[i % numel(b)].
template <bool kMul>
class BroadcastOp final : public Operator {
 public:
  std::string type() const override { return kMul ? "mul" : "add"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    const auto total = static_cast<std::int64_t>(in[0]->numel());
    const auto width = static_cast<std::int64_t>(in[1]->numel());
    if (total > 0 && width == 0) throw std::invalid_argument(type() + " broadcast operand is empty");
    at::Tensor a = f32(*in[0]).reshape({-1});
    at::Tensor b = f32(*in[1]).reshape({-1});
    if (width != total) b = b.index_select(0, at::arange(total, at::kLong).remainder(width));
    *out[0] = result((kMul ? a * b : a + b).view(in[0]->torchTensor().sizes()), in[0]->dtype());
  }
};

// silu/kernel.py:6-10 (x / (1 + exp(-x))), relu/kernel.py:6-10.
template <bool kRelu>
class ActivationOp final : public Operator {
 public:
  std::string type() const override { return kRelu ? "relu" : "silu"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireFloating(*in[0], type());
    const at::Tensor x = f32(*in[0]);
    *out[0] = result(kRelu ? at::relu(x) : x / (1 + at::exp(-x)), in[0]->dtype());
  }
};

// softmax/kernel.py:6-14: over the last dim.
class SoftmaxOp final : public Operator {
 public:
  std::string type() const override { return "softmax"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireFloating(*in[0], type());
    *out[0] = result(at::softmax(f32(*in[0]), -1), in[0]->dtype());
  }
};

// rms_norm/kernel.py:6-14: x * rsqrt(mean(x^2) + eps) * w over the last dim; attr eps.
class RmsNormOp final : public Operator {
 public:
  std::string type() const override { return "rms_norm"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    if (static_cast<std::int64_t>(in[1]->numel()) != in[0]->shape().back())
      throw std::invalid_argument("rms_norm weight size must match the last input dim");
    const double eps = attrDouble(attrs, "eps", 1e-6);
    const at::Tensor x = f32(*in[0]);
    const at::Tensor r = at::rsqrt((x * x).mean({-1}, true) + eps);
    *out[0] = result(x * r * f32(*in[1]), in[0]->dtype());
  }
};

// embedding/kernel.py:6-23: out[..., :] = table[ids[...], :]; an id outside [0, vocab) gives a
// zero row (the device plugin's rule).
class EmbeddingOp final : public Operator {
 public:
  std::string type() const override { return "embedding"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireIndex(*in[0], type(), "ids");
    requireFloating(*in[1], type());
    if (in[1]->rank() != 2) throw std::invalid_argument("embedding table must be 2-D");
    const at::Tensor& table = in[1]->torchTensor();
    const at::Tensor ids = in[0]->torchTensor().to(at::kLong);
    const at::Tensor valid = (ids >= 0).logical_and(ids < table.size(0));
    at::Tensor rows = table.index_select(0, ids.where(valid, at::zeros_like(ids)).reshape({-1}));
    rows = rows * valid.reshape({-1, 1}).to(rows.scalar_type());
    auto shape = in[0]->shape();
    shape.push_back(in[1]->dim(1));
    *out[0] = Tensor(rows.reshape(shape).contiguous());
  }
};

// linear/kernel.py:6-44, linear/template.cc:20-32: x [..., k] w[n, k]^T (+ b[n]). Extensions
// as the device plugin: attr out_dtype, attr activation = "relu".
class LinearOp final : public Operator {
 public:
  std::string type() const override { return "linear"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 2, 3, 1, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    if (in[1]->rank() != 2 || in[1]->dim(1) != in[0]->shape().back())
      throw std::invalid_argument("linear weight shape " + formatShape(in[1]->shape()) +
                                  " does not match input " + formatShape(in[0]->shape()));
    if (in.size() == 3) {
      requireSameDType(*in[0], *in[2], type());
      if (static_cast<std::int64_t>(in[2]->numel()) != in[1]->dim(0))
        throw std::invalid_argument("linear bias size must match the output features");
    }
    const bool fp32 = in[0]->dtype() == DType::Float32;
    at::Tensor y = at::linear(fp32 ? in[0]->torchTensor() : f32(*in[0]),
                              fp32 ? in[1]->torchTensor() : f32(*in[1]),
                              in.size() == 3 ? c10::optional<at::Tensor>(f32(*in[2]))
                                             : c10::nullopt);
    const std::string act = attrs.value_or<std::string>("activation", "none");
    if (act == "relu") y = at::relu(y);
    else if (act != "none") throw std::invalid_argument("linear: unsupported activation " + act);
    const std::string requested = attrs.value_or<std::string>("out_dtype", "");
    *out[0] = result(y, requested.empty() ? in[0]->dtype() : dtypeFromString(requested));
  }
};

// The device plugin's linear_residual (o_proj / down_proj with their residual add):
// out = residual + round(x W^T (+ b)); inputs x, w, residual (, bias); attr splits ignored.
class LinearResidualOp final : public Operator {
 public:
  std::string type() const override { return "linear_residual"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 3, 4, 1, type());
    requireFloating(*in[0], type());
    for (const Tensor* t : in) requireSameDType(*in[0], *t, type());
    if (in[1]->rank() != 2 || in[1]->dim(1) != in[0]->shape().back())
      throw std::invalid_argument("linear_residual weight shape mismatch");
    at::Tensor y = at::linear(f32(*in[0]), f32(*in[1]),
                              in.size() == 4 ? c10::optional<at::Tensor>(f32(*in[3]))
                                             : c10::nullopt);
    y = y.to(toTorchDType(in[0]->dtype())).to(at::kFloat);  // the linear node's rounding point
    const at::Tensor res = f32(*in[2]);
    if (res.numel() != y.numel()) throw std::invalid_argument("linear_residual residual shape");
    *out[0] = result(res.view(y.sizes()) + y, in[0]->dtype());
  }
};

// matmul/kernel.py:6-40: a [m, k] @ b [k, n].
class MatmulOp final : public Operator {
 public:
  std::string type() const override { return "matmul"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 2, 2, 1, type());
    requireFloating(*in[0], type());
    requireSameDType(*in[0], *in[1], type());
    if (in[0]->rank() != 2 || in[1]->rank() != 2 || in[0]->dim(1) != in[1]->dim(0))
      throw std::invalid_argument("matmul expects [m,k] @ [k,n]");
    *out[0] = result(at::matmul(f32(*in[0]), f32(*in[1])), in[0]->dtype());
  }
};

// rotary/kernel.py:6-35: interleaved pairs at position start_pos + token (+ positions[b], the
// optional 5th input); pairs = cos.shape[1]; positions outside [0, max_pos) leave the pair as it
// is; q and k may have different head counts.
class RotaryOp final : public Operator {
 public:
  std::string type() const override { return "rotary_embedding"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 4, 5, 2, type());
    const Tensor& q = *in[0];
    const Tensor& k = *in[1];
    requireFloating(q, type());
    requireSameDType(q, k, type());
    if (q.rank() != 4 || k.rank() != 4 || q.dim(0) != k.dim(0) || q.dim(2) != k.dim(2) ||
        q.dim(3) != k.dim(3))
      throw std::invalid_argument("rotary_embedding q/k shapes disagree");
    requireFloat(*in[2], type());
    requireFloat(*in[3], type());
    if (in[2]->rank() != 2 || in[2]->shape() != in[3]->shape())
      throw std::invalid_argument("rotary_embedding cos/sin must be [max_pos, pairs]");
    const std::int64_t B = q.dim(0), S = q.dim(2), D = q.dim(3);
    const std::int64_t pairs = in[2]->dim(1), max_pos = in[2]->dim(0);
    if (2 * pairs > D) throw std::invalid_argument("rotary_embedding has more pairs than head_dim/2");
    at::Tensor pos = at::arange(S, at::kLong).view({1, S}).expand({B, S}) +
                     attrs.value_or<std::int64_t>("start_pos", 0);
    if (in.size() == 5) {
      requireIndex(*in[4], type(), "positions");
      if (static_cast<std::int64_t>(in[4]->numel()) != B)
        throw std::invalid_argument("rotary_embedding positions must have one entry per sequence");
      pos = pos + in[4]->torchTensor().to(at::kLong).view({B, 1});
    }
    const at::Tensor inside = (pos >= 0).logical_and(pos < max_pos);  // [B, S]
    const at::Tensor safe = pos.where(inside, at::zeros_like(pos)).reshape({-1});
    // [B, 1, S, pairs]; outside the table: cos 1, sin 0
    at::Tensor c = in[2]->torchTensor().index_select(0, safe).view({B, 1, S, pairs});
    at::Tensor s = in[3]->torchTensor().index_select(0, safe).view({B, 1, S, pairs});
    const at::Tensor m = inside.view({B, 1, S, 1});
    c = c.where(m, at::ones_like(c));
    s = s.where(m, at::zeros_like(s));
    auto rotate = [&](const Tensor& t) {
      at::Tensor x = f32(t).clone();
      at::Tensor head = x.narrow(3, 0, 2 * pairs).view({B, t.dim(1), S, pairs, 2});
      const at::Tensor x0 = head.select(4, 0).clone(), x1 = head.select(4, 1).clone();
      head.select(4, 0).copy_(x0 * c - x1 * s);
      head.select(4, 1).copy_(x0 * s + x1 * c);
      return result(x, t.dtype());
    };
    *out[0] = rotate(q);
    *out[1] = rotate(k);
  }
};

// attention/kernel.py:6-62: softmax(q k^T * scale) v with the causal rule key <= (seq_k - seq_q)
// + query; attrs causal (false), kv_cache (""), scale (1/sqrt(D)). With kv_cache the new k/v go
// into the named cache entry (at positions[b], the optional 4th input, else at the host-tracked
// length) and q attends over everything the sequence has cached. Grouped KV heads.
class AttentionOp final : public Operator {
 public:
  std::string type() const override { return "attention"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext& ctx) const override {
    requireArity(in, out, 3, 4, 1, type());
    const Tensor& q = *in[0];
    const Tensor& k = *in[1];
    const Tensor& v = *in[2];
    requireFloating(q, type());
    requireSameDType(q, k, type());
    requireSameDType(q, v, type());
    if (q.rank() != 4 || k.rank() != 4 || v.rank() != 4 || k.shape() != v.shape() ||
        q.dim(0) != k.dim(0) || q.dim(3) != k.dim(3))
      throw std::invalid_argument("attention q/k/v shapes disagree");
    const std::int64_t B = q.dim(0), Hq = q.dim(1), Sq = q.dim(2), D = q.dim(3), Hkv = k.dim(1);
    if (Hkv <= 0 || Hq % Hkv != 0)
      throw std::invalid_argument("attention q heads must be a multiple of kv heads");
    const std::int64_t group = Hq / Hkv;
    const bool causal = attrs.value_or<bool>("causal", false);
    const double scale = attrDouble(attrs, "scale", 1.0 / std::sqrt(static_cast<double>(D)));
    const std::string cache_name = attrs.value_or<std::string>("kv_cache", "");
    const Tensor* positions = in.size() == 4 ? in[3] : nullptr;
    if (positions != nullptr) {
      requireIndex(*positions, type(), "positions");
      if (static_cast<std::int64_t>(positions->numel()) != B)
        throw std::invalid_argument("attention positions must have one entry per sequence");
    }
    const at::Tensor qf = f32(q).view({B, Hkv, group * Sq, D});
    at::Tensor o = at::empty({B, Hkv, group * Sq, D}, at::kFloat);

    // one sequence: keys [Hkv, L, D], values given as V^T [Hkv, D, L], past = L - Sq
    auto attend = [&](std::int64_t b, const at::Tensor& keys, const at::Tensor& values_t,
                      std::int64_t past) {
      const std::int64_t L = keys.size(1);
      at::Tensor scores = at::matmul(qf[b], keys.transpose(-1, -2)) * scale;  // [Hkv, g*Sq, L]
      if (causal) {
        const at::Tensor query = at::arange(Sq, at::kLong).repeat({group}).view({group * Sq, 1});
        const at::Tensor key = at::arange(L, at::kLong).view({1, L});
        scores = scores.masked_fill(key > query + past, -INFINITY);
      }
      o[b].copy_(at::matmul(at::softmax(scores, -1), values_t.transpose(-1, -2)));
    };

    if (cache_name.empty()) {
      if (positions != nullptr) throw std::invalid_argument("attention positions require kv_cache");
      const at::Tensor kf = f32(k), vf = f32(v);
      for (std::int64_t b = 0; b < B; ++b)
        attend(b, kf[b], vf[b].transpose(-1, -2), k.dim(2) - Sq);
    } else {
      if (ctx.kv_cache == nullptr) throw std::invalid_argument("attention missing KV cache");
      KVCache& cache = *ctx.kv_cache;
      std::vector<std::int64_t> past(static_cast<std::size_t>(B), 0);
      if (positions != nullptr) {
        cache.appendAt(cache_name, k, v, *positions);
        const at::Tensor p = positions->torchTensor().to(at::kLong).contiguous();
        for (std::int64_t b = 0; b < B; ++b) past[static_cast<std::size_t>(b)] = p[b].item<std::int64_t>();
      } else {
        const KVCacheEntry* before = cache.get(cache_name);
        const std::int64_t length = before ? before->length : 0;
        cache.append(cache_name, k, v);
        for (auto& p : past) p = length;
      }
      const KVCacheEntry& e = *cache.get(cache_name);
      const at::Tensor& kp = e.key_pool.torchTensor();    // [B, Hkv, capacity, D]
      const at::Tensor& vp = e.value_pool.torchTensor();  // [B, Hkv, D, capacity]
      for (std::int64_t b = 0; b < B; ++b) {
        const std::int64_t L = past[static_cast<std::size_t>(b)] + Sq;
        attend(b, kp[b].narrow(1, 0, L).to(at::kFloat), vp[b].narrow(2, 0, L).to(at::kFloat),
               past[static_cast<std::size_t>(b)]);
      }
    }
    *out[0] = result(o.view({B, Hq, Sq, D}), q.dtype());
  }
};

// reshape/template.cc:7-9: a view; one dim may be -1.
class ReshapeOp final : public Operator {
 public:
  std::string type() const override { return "reshape"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    *out[0] = in[0]->withShape(
        reshapeShape(in[0]->shape(), attrs.require<std::vector<std::int64_t>>("shape")));
  }
};

// transpose/template.cc:7-18: 2-D, perm [1, 0]; extension as the device plugin: rank 4 with
// perm [0, 2, 1, 3].
class TransposeOp final : public Operator {
 public:
  std::string type() const override { return "transpose"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireFloating(*in[0], type());
    const auto perm = attrs.require<std::vector<std::int64_t>>("perm");
    if (in[0]->rank() == 4 && perm == std::vector<std::int64_t>{0, 2, 1, 3}) {
      *out[0] = Tensor(in[0]->torchTensor().transpose(1, 2).contiguous());
      return;
    }
    if (in[0]->rank() != 2 || perm != std::vector<std::int64_t>{1, 0})
      throw std::invalid_argument("transpose supports 2D perm [1,0] and 4D perm [0,2,1,3]");
    *out[0] = Tensor(in[0]->torchTensor().t().contiguous());
  }
};

// conv2d/kernel.py:6-49: NCHW, zero padding; attrs stride, padding; extension activation.
class Conv2dOp final : public Operator {
 public:
  std::string type() const override { return "conv2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 2, 3, 1, type());
    requireFloating(*in[0], type());
    for (const Tensor* t : in) requireSameDType(*in[0], *t, type());
    if (in[0]->rank() != 4 || in[1]->rank() != 4 || in[0]->dim(1) != in[1]->dim(1))
      throw std::invalid_argument("conv2d expects NCHW input and [OC, C, KH, KW] weight");
    const auto stride = attrInts(attrs, "stride", {1, 1});
    const auto pad = attrInts(attrs, "padding", {0, 0});
    at::Tensor y = at::conv2d(f32(*in[0]), f32(*in[1]),
                              in.size() == 3 ? c10::optional<at::Tensor>(f32(*in[2])) : c10::nullopt,
                              stride, pad);
    if (attrs.value_or<std::string>("activation", "none") == "relu") y = at::relu(y);
    *out[0] = result(y, in[0]->dtype());
  }
};

// max_pool2d/kernel.py:6-41: -inf padding; attrs kernel_size [2,2], stride (= kernel_size),
// padding [0,0].
class MaxPool2dOp final : public Operator {
 public:
  std::string type() const override { return "max_pool2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireFloating(*in[0], type());
    if (in[0]->rank() != 4) throw std::invalid_argument("max_pool2d expects NCHW input");
    const auto ks = attrInts(attrs, "kernel_size", {2, 2});
    const auto stride = attrInts(attrs, "stride", ks);
    const auto pad = attrInts(attrs, "padding", {0, 0});
    *out[0] = result(at::max_pool2d(f32(*in[0]), ks, stride, pad), in[0]->dtype());
  }
};

// batch_norm2d/kernel.py:6-28: eval-mode batch norm; inputs x, weight, bias, mean, var; eps.
class BatchNorm2dOp final : public Operator {
 public:
  std::string type() const override { return "batch_norm2d"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes& attrs, ExecutionContext&) const override {
    requireArity(in, out, 5, 5, 1, type());
    requireFloating(*in[0], type());
    if (in[0]->rank() != 4) throw std::invalid_argument("batch_norm2d expects NCHW input");
    const double eps = attrDouble(attrs, "eps", 1e-5);
    *out[0] = result(at::batch_norm(f32(*in[0]), f32(*in[1]), f32(*in[2]), f32(*in[3]),
                                    f32(*in[4]), false, 0.0, eps, false),
                     in[0]->dtype());
  }
};

// The decode graph's greedy choice: first index of the maximum over the last dim.
class ArgmaxOp final : public Operator {
 public:
  std::string type() const override { return "argmax"; }
  void compute(const std::vector<const Tensor*>& in, const std::vector<Tensor*>& out,
               const Attributes&, ExecutionContext&) const override {
    requireArity(in, out, 1, 1, 1, type());
    requireFloating(*in[0], type());
    *out[0] = Tensor(at::argmax(f32(*in[0]), -1).reshape({-1}).contiguous());
  }
};

template <typename Op>
void add(OperatorRegistry* registry) {
  registry->registerFactory(Op().type(), [] { return std::make_unique<Op>(); });
}

}  // namespace
}  // namespace dli::aten_plugin

extern "C" __attribute__((visibility("default"))) bool dli_register_operators(
    dli::OperatorRegistry* registry) {
  using namespace dli::aten_plugin;
  if (registry == nullptr) return false;
  try {
    add<BroadcastOp<false>>(registry);
    add<BroadcastOp<true>>(registry);
    add<ActivationOp<false>>(registry);
    add<ActivationOp<true>>(registry);
    add<SoftmaxOp>(registry);
    add<RmsNormOp>(registry);
    add<EmbeddingOp>(registry);
    add<LinearOp>(registry);
    add<LinearResidualOp>(registry);
    add<MatmulOp>(registry);
    add<RotaryOp>(registry);
    add<AttentionOp>(registry);
    add<ReshapeOp>(registry);
    add<TransposeOp>(registry);
    add<Conv2dOp>(registry);
    add<MaxPool2dOp>(registry);
    add<BatchNorm2dOp>(registry);
    add<ArgmaxOp>(registry);
    return true;
  } catch (...) {
    return false;
  }
}
