// Paged KV cache (replaces src/kv_cache.cc:9-49 of the reference; layout in kv_cache.h).
#include "dli/kv_cache.h"

#include <stdexcept>
#include <string>

#include "dli_hip.h"

namespace dli {
namespace {

int hipDtype(DType dtype) {
  switch (dtype) {
    case DType::Float32: return DLI_F32;
    case DType::BFloat16: return DLI_BF16;
    case DType::Float16: return DLI_F16;
    default: throw std::invalid_argument("KV cache expects floating tensors");
  }
}

void hipCheck(int rc, const char* what) {
  if (rc != 0) throw std::runtime_error(std::string(what) + ": " + dli_hip_last_error());
}

void validatePair(const Tensor& key, const Tensor& value) {
  if (key.isCuda() != value.isCuda())
    throw std::invalid_argument("KV cache key/value must be on the same device");
  if (key.rank() != 4 || value.rank() != 4)
    throw std::invalid_argument("KV cache expects rank-4 tensors");
  if (key.shape() != value.shape()) throw std::invalid_argument("KV key/value shape mismatch");
  if (key.dtype() != value.dtype()) throw std::invalid_argument("KV key/value dtype mismatch");
  hipDtype(key.dtype());
}

Tensor identityBlockTable(std::int64_t batch, std::int64_t max_blocks, int device_id) {
  auto table = at::arange(batch * max_blocks, at::TensorOptions().dtype(at::kInt))
                   .view({batch, max_blocks});
  return Tensor(table.to(at::Device(at::kCUDA, device_id)));
}

void allocatePools(KVCacheEntry& e, DType dtype, int device_id) {
  const std::int64_t blocks = e.batch * e.max_blocks;
  // Zero-filled once, so that attention kernels reading a partially filled block see finite
  // values in the slots they mask out.
  auto options = at::TensorOptions().dtype(toTorchDType(dtype));
  options = device_id == kCpuDevice ? options.device(at::kCPU)
                                    : options.device(at::kCUDA, device_id);
  e.key_pool = Tensor(at::zeros({blocks, e.heads, e.block_size, e.head_dim}, options));
  e.value_pool = Tensor(at::zeros({blocks, e.heads, e.head_dim, e.block_size}, options));
  if (device_id == kCpuDevice) {
    e.block_table = Tensor(at::arange(blocks, at::TensorOptions().dtype(at::kInt))
                               .view({e.batch, e.max_blocks}));
  } else {
    e.block_table = identityBlockTable(e.batch, e.max_blocks, device_id);
  }
}

// Host entries hold one block per sequence (block_size = capacity), so sequence b's keys are
// key_pool[b] = [heads, capacity, head_dim] and its values value_pool[b] = [heads, head_dim,
// capacity]: contiguous per head, which the ATen CPU attention reads without a gather. Token s
// of sequence b goes to position start[b] + s.
void appendHost(KVCacheEntry& e, const Tensor& key, const Tensor& value,
                const std::vector<std::int64_t>& start) {
  const std::int64_t seq = key.dim(2);
  at::Tensor kp = e.key_pool.torchTensor(), vp = e.value_pool.torchTensor();
  const at::Tensor& k = key.torchTensor();
  const at::Tensor& v = value.torchTensor();
  for (std::int64_t b = 0; b < e.batch; ++b) {
    const std::int64_t p = start[static_cast<std::size_t>(b)];
    if (p < 0 || p + seq > e.capacity())
      throw std::out_of_range("KV cache position outside the host cache capacity");
    kp[b].narrow(1, p, seq).copy_(k[b]);
    vp[b].narrow(2, p, seq).copy_(v[b].transpose(-1, -2));
  }
}

}  // namespace

void KVCache::configure(std::int64_t block_size, std::int64_t max_seq_len) {
  if (block_size <= 0 || max_seq_len <= 0)
    throw std::invalid_argument("KV cache block_size and max_seq_len must be positive");
  block_size_ = block_size;
  max_seq_len_ = max_seq_len;
}

KVCacheEntry* KVCache::find(const std::string& name) {
  auto it = entries_.find(name);
  return it == entries_.end() ? nullptr : &it->second;
}

const KVCacheEntry* KVCache::get(const std::string& name) const {
  auto it = entries_.find(name);
  return it == entries_.end() ? nullptr : &it->second;
}

KVCacheEntry& KVCache::reserve(const std::string& name, DType dtype, std::int64_t batch,
                               std::int64_t heads, std::int64_t head_dim, int device_id) {
  if (KVCacheEntry* existing = find(name)) {
    if (existing->batch != batch || existing->heads != heads || existing->head_dim != head_dim)
      throw std::invalid_argument("KV cache append shape mismatch");
    if (existing->key_pool.dtype() != dtype) throw std::invalid_argument("KV cache dtype mismatch");
    return *existing;
  }
  if (batch <= 0 || heads <= 0 || head_dim <= 0)
    throw std::invalid_argument("KV cache geometry must be positive");
  hipDtype(dtype);
  KVCacheEntry entry;
  entry.batch = batch;
  entry.heads = heads;
  entry.head_dim = head_dim;
  entry.block_size = block_size_;
  entry.max_blocks = (max_seq_len_ + block_size_ - 1) / block_size_;
  if (device_id == kCpuDevice) {  // one block per sequence on the host
    entry.block_size *= entry.max_blocks;
    entry.max_blocks = 1;
  }
  allocatePools(entry, dtype, device_id);
  return entries_.emplace(name, std::move(entry)).first->second;
}

void KVCache::grow(KVCacheEntry& e, std::int64_t needed_tokens) {
  if (!e.key_pool.isCuda())
    throw std::out_of_range("host KV cache holds " + std::to_string(e.capacity()) +
                            " tokens per sequence (configure a larger max_seq_len)");
  std::int64_t blocks = e.max_blocks;
  while (blocks * e.block_size < needed_tokens) blocks *= 2;
  if (blocks == e.max_blocks) return;
  KVCacheEntry bigger = e;
  bigger.max_blocks = blocks;
  allocatePools(bigger, e.key_pool.dtype(), e.key_pool.deviceId());
  // Physical block (b * old_max + i) moves to (b * new_max + i); copy per sequence.
  const std::size_t block_bytes =
      static_cast<std::size_t>(e.heads * e.block_size * e.head_dim) * byteSize(e.key_pool.dtype());
  for (std::int64_t b = 0; b < e.batch; ++b) {
    const std::size_t src = static_cast<std::size_t>(b * e.max_blocks) * block_bytes;
    const std::size_t dst = static_cast<std::size_t>(b * blocks) * block_bytes;
    const std::size_t bytes = static_cast<std::size_t>(e.max_blocks) * block_bytes;
    hipCheck(dli_hip_memcpy_async(static_cast<char*>(bigger.key_pool.deviceData()) + dst,
                                  static_cast<const char*>(e.key_pool.deviceData()) + src, bytes,
                                  DLI_MEMCPY_DEVICE_TO_DEVICE, stream_),
             "KV cache grow");
    hipCheck(dli_hip_memcpy_async(static_cast<char*>(bigger.value_pool.deviceData()) + dst,
                                  static_cast<const char*>(e.value_pool.deviceData()) + src, bytes,
                                  DLI_MEMCPY_DEVICE_TO_DEVICE, stream_),
             "KV cache grow");
  }
  e = std::move(bigger);
}

void KVCache::append(const std::string& name, const Tensor& key, const Tensor& value) {
  validatePair(key, value);
  KVCacheEntry& e = reserve(name, key.dtype(), key.dim(0), key.dim(1), key.dim(3),
                            key.isCuda() ? key.deviceId() : kCpuDevice);
  const std::int64_t seq = key.dim(2);
  if (e.length + seq > e.capacity()) grow(e, e.length + seq);
  if (!key.isCuda()) {
    appendHost(e, key, value, std::vector<std::int64_t>(static_cast<std::size_t>(e.batch), e.length));
    e.length += seq;
    return;
  }
  hipCheck(dli_hip_kv_append(hipDtype(key.dtype()), key.deviceData(), value.deviceData(),
                             e.key_pool.deviceData(), e.value_pool.deviceData(),
                             static_cast<const std::int32_t*>(e.block_table.deviceData()), e.batch,
                             e.heads, seq, e.head_dim, e.block_size, e.max_blocks, e.length,
                             nullptr, DLI_I64, stream_),
           "KV cache append");
  e.length += seq;
}

void KVCache::appendAt(const std::string& name, const Tensor& key, const Tensor& value,
                       const Tensor& positions) {
  validatePair(key, value);
  if (positions.isCuda() != key.isCuda())
    throw std::invalid_argument("KV cache positions must be on the key's device");
  if (positions.dtype() != DType::Int64 && positions.dtype() != DType::Int32)
    throw std::invalid_argument("KV cache positions must be int64 or int32");
  if (static_cast<std::int64_t>(positions.numel()) != key.dim(0))
    throw std::invalid_argument("KV cache positions must hold one entry per sequence");
  KVCacheEntry& e = reserve(name, key.dtype(), key.dim(0), key.dim(1), key.dim(3),
                            key.isCuda() ? key.deviceId() : kCpuDevice);
  if (!key.isCuda()) {
    const at::Tensor pos = positions.torchTensor().to(at::kLong).contiguous();
    const std::int64_t* p = pos.data_ptr<std::int64_t>();
    appendHost(e, key, value, std::vector<std::int64_t>(p, p + e.batch));
    return;
  }
  hipCheck(dli_hip_kv_append(hipDtype(key.dtype()), key.deviceData(), value.deviceData(),
                             e.key_pool.deviceData(), e.value_pool.deviceData(),
                             static_cast<const std::int32_t*>(e.block_table.deviceData()), e.batch,
                             e.heads, key.dim(2), e.head_dim, e.block_size, e.max_blocks, 0,
                             positions.deviceData(),
                             positions.dtype() == DType::Int64 ? DLI_I64 : DLI_I32, stream_),
           "KV cache append");
}

void KVCache::setLength(std::int64_t length) {
  if (length < 0) throw std::invalid_argument("KV cache length must be non-negative");
  for (auto& [name, e] : entries_) {
    if (length > e.capacity()) grow(e, length);
    e.length = length;
  }
}

}  // namespace dli
