#pragma once

// Paged key/value cache in device memory.
//
// Replaces src/kv_cache.cc:9-44 of the reference (a contiguous fp32 [B,H,S,D] pair that is
// reallocated and fully copied on every append). Here each named entry (one per attention
// layer) owns two block pools that are allocated once:
//
//   key_pool   [num_blocks, heads, block_size, head_dim]   token-major inside a block
//   value_pool [num_blocks, heads, head_dim, block_size]   dim-major inside a block
//
// plus an int32 block table [batch, max_blocks] mapping (sequence, logical block) to a
// physical block. An append writes only the new tokens (one scatter kernel, no host sync).
// The value layout is transposed so that the attention kernels' P*V step reads 16-byte
// runs of consecutive tokens.
//
// Positions are either tracked on the host (reference semantics: every sequence has the same
// length, append() advances it) or passed per sequence as a device tensor (appendAt), which
// keeps a decode step free of host state so it can be captured into a HIP graph.
//
// Host entries (key/value on the CPU, device id kCpuDevice: the ATen CPU reference plugin) use
// the same structure with one block per sequence (block_size = capacity, identity table), so a
// sequence's keys are [heads, capacity, head_dim] and its values [heads, head_dim, capacity],
// each contiguous; they do not grow beyond the configured max_seq_len.

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "dli/tensor.h"

namespace dli {

constexpr int kCpuDevice = -1;  // device id of host KV cache entries

// The pools are named key_pool / value_pool, not key / value as in the reference's entry
// (include/dli/kv_cache.h of the reference: contiguous [B,H,S,D] tensors that its attention
// template binds directly as K and V), so that code written against that layout fails to compile
// here instead of reading a paged pool as [B,H,S,D].
struct KVCacheEntry {
  Tensor key_pool;
  Tensor value_pool;
  Tensor block_table;  // int32 [batch, max_blocks], device
  std::int64_t batch = 0;
  std::int64_t heads = 0;
  std::int64_t head_dim = 0;
  std::int64_t block_size = 0;
  std::int64_t max_blocks = 0;  // per sequence
  std::int64_t length = 0;      // host-tracked tokens per sequence (append() path)

  std::int64_t capacity() const { return max_blocks * block_size; }
};

class KVCache {
 public:
  // Reference-compatible append: key/value are [B,H,S,D] device tensors; the S new tokens are
  // written at the host-tracked length, which then advances by S.
  void append(const std::string& name, const Tensor& key, const Tensor& value);
  const KVCacheEntry* get(const std::string& name) const;
  std::size_t size() const { return entries_.size(); }
  void clear() { entries_.clear(); }

  // Appends token s of sequence b at position positions[b] + s (positions: int32/int64 [B] on
  // the device). The host-tracked length is left untouched.
  void appendAt(const std::string& name, const Tensor& key, const Tensor& value,
                const Tensor& positions);

  // Allocates (or returns) an entry ahead of time. Capacity per sequence is max_seq_len
  // rounded up to whole blocks.
  KVCacheEntry& reserve(const std::string& name, DType dtype, std::int64_t batch,
                        std::int64_t heads, std::int64_t head_dim, int device_id);
  KVCacheEntry* find(const std::string& name);

  void configure(std::int64_t block_size, std::int64_t max_seq_len);
  std::int64_t blockSize() const { return block_size_; }
  std::int64_t maxSeqLen() const { return max_seq_len_; }
  // Stream used by the scatter kernels (nullptr = the null stream).
  void setStream(void* stream) { stream_ = stream; }
  void* stream() const { return stream_; }
  // Sets the host-tracked length of every entry (e.g. after filling the cache externally).
  void setLength(std::int64_t length);

 private:
  std::map<std::string, KVCacheEntry> entries_;
  std::int64_t block_size_ = 64;
  std::int64_t max_seq_len_ = 4096;
  void* stream_ = nullptr;

  void grow(KVCacheEntry& entry, std::int64_t needed_tokens);
};

}  // namespace dli
