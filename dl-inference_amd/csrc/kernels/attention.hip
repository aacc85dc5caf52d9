// Attention kernels for gfx950.
//
//  attention_<t>         softmax(q k^T * scale [+ causal mask]) v over contiguous [B, H, S, D]
//                        tensors (attention/kernel.py:6-62) with grouped KV heads.
//  paged_attention_<t>   the same over the paged KV cache (layout in include/dli/kv_cache.h),
//                        per-sequence lengths from `positions`.
//  kv_append_<t>         scatters new key/value tokens into the paged cache.
//
// The generic kernels give one wave to one (batch, q head, query) row: 64 keys per round,
// lane j scores key j, online softmax across rounds (running max / sum in fp32), then the
// wave accumulates p_j * v_j with each lane owning head_dim/64 output dims.
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

constexpr int kMaxDimPerLane = 4;  // head_dim <= 256

template <typename T>
struct DenseKV {
  const T* k;
  const T* v;
  int64_t kv_heads, seq_k, head_dim;
  __device__ const T* keyRow(int64_t b, int64_t h, int64_t j) const {
    return k + ((b * kv_heads + h) * seq_k + j) * head_dim;
  }
  __device__ float value(int64_t b, int64_t h, int64_t j, int64_t d) const {
    return ld(v + ((b * kv_heads + h) * seq_k + j) * head_dim + d);
  }
};

template <typename T>
struct PagedKV {
  const T* k_pool;
  const T* v_pool;
  const int32_t* block_table;
  int64_t kv_heads, head_dim, block_size, max_blocks;
  __device__ int64_t block(int64_t b, int64_t j) const {
    return block_table[b * max_blocks + j / block_size];
  }
  __device__ const T* keyRow(int64_t b, int64_t h, int64_t j) const {
    return k_pool + ((block(b, j) * kv_heads + h) * block_size + j % block_size) * head_dim;
  }
  __device__ float value(int64_t b, int64_t h, int64_t j, int64_t d) const {
    return ld(v_pool + ((block(b, j) * kv_heads + h) * head_dim + d) * block_size + j % block_size);
  }
};

// One wave computes out[b, h, i, :] for keys [0, kv_len).
template <typename T, typename KV>
__device__ void attendRow(const T* qrow, T* orow, const KV& kv, int64_t b, int64_t kvh,
                          int64_t kv_len, int64_t head_dim, float scale, float* q_lds,
                          float* p_lds) {
  const int lane = threadIdx.x % kWave;
  for (int64_t d = lane; d < head_dim; d += kWave) q_lds[d] = ld(qrow + d) * scale;
  __builtin_amdgcn_wave_barrier();
  __syncthreads();
  float m_run = -INFINITY, l_run = 0.f;
  float acc[kMaxDimPerLane] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t j0 = 0; j0 < kv_len; j0 += kWave) {
    const int64_t j = j0 + lane;
    float s = -INFINITY;
    if (j < kv_len) {
      const T* krow = kv.keyRow(b, kvh, j);
      float dot = 0.f;
      for (int64_t d = 0; d < head_dim; ++d) dot = fmaf(q_lds[d], ld(krow + d), dot);
      s = dot;
    }
    const float m_new = fmaxf(m_run, waveMax(s));
    const float p = (j < kv_len) ? __expf(s - m_new) : 0.f;
    const float alpha = __expf(m_run - m_new);  // 0 on the first round (m_run = -inf)
    l_run = l_run * alpha + waveSum(p);
    m_run = m_new;
    p_lds[lane] = p;
    __syncthreads();
    const int64_t n = (kv_len - j0 < kWave) ? kv_len - j0 : kWave;
#pragma unroll
    for (int t = 0; t < kMaxDimPerLane; ++t) {
      const int64_t d = lane + t * kWave;
      if (d >= head_dim) break;
      float a = acc[t] * alpha;
      for (int64_t jj = 0; jj < n; ++jj) a = fmaf(p_lds[jj], kv.value(b, kvh, j0 + jj, d), a);
      acc[t] = a;
    }
    __syncthreads();
  }
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
  for (int t = 0; t < kMaxDimPerLane; ++t) {
    const int64_t d = lane + t * kWave;
    if (d < head_dim) st(orow + d, acc[t] * inv);
  }
}

// Block = 64 threads (one wave, so __syncthreads is a wave barrier); grid.x = B * Hq * Sq rows.
template <typename T>
__device__ void attention_impl(const void* q_, const void* k_, const void* v_, void* out_,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                               int64_t D, int causal, float scale) {
  __shared__ float q_lds[256];
  __shared__ float p_lds[kWave];
  const int64_t row = blockIdx.x;  // ((b * Hq + h) * Sq + i)
  const int64_t i = row % Sq;
  const int64_t h = (row / Sq) % Hq;
  const int64_t b = row / (Sq * Hq);
  const int64_t kvh = h / (Hq / Hkv);
  DenseKV<T> kv{static_cast<const T*>(k_), static_cast<const T*>(v_), Hkv, Sk, D};
  int64_t kv_len = Sk;
  if (causal) {
    const int64_t limit = (Sk - Sq) + i + 1;
    kv_len = limit < Sk ? (limit > 0 ? limit : 0) : Sk;
  }
  attendRow(static_cast<const T*>(q_) + row * D, static_cast<T*>(out_) + row * D, kv, b, kvh,
            kv_len, D, scale, q_lds, p_lds);
}

template <typename T>
__device__ void paged_attention_impl(const void* q_, const void* k_pool, const void* v_pool,
                                     const int32_t* block_table, void* out_, int64_t B, int64_t Hq,
                                     int64_t Hkv, int64_t Sq, int64_t D, int64_t block_size,
                                     int64_t max_blocks, int64_t past, const void* positions,
                                     int pos64, int causal, float scale) {
  __shared__ float q_lds[256];
  __shared__ float p_lds[kWave];
  const int64_t row = blockIdx.x;
  const int64_t i = row % Sq;
  const int64_t h = (row / Sq) % Hq;
  const int64_t b = row / (Sq * Hq);
  const int64_t kvh = h / (Hq / Hkv);
  const int64_t past_b = positions != nullptr ? loadIndex(positions, pos64, b) : past;
  const int64_t capacity = max_blocks * block_size;
  int64_t kv_len = causal ? past_b + i + 1 : past_b + Sq;
  if (kv_len > capacity) kv_len = capacity;
  if (kv_len < 0) kv_len = 0;
  PagedKV<T> kv{static_cast<const T*>(k_pool), static_cast<const T*>(v_pool), block_table, Hkv, D,
                block_size, max_blocks};
  attendRow(static_cast<const T*>(q_) + row * D, static_cast<T*>(out_) + row * D, kv, b, kvh,
            kv_len, D, scale, q_lds, p_lds);
}

// One thread per (b, h, s, d) element of the new tokens; grid-stride.
template <typename T>
__device__ void kv_append_impl(const void* key, const void* value, void* k_pool, void* v_pool,
                               const int32_t* block_table, int64_t B, int64_t H, int64_t S,
                               int64_t D, int64_t block_size, int64_t max_blocks, int64_t start,
                               const void* positions, int pos64) {
  const T* pk = static_cast<const T*>(key);
  const T* pv = static_cast<const T*>(value);
  T* kp = static_cast<T*>(k_pool);
  T* vp = static_cast<T*>(v_pool);
  const int64_t total = B * H * S * D;
  const int64_t capacity = max_blocks * block_size;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t d = e % D;
    const int64_t s = (e / D) % S;
    const int64_t h = (e / (D * S)) % H;
    const int64_t b = e / (D * S * H);
    const int64_t pos = (positions != nullptr ? loadIndex(positions, pos64, b) : start) + s;
    if (pos < 0 || pos >= capacity) continue;
    const int64_t blk = block_table[b * max_blocks + pos / block_size];
    const int64_t off = pos % block_size;
    kp[((blk * H + h) * block_size + off) * D + d] = pk[e];
    vp[((blk * H + h) * D + d) * block_size + off] = pv[e];
  }
}

// bf16 tokens, head_dim % 8 == 0 and <= 256, 16-byte aligned: one 256-thread workgroup per
// (b, h, 64 new tokens). Key rows go out as 16-byte runs (the key pool is token-major); the value
// chunk is staged in LDS and written d-major (the value pool holds [block][H][D][block_size]), 64
// consecutive lanes storing 64 consecutive slots of one d. Same placement as kv_append_impl.
constexpr int kAppendTokens = 64;

__device__ void kv_append_tiles_bf16(const uint16_t* key, const uint16_t* value, uint16_t* k_pool,
                                     uint16_t* v_pool, const int32_t* block_table, int64_t H,
                                     int64_t S, int D, int64_t block_size, int64_t max_blocks,
                                     int64_t start, const void* positions, int pos64) {
  __shared__ __attribute__((aligned(16))) uint16_t vs[kAppendTokens * (256 + 8)];
  const int pitch = D + 8;
  const int64_t bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * kAppendTokens;
  const int64_t base_pos = (positions != nullptr ? loadIndex(positions, pos64, b) : start) + s0;
  const int64_t capacity = max_blocks * block_size;
  const int chunks = D / 8;  // 16-byte chunks per token
  const uint16_t* kin = key + (bh * S + s0) * D;
  const uint16_t* vin = value + (bh * S + s0) * D;
  for (int c = threadIdx.x; c < kAppendTokens * chunks; c += blockDim.x) {
    const int t = c / chunks, part = c % chunks;
    if (s0 + t >= S) continue;
    const U128 kw = gload16(kin + t * D + part * 8);
    *reinterpret_cast<U128*>(&vs[t * pitch + part * 8]) = gload16(vin + t * D + part * 8);
    const int64_t pos = base_pos + t;
    if (pos < 0 || pos >= capacity) continue;
    const int64_t blk = block_table[b * max_blocks + pos / block_size];
    *gp(reinterpret_cast<U128*>(k_pool + ((blk * H + h) * block_size + pos % block_size) * D +
                                part * 8)) = kw;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kAppendTokens * D; e += blockDim.x) {
    const int d = e / kAppendTokens, t = e % kAppendTokens;
    const int64_t pos = base_pos + t;
    if (s0 + t >= S || pos < 0 || pos >= capacity) continue;
    const int64_t blk = block_table[b * max_blocks + pos / block_size];
    *gp(v_pool + ((blk * H + h) * D + d) * block_size + pos % block_size) = vs[t * pitch + d];
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
    kv_append_tiles_bf16_k(const uint16_t* key, const uint16_t* value, uint16_t* k_pool,
                           uint16_t* v_pool, const int32_t* block_table, int64_t H, int64_t S,
                           int D, int64_t block_size, int64_t max_blocks, int64_t start,
                           const void* positions, int pos64) {
  kv_append_tiles_bf16(key, value, k_pool, v_pool, block_table, H, S, D, block_size, max_blocks,
                       start, positions, pos64);
}

DK_FLOAT_KERNELS(attention, 64,
                 (const void* q, const void* k, const void* v, void* out, int64_t B, int64_t Hq,
                  int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, int causal, float scale),
                 (q, k, v, out, B, Hq, Hkv, Sq, Sk, D, causal, scale))
DK_FLOAT_KERNELS(paged_attention, 64,
                 (const void* q, const void* k_pool, const void* v_pool,
                  const int32_t* block_table, void* out, int64_t B, int64_t Hq, int64_t Hkv,
                  int64_t Sq, int64_t D, int64_t block_size, int64_t max_blocks, int64_t past,
                  const void* positions, int pos64, int causal, float scale),
                 (q, k_pool, v_pool, block_table, out, B, Hq, Hkv, Sq, D, block_size, max_blocks,
                  past, positions, pos64, causal, scale))
DK_FLOAT_KERNELS(kv_append, 256,
                 (const void* key, const void* value, void* k_pool, void* v_pool,
                  const int32_t* block_table, int64_t B, int64_t H, int64_t S, int64_t D,
                  int64_t block_size, int64_t max_blocks, int64_t start, const void* positions,
                  int pos64),
                 (key, value, k_pool, v_pool, block_table, B, H, S, D, block_size, max_blocks,
                  start, positions, pos64))

// ---------------------------------------------------------------------------------------------
// Decode attention over the paged cache with MFMA (decode_attention.h): grid (splits,
// batch * kv_heads), one unit per workgroup. The last unit of a pair merges the partials and
// leaves the pair's counter at zero for the next call.
// ---------------------------------------------------------------------------------------------
#include "decode_attention.h"

extern "C" __global__ void __launch_bounds__(dk::kDecThreads)
    decode_attention_d64(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                         const int32_t* block_table, const void* positions, int pos64, int64_t past,
                         float* ws_ml, float* ws_o, unsigned* counters, uint16_t* out, int Hq,
                         int Hkv, int64_t max_blocks, int max_splits, float scale_log2) {
  __shared__ dk::DecodeAttnLds lds;
  const dk::DecodeAttnArgs a{q,     k_pool, v_pool, block_table, positions, pos64,      past,
                             ws_ml, ws_o,   counters, out,       Hq,        Hkv,        max_blocks,
                             max_splits, scale_log2};
  dk::decodeAttentionUnit<dk::PlainMem, false>(a, blockIdx.x, blockIdx.y,
                                               static_cast<unsigned>(max_splits), true, lds,
                                               nullptr, 0, dk::NoWait{}, dk::NoWait{});
}

// ---------------------------------------------------------------------------------------------
// Decode attention for head_dim 128 (decode_attention_d128.h): grid (splits, batch * kv_heads /
// hpw), hpw kv heads per workgroup (1, or kv_heads when it divides 8).
// ---------------------------------------------------------------------------------------------
#include "decode_attention_d128.h"

extern "C" __global__ void __launch_bounds__(dk::kD128Threads)
    decode_attention_d128(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                          const int32_t* block_table, const void* positions, int pos64,
                          int64_t past, float* ws_ml, float* ws_o, unsigned* counters,
                          uint16_t* out, int Hq, int Hkv, int64_t max_blocks, int splits,
                          float scale_log2, int hpw) {
  __shared__ dk::DecodeAttn128Lds lds;
  const dk::DecodeAttn128Args a{q,     k_pool, v_pool,   block_table, positions, pos64,
                                past,  ws_ml,  ws_o,     counters,    out,       Hq,
                                Hkv,   max_blocks, splits, scale_log2};
  dk::decodeAttention128Unit(a, blockIdx.x, blockIdx.y, hpw, lds);
}
