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

}  // namespace

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
// Decode attention over the paged cache with MFMA (bf16, head_dim 64, one query per sequence,
// up to 16 query heads per KV head). "Flash decoding": grid (splits, batch * kv_heads); a
// workgroup owns a share of the cache blocks of one (sequence, kv head) and all query heads of
// that group, so each K/V byte is read once per KV head rather than once per query head.
//
// Per wave and 32-key sub-tile (v_mfma_f32_16x16x32_bf16):
//   S = K Q^T    A = 16 keys x 32 dims (two MFMAs per 64 dims), B = Q^T (16 heads).
//                The A rows of half hf are keys t0 + 8*(r/4) + 4*hf + r%4, so the output lane
//                (r, g) holds keys t0 + 8g + 4hf + i (i < 4) of head r: eight consecutive keys.
//   online softmax per head column (max/sum over the 4 lane groups with xor-shuffles)
//   O^T += V^T P^T  A = V^T (16 dims x 32 keys, dim-major cache blocks give 16-byte runs),
//                B = P^T straight from the registers above (no LDS round trip).
// The 8 waves of a workgroup merge (m, l, O) through LDS; the last split of a (sequence, kv
// head) to finish merges the splits' partials.
// ---------------------------------------------------------------------------------------------
#include "skinny.h"

namespace {

constexpr int kDecD = 64;

// Workgroup = kDecWaves waves over the key range of one split; wave w takes cache blocks
// w, w + kDecWaves, ... of that range (a whole block of 64 keys = two 32-key MFMA sub-tiles,
// so every V row segment of a block is consumed by one wave). The next block's K/V loads are
// issued before the current block is computed (two register buffers).
constexpr int kDecWaves = 8;
constexpr int kDecBlock = 64;  // keys per cache block handled by this kernel

struct KvBlockRegs {
  U128 k[2][2][2];  // [sub-tile][half][dim half]
  U128 v[2][4];     // [sub-tile][16-dim group]
};

__device__ __forceinline__ void loadKvBlock(KvBlockRegs& regs, const uint16_t* k_pool,
                                            const uint16_t* v_pool, int64_t blk,
                                            int64_t blk_index, int64_t end, int Hkv, int kvh,
                                            int r, int g) {
  const int64_t t_block = blk_index * kDecBlock;
  const int64_t head_stride = static_cast<int64_t>(kDecBlock) * kDecD;
  const uint16_t* kbase = k_pool + (blk * Hkv + kvh) * head_stride;
  const uint16_t* vbase = v_pool + (blk * Hkv + kvh) * head_stride;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int off = 32 * st + 8 * (r / 4) + 4 * hf + (r % 4);
      const bool ok = t_block + off < end;
      regs.k[st][hf][0] = ok ? load16(kbase + off * kDecD + g * 8) : zero16();
      regs.k[st][hf][1] = ok ? load16(kbase + off * kDecD + 32 + g * 8) : zero16();
    }
    const bool vok = t_block + 32 * st + 8 * g < end;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      regs.v[st][d] = vok ? load16(vbase + (d * 16 + r) * kDecBlock + 32 * st + 8 * g) : zero16();
  }
}

struct SoftmaxState {
  float m = -INFINITY;
  float l = 0.f;
  f32x4 o[4];
};

__device__ __forceinline__ void attendBlock(SoftmaxState& st8, const KvBlockRegs& regs,
                                            const U128 (&qf)[2], int64_t t_block, int64_t end,
                                            int g, float scale_log2) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int64_t t0 = t_block + 32 * st;
    if (t0 >= end) break;  // uniform per wave
    f32x4 sc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      sc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
      sc[hf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.k[st][hf][0]), asBf16x8(qf[0]), sc[hf], 0, 0, 0);
      sc[hf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.k[st][hf][1]), asBf16x8(qf[1]), sc[hf], 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t tok = t0 + 8 * g + 4 * hf + e;
        const float v = tok < end ? sc[hf][e] * scale_log2 : -INFINITY;
        sc[hf][e] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(st8.m, mx);
    const float alpha = exp2f(st8.m - m_new);
    float p[2][4];
    float sum = 0.f;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[hf][e] = exp2f(sc[hf][e] - m_new);
        sum += p[hf][e];
      }
    sum += __shfl_xor(sum, 16, kWave);
    sum += __shfl_xor(sum, 32, kWave);
    st8.l = st8.l * alpha + sum;
    st8.m = m_new;
    // P in two bf16 terms (hi + lo) so the P*V products carry ~16 significant bits of P.
    U128 phi, plo;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float a0 = p[w2 / 2][(w2 % 2) * 2], a1 = p[w2 / 2][(w2 % 2) * 2 + 1];
      phi[w2] = packBf16x2(a0, a1);
      plo[w2] = packBf16x2(a0 - bf16ToFloat(static_cast<uint16_t>(phi[w2])),
                             a1 - bf16ToFloat(static_cast<uint16_t>(phi[w2] >> 16)));
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      st8.o[d] *= alpha;
      st8.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.v[st][d]), asBf16x8(phi), st8.o[d], 0, 0, 0);
      st8.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.v[st][d]), asBf16x8(plo), st8.o[d], 0, 0, 0);
    }
  }
}

// grid (splits, batch * kv_heads), kDecWaves * 64 threads. The live cache blocks of a
// (sequence, kv head) are dealt round-robin over the splits x kDecWaves waves of its
// workgroups: wave w of split s takes blocks s * kDecWaves + w, + splits * kDecWaves, ..., so
// every wave streams the same number of blocks whatever the sequence length. With one split
// the normalized output is written directly. Otherwise each split stores its (m, l, O) partial
// with agent-scope stores and arrives at counters[b * Hkv + kvh]; the last split to arrive
// reads every partial with agent-scope loads and merges them in split order (no
// cross-workgroup fence, no second kernel), then resets the counter to zero for the next call.
// Requires max_blocks <= max_splits * kDecWaves * 64 (a wave keeps its block ids in 64 lanes).
__device__ void decode_attention_impl(const uint16_t* q, const uint16_t* k_pool,
                                      const uint16_t* v_pool, const int32_t* block_table,
                                      const void* positions, int pos64, int64_t past, float* ws_ml,
                                      float* ws_o, unsigned* counters, uint16_t* out, int Hq,
                                      int Hkv, int64_t max_blocks, int max_splits,
                                      float scale_log2) {
  __shared__ float sm[kDecWaves][16];
  __shared__ float sl[kDecWaves][16];
  __shared__ float so[kDecWaves][kDecD][17];
  __shared__ int is_last;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int r = lane % 16, g = lane / 16;
  const int bk = blockIdx.y;
  const int b = bk / Hkv, kvh = bk % Hkv;
  const int group = Hq / Hkv;
  const int64_t stride = static_cast<int64_t>(max_splits) * kDecWaves;  // waves per sequence
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kDecWaves + wave;
  // The sequence length and this wave's cache block ids are independent loads: issue both,
  // one block id per lane (lane k holds the id of the wave's k-th block).
  const int32_t* table = block_table + static_cast<int64_t>(b) * max_blocks;
  const int64_t my_blk_index = first + static_cast<int64_t>(lane) * stride;
  const int32_t my_blk = my_blk_index < max_blocks ? table[my_blk_index] : 0;
  const int64_t past_b = positions != nullptr ? loadIndex(positions, pos64, b) : past;
  int64_t L = past_b + 1;
  if (L > max_blocks * kDecBlock) L = max_blocks * kDecBlock;
  const int64_t n_live = L > 0 ? (L + kDecBlock - 1) / kDecBlock : 0;
  // splits holding at least one block (split s holds block s * kDecWaves first)
  const int n_active = static_cast<int>(
      n_live > static_cast<int64_t>(max_splits) * kDecWaves ? max_splits
                                                            : (n_live + kDecWaves - 1) / kDecWaves);
  const bool active = static_cast<int>(blockIdx.x) < n_active;  // uniform per workgroup
  if (!active && max_splits == 1) {  // empty sequence: zeros
    for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x)
      out[(static_cast<int64_t>(b) * Hq + kvh * group + idx / kDecD) * kDecD + idx % kDecD] = 0;
    return;
  }

  if (active) {
    U128 qf[2];
    if (r < group) {
      const uint16_t* qp = q + (static_cast<int64_t>(b) * Hq + kvh * group + r) * kDecD + g * 8;
      qf[0] = load16(qp);
      qf[1] = load16(qp + 32);
    } else {
      qf[0] = zero16();
      qf[1] = zero16();
    }

    SoftmaxState st8;
#pragma unroll
    for (int d = 0; d < 4; ++d) st8.o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    KvBlockRegs bufA, bufB;
    int k = 0;  // ordinal of the wave's block
    int64_t i = first;
    if (i < n_live) loadKvBlock(bufA, k_pool, v_pool, __shfl(my_blk, 0, kWave), i, L, Hkv, kvh, r, g);
    for (; i < n_live; i += 2 * stride, k += 2) {
      const int64_t j = i + stride;
      if (j < n_live) loadKvBlock(bufB, k_pool, v_pool, __shfl(my_blk, k + 1, kWave), j, L, Hkv, kvh, r, g);
      attendBlock(st8, bufA, qf, i * kDecBlock, L, g, scale_log2);
      if (j >= n_live) break;
      const int64_t k2 = j + stride;
      if (k2 < n_live) loadKvBlock(bufA, k_pool, v_pool, __shfl(my_blk, k + 2, kWave), k2, L, Hkv, kvh, r, g);
      attendBlock(st8, bufB, qf, j * kDecBlock, L, g, scale_log2);
    }

    if (g == 0) {
      sm[wave][r] = st8.m;
      sl[wave][r] = st8.l;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) so[wave][d * 16 + 4 * g + e][r] = st8.o[d][e];
    __syncthreads();
    for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x) {
      const int hl = idx / kDecD, d = idx % kDecD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, sm[w][hl]);
      float l = 0.f, acc = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float e = sm[w][hl] == -INFINITY ? 0.f : exp2f(sm[w][hl] - M);
        l += e * sl[w][hl];
        acc += e * so[w][d][hl];
      }
      const int64_t row = static_cast<int64_t>(b) * Hq + kvh * group + hl;
      if (max_splits == 1) {
        out[row * kDecD + d] = floatToBf16(acc / l);
        continue;
      }
      const int64_t slot = row * max_splits + blockIdx.x;
      if (d == 0) {
        __hip_atomic_store(ws_ml + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ws_ml + slot * 2 + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(ws_o + slot * kDecD + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (max_splits == 1) return;

  // Arrive: every partial store of this workgroup has completed before the counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(counters + bk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = old + 1 == static_cast<unsigned>(max_splits);
    if (is_last) __hip_atomic_store(counters + bk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;

  // Merge the splits that hold keys (the rest wrote nothing this call), in split order. The
  // loads of a chunk of kCombineChunk splits are all issued before any is used, so their
  // memory round trips overlap.
  constexpr int kCombineChunk = 8;
  const int n = n_active;
  for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x) {
    const int hl = idx / kDecD, d = idx % kDecD;
    const int64_t row = static_cast<int64_t>(b) * Hq + kvh * group + hl;
    float M = -INFINITY, l = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < n; s0 += kCombineChunk) {
      float ms[kCombineChunk], ls[kCombineChunk], os[kCombineChunk];
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        const bool live = s0 + c < n;
        const int64_t slot = row * max_splits + (live ? s0 + c : 0);
        ms[c] = live ? __hip_atomic_load(ws_ml + slot * 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : -INFINITY;
        ls[c] = live ? __hip_atomic_load(ws_ml + slot * 2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
        os[c] = live ? __hip_atomic_load(ws_o + slot * kDecD + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
      }
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        if (s0 + c >= n) break;
        const float m_new = fmaxf(M, ms[c]);
        const float a = M == -INFINITY ? 0.f : exp2f(M - m_new);
        const float e = ms[c] == -INFINITY ? 0.f : exp2f(ms[c] - m_new);
        l = l * a + ls[c] * e;
        acc = acc * a + os[c] * e;
        M = m_new;
      }
    }
    out[row * kDecD + d] = n > 0 ? floatToBf16(acc / l) : uint16_t{0};  // no keys: zeros
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(kDecWaves * 64)
    decode_attention_d64(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                         const int32_t* block_table, const void* positions, int pos64, int64_t past,
                         float* ws_ml, float* ws_o, unsigned* counters, uint16_t* out, int Hq,
                         int Hkv, int64_t max_blocks, int max_splits, float scale_log2) {
  decode_attention_impl(q, k_pool, v_pool, block_table, positions, pos64, past, ws_ml, ws_o,
                        counters, out, Hq, Hkv, max_blocks, max_splits, scale_log2);
}
