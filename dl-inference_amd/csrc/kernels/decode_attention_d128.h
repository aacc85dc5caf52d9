#pragma once

// Decode attention over the paged cache with MFMA for head_dim 128 (the Qwen2-7B geometry: 28
// query heads over 4 KV heads, groups of 7), attention/kernel.py:6-62 semantics for one query
// row per sequence at position positions[b] (keys [0, positions[b]] visible; the new token's
// key and value are already in the cache).
//
// One workgroup of 8 waves per (sequence, group of kv heads, split): hpw kv heads per
// workgroup, 8 / hpw waves per head (hpw = 1: all eight on one head, the head_dim-64 kernel's
// decomposition). The query heads of a GQA group form the 16 columns of the MFMA; a sequence's
// 64-key cache blocks are dealt round-robin over the waves of one head in all its splits.
// With hpw = Hkv (the host's choice when Hkv divides 8) a workgroup reads every kv head of the
// same cache blocks, which sit next to each other in the pools ([block, Hkv, ...]): contiguous
// 4 x 16 KB per block at the Qwen2-7B geometry. A streaming probe read that order at 5.6 TB/s
// against 4.9 TB/s for one head's 16 KB out of every 64 KB, the order of one head per
// workgroup. A 64-key block of a 128-dim head is 32 KB of K and V; a wave loads a whole block
// into registers and works through it as two 32-key halves:
//   S = K Q^T   four MFMAs per 16 keys (v_mfma_f32_16x16x32_bf16, 32 dims each); the A rows
//               of half hf are keys 8 (r / 4) + 4 hf + r % 4, so output lane (r, g) holds keys
//               8g .. 8g + 7 of the 32-key half for head r
//   O^T += V^T P^T   eight 16-dim groups; V is dim-major in the pool, so each A fragment is a
//               16-byte run of 8 keys; P^T is the lane's own probabilities (hi + lo bf16 parts)
// Online softmax in base 2 with one maximum per 32-key half. The 8 waves merge (m, l, O)
// through LDS; with several splits the last unit of a pair to arrive merges the units'
// partials in split order (agent-scope stores and loads, a per-pair counter it leaves at zero).
#include "common.h"
#include "skinny.h"

namespace dk {

constexpr int kD128 = 128;
constexpr int kD128Waves = 8;
constexpr int kD128Threads = kD128Waves * kWave;
constexpr int kD128Block = 64;  // keys per cache block

// K and V fragments of one 32-key half of a cache block.
struct KvHalf128 {
  U128 k[2][4];  // [hf][32-dim chunk]
  U128 v[8];     // [16-dim group]
};

// Both 32-key halves of one cache block: K of half 0 and 1, then V with the two loads of each
// 16-dim group (slots 0-31 and 32-63 of the same 128-byte dim rows) next to each other. A
// fragment load reads 64 bytes of each of 16 rows, so every V line is read by two loads; when
// they went out far apart (one per half, or the compiler sinking loads towards their first
// use) the line was often fetched from HBM twice: 1.48 GB per launch for 1.07 GB of K and V at
// the Qwen2-7B geometry, all of the excess on V. The caller keeps the loads together with a
// scheduling barrier.
__device__ __forceinline__ void loadKvBlock128(KvHalf128& h0, KvHalf128& h1,
                                               const uint16_t* k_pool, const uint16_t* v_pool,
                                               int64_t blk, int Hkv, int kvh, int r, int g) {
  const int64_t head_stride = static_cast<int64_t>(kD128Block) * kD128;
  const uint16_t* kbase = k_pool + (blk * Hkv + kvh) * head_stride;
  const uint16_t* vbase = v_pool + (blk * Hkv + kvh) * head_stride;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    KvHalf128& h = st ? h1 : h0;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int key = 32 * st + 8 * (r / 4) + 4 * hf + (r % 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) h.k[hf][c] = gload16(kbase + key * kD128 + 32 * c + g * 8);
    }
  }
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    h0.v[d] = gload16(vbase + (d * 16 + r) * kD128Block + 8 * g);
    h1.v[d] = gload16(vbase + (d * 16 + r) * kD128Block + 32 + 8 * g);
  }
}

struct Softmax128 {
  float m = -INFINITY;
  float l = 0.f;
  f32x4 o[8];
};

// One 32-key half whose first key is t0; keys at or past `end` are masked.
__device__ __forceinline__ void attendHalf128(Softmax128& s, const KvHalf128& h,
                                              const U128 (&qf)[4], int64_t t0, int64_t end,
                                              int g, float scale_log2) {
  FP_EXACT;
  f32x4 sc[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    sc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      sc[hf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(h.k[hf][c]), asBf16x8(qf[c]),
                                                       sc[hf], 0, 0, 0);
  }
  const int64_t rem64 = end - t0;
  const int rem = rem64 < 32 ? static_cast<int>(rem64) : 32;
  float mx = -INFINITY;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = 8 * g + 4 * hf + e;
      const float v = (rem == 32 || key < rem) ? sc[hf][e] * scale_log2 : -INFINITY;
      sc[hf][e] = v;
      mx = fmaxf(mx, v);
    }
  mx = rowsMax(mx);
  const float m_new = fmaxf(s.m, mx);
  const float alpha = exp2f(s.m - m_new);
  float p[2][4];
  float sum = 0.f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[hf][e] = exp2f(sc[hf][e] - m_new);
      sum += p[hf][e];
    }
  s.l = s.l * alpha + sum;
  s.m = m_new;
#pragma unroll
  for (int d = 0; d < 8; ++d) s.o[d] *= alpha;
  // V rows of keys past the end are zeroed (whole 8-key groups of a lane), so stale pool
  // contents never reach O even where P is 0.
  const bool live = rem == 32 || 8 * g < rem;
  U128 phi, plo;
#pragma unroll
  for (int w2 = 0; w2 < 4; ++w2) {
    const float a0 = p[w2 / 2][(w2 % 2) * 2], a1 = p[w2 / 2][(w2 % 2) * 2 + 1];
    phi[w2] = packBf16x2(a0, a1);
    plo[w2] = packBf16x2(a0 - bf16ToFloat(static_cast<uint16_t>(phi[w2])),
                         a1 - bf16ToFloat(static_cast<uint16_t>(phi[w2] >> 16)));
  }
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const U128 vf = live ? h.v[d] : zero16();
    s.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vf), asBf16x8(phi), s.o[d], 0, 0, 0);
    s.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vf), asBf16x8(plo), s.o[d], 0, 0, 0);
  }
}

struct DecodeAttn128Lds {
  float sm[kD128Waves][16];
  float sl[kD128Waves][16];
  float so[kD128Waves][kD128][17];
  int is_last[kD128Waves];
};

struct DecodeAttn128Args {
  const uint16_t* q;  // [B, Hq, 128]
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  const int32_t* block_table;  // [B, max_blocks]
  const void* positions;       // [B] int32/int64, or NULL: every sequence at `past`
  int pos64;
  int64_t past;
  float* ws_ml;        // [B Hq][splits][2]
  float* ws_o;         // [B Hq][splits][128]
  unsigned* counters;  // [B Hkv]
  uint16_t* out;       // [B, Hq, 128]
  int Hq, Hkv;
  int64_t max_blocks;
  int splits;
  float scale_log2;
};

// Unit `split` of kv heads [h0, h0 + hpw) of sequence b (unit = (b Hkv + h0) / hpw). Wave w
// serves head h0 + w / wph (wph = 8 / hpw waves per head) and, as sub-wave u = w % wph of split
// s, takes cache blocks s * wph + u, + splits * wph, ... of the sequence's L = positions[b] + 1
// keys. Returns after writing each head's output (one split) or its partials (and, in the last
// unit of a (sequence, kv head) pair to arrive, that pair's merge).
__device__ __forceinline__ void decodeAttention128Unit(const DecodeAttn128Args& a, int split,
                                                       int unit, int hpw, DecodeAttn128Lds& s) {
  FP_EXACT;
  const int tid = freshThreadIdx();
  const int lane = tid % kWave, wave = tid / kWave;
  const int r = lane % 16, g = lane / 16;
  const int wph = kD128Waves / hpw;
  const int b = (unit * hpw) / a.Hkv, h0 = (unit * hpw) % a.Hkv;
  // uniform over the wave: the head's pool offsets and the block walk stay scalar
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int kvh = h0 + wave_u / wph;
  const int group = a.Hq / a.Hkv;
  const int64_t stride = static_cast<int64_t>(a.splits) * wph;
  const int64_t first = static_cast<int64_t>(split) * wph + wave_u % wph;
  // The wave's cache block ids, one per lane (lane k holds the id of the wave's k-th block; the
  // split count keeps that below 64), loaded once: a block id read in the loop made every fetch
  // wait, in order, for the loads issued before it.
  const int32_t* table = a.block_table + static_cast<int64_t>(b) * a.max_blocks;
  const int64_t my_blk_index = first + static_cast<int64_t>(lane) * stride;
  const int32_t my_blk = my_blk_index < a.max_blocks ? gp(table)[my_blk_index] : 0;
  const int64_t past_b = a.positions != nullptr ? loadIndex(a.positions, a.pos64, b) : a.past;
  int64_t L = past_b + 1;
  if (L > a.max_blocks * kD128Block) L = a.max_blocks * kD128Block;
  if (L < 0) L = 0;
  const int64_t n_blocks = (L + kD128Block - 1) / kD128Block;

  Softmax128 st;
#pragma unroll
  for (int d = 0; d < 8; ++d) st.o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  U128 qf[4];
  if (r < group) {
    const uint16_t* qp = a.q + (static_cast<int64_t>(b) * a.Hq + kvh * group + r) * kD128 + g * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = gload16(qp + 32 * c);
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[c] = zero16();
  }
  // this wave's blocks in order: block i is first + i * stride, attended as two 32-key halves.
  // One block's loads are in flight per wave at a time, issued together (the scheduling barrier
  // keeps the compiler from spreading them out: a V line read by two loads far apart was often
  // fetched twice); the CU's other waves keep the memory busy meanwhile. Measured at batch 64,
  // context 8192: 240 -> 203 us, 1.48 -> 1.10 GB fetched per launch.
  const int64_t my_blocks = first < n_blocks ? (n_blocks - first + stride - 1) / stride : 0;
  KvHalf128 buf[2];
  for (int64_t i = 0; i < my_blocks; ++i) {
    const int64_t blk = __builtin_amdgcn_readlane(my_blk, static_cast<int>(i));
    loadKvBlock128(buf[0], buf[1], a.k_pool, a.v_pool, blk, a.Hkv, kvh, r, g);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t t0 = (first + i * stride) * kD128Block;
    attendHalf128(st, buf[0], qf, t0, L, g, a.scale_log2);
    attendHalf128(st, buf[1], qf, t0 + 32, L, g, a.scale_log2);
  }

  // merge the waves through LDS (each lane holds l for its 8 keys of every half: rowsSum)
  const float l_col = rowsSum(st.l);
  if (g == 0) {
    s.sm[wave][r] = st.m;
    s.sl[wave][r] = l_col;
  }
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int e = 0; e < 4; ++e) s.so[wave][d * 16 + 4 * g + e][r] = st.o[d][e];
  __syncthreads();
  // merge each head's wph waves in wave order
  for (int idx = threadIdx.x; idx < hpw * group * kD128; idx += kD128Threads) {
    const int hw = idx / (group * kD128), hl = idx / kD128 % group, d = idx % kD128;
    const int w0 = hw * wph;
    float M = -INFINITY;
    for (int w = w0; w < w0 + wph; ++w) M = fmaxf(M, s.sm[w][hl]);
    float l = 0.f, acc = 0.f;
    for (int w = w0; w < w0 + wph; ++w) {
      const float e = s.sm[w][hl] == -INFINITY ? 0.f : exp2f(s.sm[w][hl] - M);
      l += e * s.sl[w][hl];
      acc += e * s.so[w][d][hl];
    }
    const int64_t row = static_cast<int64_t>(b) * a.Hq + (h0 + hw) * group + hl;
    if (a.splits == 1) {
      *gp(a.out + row * kD128 + d) = l > 0.f ? floatToBf16(acc / l) : uint16_t{0};
      continue;
    }
    const int64_t slot = row * a.splits + split;
    if (d == 0) {
      __hip_atomic_store(gp(a.ws_ml) + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gp(a.ws_ml) + slot * 2 + 1, l, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(gp(a.ws_o) + slot * kD128 + d, acc, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  if (a.splits == 1) return;

  // arrive: every partial store of this workgroup has completed before the counters move (one
  // per (sequence, kv head) pair of the unit)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x < hpw) {
    const int pair = b * a.Hkv + h0 + threadIdx.x;
    const unsigned old = __hip_atomic_fetch_add(gp(a.counters) + pair, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == static_cast<unsigned>(a.splits);
    s.is_last[threadIdx.x] = last;
    if (last)
      __hip_atomic_store(gp(a.counters) + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // merge every split's partial in split order (a split without keys left m = -inf, l = 0), for
  // the pairs whose last unit this is
  for (int idx = threadIdx.x; idx < hpw * group * kD128; idx += kD128Threads) {
    const int hw = idx / (group * kD128), hl = idx / kD128 % group, d = idx % kD128;
    if (!s.is_last[hw]) continue;
    const int64_t row = static_cast<int64_t>(b) * a.Hq + (h0 + hw) * group + hl;
    float M = -INFINITY, l = 0.f, acc = 0.f;
    for (int sp = 0; sp < a.splits; ++sp) {
      const int64_t slot = row * a.splits + sp;
      const float mc = __hip_atomic_load(gp(a.ws_ml) + slot * 2, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float lc = __hip_atomic_load(gp(a.ws_ml) + slot * 2 + 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float oc = __hip_atomic_load(gp(a.ws_o) + slot * kD128 + d, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float m_new = fmaxf(M, mc);
      const float al = M == -INFINITY ? 0.f : exp2f(M - m_new);
      const float ec = mc == -INFINITY ? 0.f : exp2f(mc - m_new);
      l = l * al + lc * ec;
      acc = acc * al + oc * ec;
      M = m_new;
    }
    *gp(a.out + row * kD128 + d) = l > 0.f ? floatToBf16(acc / l) : uint16_t{0};
  }
}

}  // namespace dk
