#pragma once

// Decode attention over the paged cache with MFMA (bf16, head_dim 64, one query per sequence,
// up to 16 query heads per KV head), attention/kernel.py:6-62 semantics for a single query row
// at position positions[b] (past = positions[b], keys [0, positions[b]] visible).
//
// "Flash decoding": the work of one (sequence, kv head) pair is split along the keys into
// `splits` units; a unit owns a share of the pair's cache blocks and all query heads of the
// group, so each K/V byte is read once per KV head rather than once per query head. A unit is
// one 8-wave workgroup (the one-stage kernel in attention.hip, or one turn of the persistent
// decoder-stack kernel in stack.hip).
//
// Per wave and 32-key sub-tile (v_mfma_f32_16x16x32_bf16):
//   S = K Q^T    A = 16 keys x 32 dims (two MFMAs per 64 dims), B = Q^T (16 heads).
//                The A rows of half hf are keys t0 + 8*(r/4) + 4*hf + r%4, so the output lane
//                (r, g) holds keys t0 + 8g + 4hf + i (i < 4) of head r: eight consecutive keys.
//   online softmax per head column (max/sum over the 4 lane groups with xor-shuffles)
//   O^T += V^T P^T  A = V^T (16 dims x 32 keys, dim-major cache blocks give 16-byte runs),
//                B = P^T straight from the registers above (no LDS round trip).
// The 8 waves of a unit merge (m, l, O) through LDS; the last unit of a pair to finish merges
// the units' partials.
#include "common.h"
#include "skinny.h"

namespace dk {

constexpr int kDecD = 64;
// Workgroup = kDecWaves waves over the key range of one unit; wave w takes cache blocks
// w, w + kDecWaves, ... of that range (a whole block of 64 keys = two 32-key MFMA sub-tiles,
// so every V row segment of a block is consumed by one wave). The next block's K/V loads are
// issued before the current block is computed (two register buffers).
constexpr int kDecWaves = 8;
constexpr int kDecThreads = kDecWaves * kWave;
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

// One cache block of one kv head staged in LDS (the pools' layouts: K token-major, V dim-major).
struct KvBlockLds {
  uint16_t k[kDecBlock * kDecD];
  uint16_t v[kDecD * kDecBlock];
};

// Copies block `blk` of kv head kvh into dst with direct global-to-LDS loads
// (global_load_lds_dwordx4: no registers held while the data is in flight). Copy j of lane i
// moves bytes [1024 j + 16 i, +16) of the K block and then of the V block. One wave.
__device__ __forceinline__ void stageKvBlock(KvBlockLds* dst, const uint16_t* k_pool,
                                             const uint16_t* v_pool, int64_t blk, int Hkv,
                                             int kvh, int lane) {
  const int64_t head_stride = static_cast<int64_t>(kDecBlock) * kDecD;
  const uint16_t* kb = k_pool + (blk * Hkv + kvh) * head_stride;
  const uint16_t* vb = v_pool + (blk * Hkv + kvh) * head_stride;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_global_load_lds(kb + j * 512 + lane * 8, dst->k + j * 512, 16, 0, 0);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_global_load_lds(vb + j * 512 + lane * 8, dst->v + j * 512, 16, 0, 0);
}

// loadKvBlock from a block staged in LDS (same fragments, same masking).
__device__ __forceinline__ void loadKvBlockLds(KvBlockRegs& regs, const KvBlockLds* src,
                                               int64_t blk_index, int64_t end, int r, int g) {
  const int64_t t_block = blk_index * kDecBlock;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int off = 32 * st + 8 * (r / 4) + 4 * hf + (r % 4);
      const bool ok = t_block + off < end;
      regs.k[st][hf][0] = ok ? load16(src->k + off * kDecD + g * 8) : zero16();
      regs.k[st][hf][1] = ok ? load16(src->k + off * kDecD + 32 + g * 8) : zero16();
    }
    const bool vok = t_block + 32 * st + 8 * g < end;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      regs.v[st][d] = vok ? load16(src->v + (d * 16 + r) * kDecBlock + 32 * st + 8 * g) : zero16();
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
  FP_EXACT;
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

struct DecodeAttnArgs {
  const uint16_t* q;  // [B, Hq, D]
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  const int32_t* block_table;  // [B, max_blocks]
  const void* positions;       // [B] int32/int64, or NULL: every sequence at `past`
  int pos64;
  int64_t past;
  float* ws_ml;  // [B Hq][max_splits][2]   (m, l) per unit
  float* ws_o;   // [B Hq][max_splits][64]  unnormalized O per unit
  unsigned* counters;  // [B Hkv] arrivals per pair
  uint16_t* out;       // [B, Hq, D]
  int Hq, Hkv;
  int64_t max_blocks;
  int max_splits;
  float scale_log2;  // softmax scale * log2(e)
};

// LDS of one unit (kDecWaves waves).
struct DecodeAttnLds {
  float sm[kDecWaves][16];
  float sl[kDecWaves][16];
  float so[kDecWaves][kDecD][17];
  int is_last;
};

// Stages in stage[w], for each wave w < waves of unit `split` of pair `pair`, the third cache
// block decodeAttentionUnit would stage at its start (never the newest-token block), so that a
// later call with prestaged = waves on the same positions, block table and pools finds it there
// and streams less after its gate. Loads complete in issue order: the caller issues this where
// nothing latency-critical of the same waves follows soon.
__device__ __forceinline__ void stageThirdKvBlocks(const DecodeAttnArgs& a, int split, int pair,
                                                   KvBlockLds* stage, int waves) {
  const int tid = freshThreadIdx();
  const int lane = tid % kWave, wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  if (wave >= waves) return;
  const int b = pair / a.Hkv, kvh = pair % a.Hkv;
  const int64_t stride = static_cast<int64_t>(a.max_splits) * kDecWaves;
  const int64_t third = static_cast<int64_t>(split) * kDecWaves + wave + 2 * stride;
  const int64_t past_b = a.positions != nullptr ? loadIndex(a.positions, a.pos64, b) : a.past;
  int64_t L = past_b + 1;
  if (L > a.max_blocks * kDecBlock) L = a.max_blocks * kDecBlock;
  const int64_t n_live = L > 0 ? (L + kDecBlock - 1) / kDecBlock : 0;
  if (third >= n_live || third == n_live - 1) return;
  const int32_t blk = a.block_table[static_cast<int64_t>(b) * a.max_blocks + third];
  stageKvBlock(stage + wave, a.k_pool, a.v_pool, blk, a.Hkv, kvh, lane);
}

// One unit: split `split` of pair (b, kvh) = `pair`. The live cache blocks of a pair are dealt
// round-robin over the splits x kDecWaves waves of its units: wave w of split s takes blocks
// s * kDecWaves + w, + splits * kDecWaves, ..., so every wave streams the same number of blocks
// whatever the sequence length. With one split the normalized output is written directly.
// Otherwise each unit stores its (m, l, O) partial with agent-scope stores and arrives at
// counters[pair]; the unit whose arrival brings the counter to `arrivals` reads every partial
// with agent-scope loads and merges them in split order (no cross-workgroup fence), resetting
// the counter to zero first when `reset` is set. q is read and out written with Mem.
// Returns true in the unit that wrote the pair's output rows. Requires max_blocks <= max_splits
// * kDecWaves * 64 (a wave keeps its block ids in 64 lanes).
//
// When q and the newest token's k/v are produced by another workgroup of the same launch:
// gate() (every thread of the workgroup calls it) returns once q is ready, and kv_ready() (one
// wave calls it) once the cache holds the newest token, which only the block holding position
// positions[b] needs. With kPreload each wave requests its first two cache blocks before gate()
// (except the newest-token block), so the K/V stream overlaps the wait. The arithmetic does not
// depend on these choices. With `stage` (kDecWaves blocks of LDS, which may overlap `s`) each
// wave also stages its third block in LDS before gate(), so a wave with three blocks streams
// nothing after the wait either; waves below `prestaged` find that block already staged there
// by stageThirdKvBlocks. The wave holding the newest-token block calls kv_ready() right after
// gate() and requests that block into the slot left free for it.
template <class Mem, bool kPreload, class Gate, class KvReady>
__device__ __forceinline__ bool decodeAttentionUnit(const DecodeAttnArgs& a, int split, int pair,
                                                    unsigned arrivals, bool reset,
                                                    DecodeAttnLds& s, KvBlockLds* stage,
                                                    int prestaged, Gate&& gate,
                                                    KvReady&& kv_ready) {
  FP_EXACT;
  const int tid = freshThreadIdx();
  const int lane = tid % kWave, wave = tid / kWave;
  const int r = lane % 16, g = lane / 16;
  const int b = pair / a.Hkv, kvh = pair % a.Hkv;
  const int group = a.Hq / a.Hkv;
  const int max_splits = a.max_splits;
  const int64_t stride = static_cast<int64_t>(max_splits) * kDecWaves;  // waves per sequence
  const int64_t first = static_cast<int64_t>(split) * kDecWaves + wave;
  // The sequence length and this wave's cache block ids are independent loads: issue both,
  // one block id per lane (lane k holds the id of the wave's k-th block).
  const int32_t* table = a.block_table + static_cast<int64_t>(b) * a.max_blocks;
  const int64_t my_blk_index = first + static_cast<int64_t>(lane) * stride;
  const int32_t my_blk = my_blk_index < a.max_blocks ? table[my_blk_index] : 0;
  const int64_t past_b = a.positions != nullptr ? loadIndex(a.positions, a.pos64, b) : a.past;
  int64_t L = past_b + 1;
  if (L > a.max_blocks * kDecBlock) L = a.max_blocks * kDecBlock;
  const int64_t n_live = L > 0 ? (L + kDecBlock - 1) / kDecBlock : 0;
  // splits holding at least one block (split s holds block s * kDecWaves first)
  const int n_active = static_cast<int>(
      n_live > static_cast<int64_t>(max_splits) * kDecWaves ? max_splits
                                                            : (n_live + kDecWaves - 1) / kDecWaves);
  const bool active = split < n_active;  // uniform per workgroup
  if (!active && max_splits == 1) {  // empty sequence: zeros
    for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x)
      Mem::storeU16(a.out + (static_cast<int64_t>(b) * a.Hq + kvh * group + idx / kDecD) * kDecD +
                        idx % kDecD,
                    uint16_t{0});
    return true;
  }

  SoftmaxState st8;
#pragma unroll
  for (int d = 0; d < 4; ++d) st8.o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  KvBlockRegs bufA, bufB;
  const int64_t newest = n_live - 1;  // the block holding position L - 1
  bool kv_seen = false;  // kv_ready() has returned in this wave
  auto fetch = [&](KvBlockRegs& buf, int64_t bi, int ordinal) {
    if (bi == newest && !kv_seen) {
      kv_ready();
      kv_seen = true;
    }
    loadKvBlock(buf, a.k_pool, a.v_pool, __shfl(my_blk, ordinal, kWave), bi, L, a.Hkv, kvh, r, g);
  };
  bool a_ready = false, b_ready = false, c_staged = false;
  if (kPreload && active) {
    if (first < n_live && first != newest) {
      fetch(bufA, first, 0);
      a_ready = true;
    }
    if (first + stride < n_live && first + stride != newest) {
      fetch(bufB, first + stride, 1);
      b_ready = true;
    }
    const int64_t third = first + 2 * stride;
    if (stage != nullptr && third < n_live && third != newest) {
      if (wave >= prestaged)
        stageKvBlock(stage + wave, a.k_pool, a.v_pool, __shfl(my_blk, 2, kWave), a.Hkv, kvh,
                     lane);
      c_staged = true;
    }
  }
  gate();  // also before an inactive unit arrives, so arrivals of one call never mix with the next

  if (active) {
    U128 qf[2];
    if (r < group) {
      const uint16_t* qp = a.q + (static_cast<int64_t>(b) * a.Hq + kvh * group + r) * kDecD + g * 8;
      qf[0] = Mem::load16(qp);
      qf[1] = Mem::load16(qp + 32);
    } else {
      qf[0] = zero16();
      qf[1] = zero16();
    }
    // The wave holding the newest-token block waits for it now, while q is in flight, and
    // requests it into the slot the preload left free for it (so its latency overlaps the
    // wave's other blocks instead of following them).
    if (kPreload && newest >= first && (newest - first) % stride == 0) {
      const int64_t kn = (newest - first) / stride;
      if (kn == 0) {
        fetch(bufA, newest, 0);
        a_ready = true;
      } else if (kn == 1) {
        fetch(bufB, newest, 1);
        b_ready = true;
      } else if (kn == 2 && stage != nullptr) {
        kv_ready();
        kv_seen = true;
        stageKvBlock(stage + wave, a.k_pool, a.v_pool, __shfl(my_blk, 2, kWave), a.Hkv, kvh, lane);
        c_staged = true;
      }
    }
    int k = 0;  // ordinal of the wave's block
    for (int64_t i = first; i < n_live; i += 2 * stride, k += 2) {
      if (!a_ready) fetch(bufA, i, k);
      const int64_t j = i + stride;
      if (j < n_live && !b_ready) fetch(bufB, j, k + 1);
      a_ready = b_ready = false;
      attendBlock(st8, bufA, qf, i * kDecBlock, L, g, a.scale_log2);
      if (j >= n_live) break;
      const int64_t k2 = j + stride;
      if (k2 < n_live) {
        if (c_staged && k == 0) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged block has landed
          loadKvBlockLds(bufA, stage + wave, k2, L, r, g);
        } else {
          fetch(bufA, k2, k + 2);
        }
        a_ready = true;
      }
      attendBlock(st8, bufB, qf, j * kDecBlock, L, g, a.scale_log2);
    }
    if (stage != nullptr) __syncthreads();  // staged blocks are consumed before s reuses LDS

    if (g == 0) {
      s.sm[wave][r] = st8.m;
      s.sl[wave][r] = st8.l;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) s.so[wave][d * 16 + 4 * g + e][r] = st8.o[d][e];
    __syncthreads();
    for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x) {
      const int hl = idx / kDecD, d = idx % kDecD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, s.sm[w][hl]);
      float l = 0.f, acc = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float e = s.sm[w][hl] == -INFINITY ? 0.f : exp2f(s.sm[w][hl] - M);
        l += e * s.sl[w][hl];
        acc += e * s.so[w][d][hl];
      }
      const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + hl;
      if (max_splits == 1) {
        Mem::storeU16(a.out + row * kDecD + d, floatToBf16(acc / l));
        continue;
      }
      const int64_t slot = row * max_splits + split;
      if (d == 0) {
        __hip_atomic_store(a.ws_ml + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ws_ml + slot * 2 + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(a.ws_o + slot * kDecD + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (max_splits == 1) return true;

  // Arrive: every partial store of this workgroup has completed before the counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(a.counters + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s.is_last = old + 1 == arrivals;
    if (s.is_last && reset)
      __hip_atomic_store(a.counters + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s.is_last) return false;

  // Merge the splits that hold keys (the rest wrote nothing this call), in split order. The
  // loads of a chunk of kCombineChunk splits are all issued before any is used, so their
  // memory round trips overlap.
  constexpr int kCombineChunk = 8;
  const int n = n_active;
  for (int idx = threadIdx.x; idx < group * kDecD; idx += blockDim.x) {
    const int hl = idx / kDecD, d = idx % kDecD;
    const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + hl;
    float M = -INFINITY, l = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < n; s0 += kCombineChunk) {
      float ms[kCombineChunk], ls[kCombineChunk], os[kCombineChunk];
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        const bool live = s0 + c < n;
        const int64_t slot = row * max_splits + (live ? s0 + c : 0);
        ms[c] = live ? __hip_atomic_load(a.ws_ml + slot * 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : -INFINITY;
        ls[c] = live ? __hip_atomic_load(a.ws_ml + slot * 2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
        os[c] = live ? __hip_atomic_load(a.ws_o + slot * kDecD + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
      }
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        if (s0 + c >= n) break;
        const float m_new = fmaxf(M, ms[c]);
        const float al = M == -INFINITY ? 0.f : exp2f(M - m_new);
        const float e = ms[c] == -INFINITY ? 0.f : exp2f(ms[c] - m_new);
        l = l * al + ls[c] * e;
        acc = acc * al + os[c] * e;
        M = m_new;
      }
    }
    Mem::storeU16(a.out + row * kDecD + d, n > 0 ? floatToBf16(acc / l) : uint16_t{0});  // no keys: zeros
  }
  return true;
}

}  // namespace dk
