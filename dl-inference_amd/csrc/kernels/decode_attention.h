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
//   online softmax per head column, one maximum per 64-key block over the 4 lane rows
//                (permlane swaps); each lane keeps its own share of the sum
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

// K/V fragments of cache block `blk` (kv head kvh). The loads are unconditional: every cache
// block a unit reads is live, so all of its 64 positions are in the pool, and positions past the
// sequence end are masked by attendBlock (scores to -inf, V to zero). Branch-free loads also let
// the compiler wait for exactly the block it computes next (s_waitcnt vmcnt(n)) instead of for
// every load in flight.
__device__ __forceinline__ void loadKvBlock(KvBlockRegs& regs, const uint16_t* k_pool,
                                            const uint16_t* v_pool, int64_t blk, int Hkv, int kvh,
                                            int r, int g) {
  const int64_t head_stride = static_cast<int64_t>(kDecBlock) * kDecD;
  const uint16_t* kbase = k_pool + (blk * Hkv + kvh) * head_stride;
  const uint16_t* vbase = v_pool + (blk * Hkv + kvh) * head_stride;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int off = 32 * st + 8 * (r / 4) + 4 * hf + (r % 4);
      regs.k[st][hf][0] = gload16(kbase + off * kDecD + g * 8);
      regs.k[st][hf][1] = gload16(kbase + off * kDecD + 32 + g * 8);
    }
  }
  // the two halves of each 128-byte V dim row next to each other: a line read by two loads far
  // apart can be fetched from HBM twice
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int st = 0; st < 2; ++st)
      regs.v[st][d] = gload16(vbase + (d * 16 + r) * kDecBlock + 32 * st + 8 * g);
}

// One cache block of one kv head staged in LDS (the pools' layouts: K token-major, V dim-major).
struct KvBlockLds {
  uint16_t k[kDecBlock * kDecD];
  uint16_t v[kDecD * kDecBlock];
};

// Copies block `blk` of kv head kvh into dst with direct global-to-LDS loads
// (global_load_lds_dwordx4: no registers held while the data is in flight). Copy j of lane i
// moves bytes [1024 j + 16 i, +16) of the K block and then of the V block. One wave. The loads
// are nontemporal: each covers whole 128-byte lines of a block read once per step (a streaming
// probe read 6.9 TB/s that way against 6.0 TB/s with the default policy).
__device__ __forceinline__ void stageKvBlock(KvBlockLds* dst, const uint16_t* k_pool,
                                             const uint16_t* v_pool, int64_t blk, int Hkv,
                                             int kvh, int lane) {
  const int64_t head_stride = static_cast<int64_t>(kDecBlock) * kDecD;
  const uint16_t* kb = k_pool + (blk * Hkv + kvh) * head_stride;
  const uint16_t* vb = v_pool + (blk * Hkv + kvh) * head_stride;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_global_load_lds(kb + j * 512 + lane * 8, dst->k + j * 512, 16, 0, 2);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_global_load_lds(vb + j * 512 + lane * 8, dst->v + j * 512, 16, 0, 2);
}

// loadKvBlock from a block staged in LDS (same fragments).
__device__ __forceinline__ void loadKvBlockLds(KvBlockRegs& regs, const KvBlockLds* src, int r,
                                               int g) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int off = 32 * st + 8 * (r / 4) + 4 * hf + (r % 4);
      regs.k[st][hf][0] = load16(src->k + off * kDecD + g * 8);
      regs.k[st][hf][1] = load16(src->k + off * kDecD + 32 + g * 8);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
      regs.v[st][d] = load16(src->v + (d * 16 + r) * kDecBlock + 32 * st + 8 * g);
  }
}

// Online-softmax state of one wave: m is the running maximum (log2 domain) of each head
// column, the same in the four lanes of a column; l is this lane's share of the running sum
// (the lanes of a column are added once, at the end: rowsSum); o is the unnormalized O^T.
struct SoftmaxState {
  float m = -INFINITY;
  float l = 0.f;
  f32x4 o[4];
};

// One 64-key cache block: S for both 32-key sub-tiles first (four independent MFMA chains),
// then one max over the block's keys, P, and O^T += V^T P^T.
__device__ __forceinline__ void attendBlock(SoftmaxState& st8, const KvBlockRegs& regs,
                                            const U128 (&qf)[2], int64_t t_block, int64_t end,
                                            int g, float scale_log2) {
  FP_EXACT;
  f32x4 sc[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      sc[st][hf] = f32x4{0.f, 0.f, 0.f, 0.f};
      sc[st][hf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.k[st][hf][0]), asBf16x8(qf[0]), sc[st][hf], 0, 0, 0);
      sc[st][hf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(regs.k[st][hf][1]), asBf16x8(qf[1]), sc[st][hf], 0, 0, 0);
    }
  // keys of the block below end (uniform per wave; >= 1 for a live block)
  const int64_t rem64 = end - t_block;
  const int rem = rem64 < kDecBlock ? static_cast<int>(rem64) : kDecBlock;
  float mx = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 32 * st + 8 * g + 4 * hf + e;
        const float v = (rem == kDecBlock || key < rem) ? sc[st][hf][e] * scale_log2 : -INFINITY;
        sc[st][hf][e] = v;
        mx = fmaxf(mx, v);
      }
  mx = rowsMax(mx);
  const float m_new = fmaxf(st8.m, mx);
  // The raw v_exp_f32 (2^x without subnormal results): the library exp2f adds five instructions
  // per call to produce subnormal results, 80 of the block's VALU instructions, and this loop is
  // VALU-bound (8 waves, 2 per SIMD). A subnormal p only ever meets a sum l >= 1 (the running
  // maximum contributes 2^0) and P*V terms far below O's last bit, and every path that attends
  // blocks uses this code, so they stay bit-identical to each other.
  const float alpha = __builtin_amdgcn_exp2f(st8.m - m_new);
  float p[2][2][4];
  float sum = 0.f;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[st][hf][e] = __builtin_amdgcn_exp2f(sc[st][hf][e] - m_new);
        sum += p[st][hf][e];
      }
  st8.l = st8.l * alpha + sum;
  st8.m = m_new;
#pragma unroll
  for (int d = 0; d < 4; ++d) st8.o[d] *= alpha;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    // V rows of keys past the end are zeroed (whole 8-key groups of a lane), so stale pool
    // contents there never reach O even where P is 0.
    U128 vf[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      vf[d] = (rem == kDecBlock || 32 * st + 8 * g < rem) ? regs.v[st][d] : zero16();
    // P in two bf16 terms (hi + lo) so the P*V products carry ~16 significant bits of P.
    U128 phi, plo;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float a0 = p[st][w2 / 2][(w2 % 2) * 2], a1 = p[st][w2 / 2][(w2 % 2) * 2 + 1];
      phi[w2] = packBf16x2(a0, a1);
      plo[w2] = packBf16x2(a0 - bf16ToFloat(static_cast<uint16_t>(phi[w2])),
                             a1 - bf16ToFloat(static_cast<uint16_t>(phi[w2] >> 16)));
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      st8.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vf[d]), asBf16x8(phi), st8.o[d], 0, 0, 0);
      st8.o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vf[d]), asBf16x8(plo), st8.o[d], 0, 0, 0);
    }
  }
}

// Folds split partial (mc, lc, oc) into the running merge (M, l, acc) (splits in order).
__device__ __forceinline__ void combineSplit(float& M, float& l, float& acc, float mc, float lc,
                                             float oc) {
  FP_EXACT;
  const float m_new = fmaxf(M, mc);
  const float al = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - m_new);
  const float e = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - m_new);
  l = l * al + lc * e;
  acc = acc * al + oc * e;
  M = m_new;
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
  uint16_t* out;       // [B, Hq, D] (row-major, or fragment order: out_frag_steps)
  int Hq, Hkv;
  int64_t max_blocks;
  int max_splits;
  float scale_log2;  // softmax scale * log2(e)
  // Tagged partials (persistent launches, every unit resident): [B Hq][max_splits][kTagSlot]
  // words (O[64], m, l), or NULL for the counter protocol. See decodeAttentionUnit.
  uint64_t* ws_tag = nullptr;
  unsigned tag = 0;
  unsigned* abort_word = nullptr;
  // > 0: out is [B, Hq * D] in fragment order (fragOffset) with Hq * D / 64 steps
  int out_frag_steps = 0;
  // When set, q is read from here instead: [B, Hq, D / 2] tagged words (the bf16 pair (d, d + 1)
  // and tag `tag`, QkvParams::q_tagged), polled by wave 0 until every word carries the tag.
  const uint64_t* q_tagged = nullptr;
};

// Address of output element (sequence b, query head `head`, dim d).
__device__ __forceinline__ uint16_t* attnOut(const DecodeAttnArgs& a, int64_t b, int64_t head,
                                             int d) {
  const int64_t k = head * kDecD + d;
  return a.out + (a.out_frag_steps > 0 ? fragOffset(static_cast<int>(b), k, a.out_frag_steps)
                                       : b * a.Hq * kDecD + k);
}

constexpr int kTagSlot = kDecD + 2;  // tagged words per (row, split): O, then m and l

// LDS of one unit (kDecWaves waves).
// Splits whose words the merger polls per round (decodeAttentionUnit): kMergeChunk in the
// general loop; up to kOneRoundSplits in one round when it would take more than one.
constexpr int kMergeChunk = 4;
constexpr int kOneRoundSplits = 8;

struct DecodeAttnLds {
  float sm[kDecWaves][16];
  float sl[kDecWaves][16];
  float so[kDecWaves][kDecD][17];
  float pm[kOneRoundSplits][16];  // the other splits' (m, l) of each head, for the merger
  float pl[kOneRoundSplits][16];
  // q of the unit, handed from wave 0 to the others (tagged q). Kept clear of the first
  // sizeof(KvBlockLds) bytes, which a caller may overlay with the last wave's staged cache block.
  U128 q[2 * kWave];
  int is_last;
};

// Stages in stage[w], for each wave w < waves of unit `split` of pair `pair`, the third cache
// block decodeAttentionUnit would stage at its start, so that a
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
  const int64_t L_old = L > 0 ? L - 1 : 0;  // the blocks hold keys [0, L - 1)
  const int64_t n_live = (L_old + kDecBlock - 1) / kDecBlock;
  if (third >= n_live) return;
  const int32_t blk = gp(a.block_table)[static_cast<int64_t>(b) * a.max_blocks + third];
  stageKvBlock(stage + wave, a.k_pool, a.v_pool, blk, a.Hkv, kvh, lane);
}

// One unit: split `split` of pair (b, kvh) = `pair`. The cache blocks holding keys
// [0, positions[b]) are dealt round-robin over the splits x kDecWaves waves of its units: wave w
// of split s takes blocks s * kDecWaves + w, + splits * kDecWaves, ..., so every wave streams the
// same number of blocks whatever the sequence length; the newest key, positions[b], is attended
// as a one-key block by the next wave in that order, after its blocks. With one split the
// normalized output is written directly.
// Otherwise each unit stores its (m, l, O) partial with agent-scope stores and arrives at
// counters[pair]; the unit whose arrival brings the counter to `arrivals` reads every partial
// with agent-scope loads and merges them in split order (no cross-workgroup fence), resetting
// the counter to zero first when `reset` is set. q is read and out written with Mem.
// Returns true in the unit that wrote the pair's output rows. Requires max_blocks <= max_splits
// * kDecWaves * 64 (a wave keeps its block ids in 64 lanes).
//
// With a.ws_tag (every unit of the call resident at once) there is no counter: every active
// unit but the last stores its partial as tagged words (storeTagged, tag a.tag) and is done; the
// last active unit, which holds the fewest blocks, merges the others' partials as their words
// arrive (loadTagged) with its own and writes the output. The merge arithmetic and split order
// are the same as the counter protocol's, so both give bit-identical outputs.
//
// When q and the newest token's k/v are produced by another workgroup of the same launch:
// gate() (every thread of the workgroup calls it) returns once q is ready, and kv_ready() (the
// wave that attends the newest key calls it, after its blocks) once the cache holds the newest
// token; that wave reads the token with agent-scope loads. Every cache block a unit reads was
// complete before the call, so with kPreload each wave requests its first two blocks before
// gate() and the K/V stream overlaps the wait. The arithmetic does not depend on these choices.
// With `stage` (kDecWaves blocks of LDS, which may overlap `s`) each wave also stages its third
// block in LDS before gate(), so a wave with three blocks streams nothing after the wait either;
// waves below `prestaged` find that block already staged there by stageThirdKvBlocks.
//
// mark(p) (every thread calls it) marks internal points for a timeline: 0 when this wave's
// blocks are attended, 1 when every wave's are (after the barrier), 2 after the unit's arrival,
// 3 and 4 when this wave has attended its first and second block, 5 when this wave has q.
static_assert(offsetof(DecodeAttnLds, q) >= sizeof(KvBlockLds), "q clear of a staged block");
template <class Mem, bool kPreload, bool kOneRound = false, class Gate, class KvReady,
          class Mark = NoMark>
__device__ __forceinline__ bool decodeAttentionUnit(const DecodeAttnArgs& a, int split, int pair,
                                                    unsigned arrivals, bool reset,
                                                    DecodeAttnLds& s, KvBlockLds* stage,
                                                    int prestaged, Gate&& gate,
                                                    KvReady&& kv_ready, Mark mark = Mark{}) {
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
  const int32_t my_blk = my_blk_index < a.max_blocks ? gp(table)[my_blk_index] : 0;
  const int64_t past_b = a.positions != nullptr ? loadIndex(a.positions, a.pos64, b) : a.past;
  int64_t L = past_b + 1;
  if (L > a.max_blocks * kDecBlock) L = a.max_blocks * kDecBlock;
  // Keys [0, L - 1) come from cache blocks that were complete before this call; the newest key
  // L - 1 (written by this step) is attended on its own by the wave next in the round-robin
  // after the last block (newest_wave, which holds no more blocks than any other wave), after
  // its blocks and once kv_ready() has returned.
  const int64_t L_old = L > 0 ? L - 1 : 0;
  const int64_t n_live = (L_old + kDecBlock - 1) / kDecBlock;
  const int64_t newest_wave = L > 0 ? n_live % stride : -1;
  // splits holding a block or the newest key (split s holds block s * kDecWaves first)
  const int n_active = static_cast<int>(
      L <= 0 ? 0
             : (n_live >= stride ? max_splits : n_live / kDecWaves + 1));
  const bool active = split < n_active;  // uniform per workgroup
  const bool tagged = a.ws_tag != nullptr && max_splits > 1;
  // the unit that writes the output in the tagged protocol: the last active split, which holds
  // the fewest blocks
  const int merger = n_active > 0 ? n_active - 1 : 0;
  if (!active && (max_splits == 1 || (tagged && split == merger))) {  // empty sequence: zeros
    for (int idx = freshThreadIdx(); idx < group * kDecD; idx += kDecThreads)
      Mem::storeU16(attnOut(a, b, kvh * group + idx / kDecD, idx % kDecD), uint16_t{0});
    return true;
  }

  SoftmaxState st8;
#pragma unroll
  for (int d = 0; d < 4; ++d) st8.o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  KvBlockRegs bufA, bufB;
  auto fetch = [&](KvBlockRegs& buf, int ordinal) {
    loadKvBlock(buf, a.k_pool, a.v_pool, __shfl(my_blk, ordinal, kWave), a.Hkv, kvh, r, g);
  };
  bool a_ready = false, b_ready = false, c_staged = false;
  if (kPreload && active) {
    if (first < n_live) {
      fetch(bufA, 0);
      a_ready = true;
    }
    if (first + stride < n_live) {
      fetch(bufB, 1);
      b_ready = true;
    }
    if (stage != nullptr && first + 2 * stride < n_live) {
      if (wave >= prestaged)
        stageKvBlock(stage + wave, a.k_pool, a.v_pool, __shfl(my_blk, 2, kWave), a.Hkv, kvh,
                     lane);
      c_staged = true;
    }
  }
  gate();  // also before an inactive unit arrives, so arrivals of one call never mix with the next

  if (active) {
    U128 qf[2];
    const int64_t q_at = (static_cast<int64_t>(b) * a.Hq + kvh * group + r) * kDecD + g * 8;
    if (a.q_tagged != nullptr) {
      // Wave 0 polls the unit's q words (one request per 128-byte line and lane group, as few as
      // one counter poll would make) and hands q to the other waves through LDS (every wave of
      // an earlier unit has read s.q before that unit's merge barrier).
      U128* const q_lds = s.q;
      if (wave == 0 && r < group) {
        // dims g*8 .. g*8+7 and 32+g*8 .. 32+g*8+7: words q_at/2 .. +3 and q_at/2+16 .. +19
        const uint64_t* const qw = a.q_tagged + q_at / 2;
        const uint64_t* const ptr[8] = {qw,      qw + 1,  qw + 2,  qw + 3,
                                        qw + 16, qw + 17, qw + 18, qw + 19};
        uint32_t bits[8];
        loadTagged<8>(bits, ptr, 8, a.tag, a.abort_word);
        q_lds[lane] = U128{bits[0], bits[1], bits[2], bits[3]};
        q_lds[kWave + lane] = U128{bits[4], bits[5], bits[6], bits[7]};
      }
      __syncthreads();
      qf[0] = r < group ? q_lds[lane] : zero16();
      qf[1] = r < group ? q_lds[kWave + lane] : zero16();
    } else if (r < group) {
      qf[0] = Mem::load16(a.q + q_at);
      qf[1] = Mem::load16(a.q + q_at + 32);
    } else {
      qf[0] = zero16();
      qf[1] = zero16();
    }
    mark(5);
    int k = 0;  // ordinal of the wave's block
    for (int64_t i = first; i < n_live; i += 2 * stride, k += 2) {
      if (!a_ready) fetch(bufA, k);
      const int64_t j = i + stride;
      if (j < n_live && !b_ready) fetch(bufB, k + 1);
      a_ready = b_ready = false;
      attendBlock(st8, bufA, qf, i * kDecBlock, L_old, g, a.scale_log2);
      if (k == 0) mark(3);
      if (j >= n_live) break;
      const int64_t k2 = j + stride;
      if (k2 < n_live) {
        if (c_staged && k == 0) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged block has landed
          loadKvBlockLds(bufA, stage + wave, r, g);
        } else {
          fetch(bufA, k + 2);
        }
        a_ready = true;
      }
      attendBlock(st8, bufB, qf, j * kDecBlock, L_old, g, a.scale_log2);
      if (k == 0) mark(4);
    }
    if (newest_wave == first) {
      // The newest key as a one-key block: K row 0 and V column 0 of the fragments (lanes r = 0
      // and g = 0), everything else zero and masked (end = L).
      kv_ready();
      const int64_t pos = L - 1;
      const int64_t blk = gp(table)[pos / kDecBlock];
      const int64_t off = pos % kDecBlock;
      const int64_t head_stride = static_cast<int64_t>(kDecBlock) * kDecD;
      const uint16_t* kb = a.k_pool + (blk * a.Hkv + kvh) * head_stride + off * kDecD;
      const uint16_t* vb = a.v_pool + (blk * a.Hkv + kvh) * head_stride + off;
      KvBlockRegs nk;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          nk.k[st][hf][0] = zero16();
          nk.k[st][hf][1] = zero16();
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) nk.v[st][d] = zero16();
      }
      // Agent-scope loads: the preload above may have brought the (then stale) lines of this
      // slot into this XCD's L2, and another workgroup of the launch has just written it.
      if (r == 0) {
        const uint32_t* kw = reinterpret_cast<const uint32_t*>(kb + g * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          nk.k[0][0][0][e] = __hip_atomic_load(gp(kw + e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          nk.k[0][0][1][e] =
              __hip_atomic_load(gp(kw + 16 + e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (g == 0) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          nk.v[0][d][0] = static_cast<uint32_t>(__hip_atomic_load(
              gp(vb + (d * 16 + r) * kDecBlock), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      }
      attendBlock(st8, nk, qf, pos, L, g, a.scale_log2);
    }
    mark(0);
    if (stage != nullptr) __syncthreads();  // staged blocks are consumed before s reuses LDS
    mark(1);

    const float l_col = rowsSum(st8.l);
    if (g == 0) {
      s.sm[wave][r] = st8.m;
      s.sl[wave][r] = l_col;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) s.so[wave][d * 16 + 4 * g + e][r] = st8.o[d][e];
    __syncthreads();
    // The merger in one polling round where the loop below would take several (more than
    // kMergeChunk other splits, at most kOneRoundSplits) and the unit's (head, d) items leave
    // its last wave free: that wave polls the splits' (m, l) words into LDS while each item
    // thread polls its O[d] words, so the merge waits one round trip after the last partial
    // lands rather than one per chunk. The arithmetic and the split order are the loop's.
    // (With one chunk the loop is faster: no barrier between the polls and the combine.)
    // kOneRound compiles this path in: the 16-row stack kernel (small batches, up to 9 splits
    // per pair); the others keep the code they had, which measured faster at batch 32.
    if (kOneRound && tagged && split == merger && merger > kMergeChunk &&
        merger <= kOneRoundSplits && group * kDecD <= kDecThreads - kWave) {
      const int t = freshThreadIdx();
      const int hl = t / kDecD, d = t % kDecD;
      const bool item = t < group * kDecD;
      float M = -INFINITY, l = 0.f, acc = 0.f, o[kOneRoundSplits];
      if (t >= kDecThreads - kWave) {
        const int j = t - (kDecThreads - kWave);
        if (j < group * merger) {
          const int h = j / merger, sp = j % merger;
          const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + h;
          const uint64_t* const slot = a.ws_tag + (row * max_splits + sp) * kTagSlot;
          const uint64_t* const p[2] = {slot + kDecD, slot + kDecD + 1};
          float v[2];
          loadTagged<2>(v, p, 2, a.tag, a.abort_word);
          s.pm[sp][h] = v[0];
          s.pl[sp][h] = v[1];
        }
      } else if (item) {
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, s.sm[w][hl]);
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) {
          const float e = s.sm[w][hl] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s.sm[w][hl] - M);
          l += e * s.sl[w][hl];
          acc += e * s.so[w][d][hl];
        }
        const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + hl;
        const uint64_t* ptr[kOneRoundSplits];
#pragma unroll
        for (int c = 0; c < kOneRoundSplits; ++c)  // dead slots repeat split 0
          ptr[c] = a.ws_tag + (row * max_splits + (c < merger ? c : 0)) * kTagSlot + d;
        loadTagged<kOneRoundSplits>(o, ptr, kOneRoundSplits, a.tag, a.abort_word);
      }
      __syncthreads();
      if (item) {
        float Mt = -INFINITY, lt = 0.f, at = 0.f;
#pragma unroll
        for (int c = 0; c < kOneRoundSplits; ++c)
          if (c < merger) combineSplit(Mt, lt, at, s.pm[c][hl], s.pl[c][hl], o[c]);
        combineSplit(Mt, lt, at, M, l, acc);
        Mem::storeU16(attnOut(a, b, kvh * group + hl, d), floatToBf16(at / lt));
      }
      return true;
    }
    for (int idx = freshThreadIdx(); idx < group * kDecD; idx += kDecThreads) {
      const int hl = idx / kDecD, d = idx % kDecD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, s.sm[w][hl]);
      float l = 0.f, acc = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float e = s.sm[w][hl] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s.sm[w][hl] - M);
        l += e * s.sl[w][hl];
        acc += e * s.so[w][d][hl];
      }
      const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + hl;
      if (max_splits == 1) {
        Mem::storeU16(attnOut(a, b, row - static_cast<int64_t>(b) * a.Hq, d), floatToBf16(acc / l));
        continue;
      }
      if (tagged) {
        if (split != merger) {
          uint64_t* const mine = a.ws_tag + (row * max_splits + split) * kTagSlot;
          storeTagged(mine + d, acc, a.tag);
          if (d == 0) {
            storeTagged(mine + kDecD, M, a.tag);
            storeTagged(mine + kDecD + 1, l, a.tag);
          }
          continue;
        }
        // the merger (last active split): splits 0.. in order as their words arrive, then its
        // own partial
        float Mt = -INFINITY, lt = 0.f, at = 0.f;
        constexpr int kChunk = kMergeChunk;
        for (int s0 = 0; s0 < merger; s0 += kChunk) {
          const uint64_t* ptr[3 * kChunk];
          const int live = merger - s0 < kChunk ? merger - s0 : kChunk;
#pragma unroll
          for (int c = 0; c < kChunk; ++c) {
            const uint64_t* slot =
                a.ws_tag + (row * max_splits + s0 + (c < live ? c : 0)) * kTagSlot;
            ptr[c] = slot + kDecD;
            ptr[kChunk + c] = slot + kDecD + 1;
            ptr[2 * kChunk + c] = slot + d;
          }
          float v[3 * kChunk];
          // the words of the first `live` splits of each kind: ptr is laid out kind-major, so
          // every index below 3 * kChunk is loaded (dead chunk slots repeat a live split)
          loadTagged<3 * kChunk>(v, ptr, 3 * kChunk, a.tag, a.abort_word);
#pragma unroll
          for (int c = 0; c < kChunk; ++c)
            if (c < live) combineSplit(Mt, lt, at, v[c], v[kChunk + c], v[2 * kChunk + c]);
        }
        combineSplit(Mt, lt, at, M, l, acc);
        Mem::storeU16(attnOut(a, b, row - static_cast<int64_t>(b) * a.Hq, d), floatToBf16(at / lt));
        continue;
      }
      const int64_t slot = row * max_splits + split;
      if (d == 0) {
        __hip_atomic_store(gp(a.ws_ml) + slot * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gp(a.ws_ml) + slot * 2 + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(gp(a.ws_o) + slot * kDecD + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (max_splits == 1) return true;
  if (tagged) return split == merger;

  // Arrive: every partial store of this workgroup has completed before the counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(gp(a.counters) + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s.is_last = old + 1 == arrivals;
    if (s.is_last && reset)
      __hip_atomic_store(gp(a.counters) + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  mark(2);
  if (!s.is_last) return false;

  // Merge the splits that hold keys (the rest wrote nothing this call), in split order. The
  // loads of a chunk of kCombineChunk splits are all issued before any is used, so their
  // memory round trips overlap.
  constexpr int kCombineChunk = 8;
  const int n = n_active;
  for (int idx = freshThreadIdx(); idx < group * kDecD; idx += kDecThreads) {
    const int hl = idx / kDecD, d = idx % kDecD;
    const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * group + hl;
    float M = -INFINITY, l = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < n; s0 += kCombineChunk) {
      float ms[kCombineChunk], ls[kCombineChunk], os[kCombineChunk];
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        const bool live = s0 + c < n;
        const int64_t slot = row * max_splits + (live ? s0 + c : 0);
        ms[c] = live ? __hip_atomic_load(gp(a.ws_ml) + slot * 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : -INFINITY;
        ls[c] = live ? __hip_atomic_load(gp(a.ws_ml) + slot * 2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
        os[c] = live ? __hip_atomic_load(gp(a.ws_o) + slot * kDecD + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0.f;
      }
#pragma unroll
      for (int c = 0; c < kCombineChunk; ++c) {
        if (s0 + c >= n) break;
        combineSplit(M, l, acc, ms[c], ls[c], os[c]);
      }
    }
    Mem::storeU16(attnOut(a, b, row - static_cast<int64_t>(b) * a.Hq, d), n > 0 ? floatToBf16(acc / l) : uint16_t{0});  // no keys: zeros
  }
  return true;
}

}  // namespace dk
