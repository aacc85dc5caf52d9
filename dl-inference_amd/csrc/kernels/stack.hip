// Persistent decoder stack for batched decode on gfx950: every decoder layer of a Qwen2-style
// model in ONE launch. The reference runs a decoder layer as 19 graph nodes
// (python/dli_export/export.py:272-446); the five-launch fused path (decode.hip, attention.hip)
// runs it as five kernels. Here one 8-wave workgroup per CU walks the layers and, per layer,
// five stages:
//
//   S1 qkv     RMSNorm(h) W_qkv^T + b, RoPE, k/v into the paged cache, q     (16-row tiles)
//   S2 attn    decode attention units (pair = (sequence, kv head), split)    (decode_attention.h)
//   S3 o       h_mid = h + attn W_o^T                                         (16-row tiles)
//   S4 gate_up act = bf16(silu(gate)) * up of RMSNorm(h_mid)                  (32-row tiles)
//   S5 down    h = h_mid + act W_down^T, split-K, split 0 merges             (16-row tiles)
//
// Every tile is computed with the same code and order as the one-stage kernels, so the stack
// and the five-launch path give bit-identical results.
//
// Synchronisation. A stage's consumers wait on an arrival counter instead of a kernel boundary:
// each producing workgroup stores its outputs with agent-scope stores (written through to the
// coherent memory side; the L2 caches of the 8 XCDs are not coherent with each other), waits
// for them (s_waitcnt vmcnt(0)) and adds to its shard of the stage counter; a consumer polls the
// shards until they sum to (layer + 1) x the producers of that stage. Consumers then read with
// plain loads, so each XCD's L2 serves the repeated reads of an activation row (q, read by few
// units per row, is the exception: see Work placement). That is correct
// because every layer has its own activation buffers (slabs): no line a consumer reads can have
// been read, and cached stale, earlier in the launch. Before waiting, a workgroup requests the
// weights of its next tile (attention units: their first cache blocks), which do not depend on
// the previous stage, so that stream overlaps the wait.
//
// Work placement. q|k|v tiles go to the last qkv_wgs workgroups of the grid (one per q tile,
// two k/v tiles per workgroup), which have no down_proj unit and reach the stage first;
// attention units go to the other workgroups; o_proj tiles to the q|k|v workgroups (idle
// through attention, so they request the o_proj weights meanwhile); gate_up tiles bid,
// bid + a_wgs, ... to the a_wgs other workgroups; down_proj units to the first ones. q and the
// new k/v are signalled apart: attention needs q at once, and q goes out as tagged words
// (common.h) that wave 0 of each attention unit polls directly and hands to the other waves
// through LDS, with no store acknowledgement and no counter between the q|k|v tile and the
// unit; the new k/v is needed only for the block holding the newest token and has its own
// counter. A wave with a third cache block stages it in LDS
// (direct global-to-LDS loads) next to the two it requests into registers, so nothing streams
// after the wait; waves 0..kEarly-1 stage it during the previous layer, right after their
// attention unit, so that part of the K/V stream overlaps o_proj, gate_up and down_proj, when
// the memory system is otherwise lightly loaded.
//
// Progress. The grid is at most one workgroup per CU and a workgroup fits a CU on its own, so
// every workgroup is resident at once, and a stage only waits on earlier stages, which every
// workgroup passes in the same order. Every wait is still bounded: after kSpinLimit polls the
// workgroup raises the abort word, every later wait returns at once, and the launch ends with
// the abort word set for the host to read (the outputs are then invalid).
//
// The counters only grow during a launch; the last workgroup to finish resets them all to zero
// (and, when the launch reports into a status word, moves the abort word there), so the next
// launch starts from zero without a memset.
#include "decode_attention.h"
#include "decode_parts.h"
#include "stack_args.h"

using namespace dk;
using dli_stack::Args;
using dli_stack::Layer;

namespace {

constexpr int kStackThreads = 512;
constexpr int kSpinLimit = 1 << 20;
constexpr int kAbortPollEvery = 64;

__device__ __forceinline__ unsigned loadAgent(const unsigned* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Adds n to this workgroup's shard of a stage counter once every thread's stores have
// completed.
__device__ __forceinline__ void arrive(unsigned* stage, unsigned n) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(gp(stage) + (blockIdx.x % dli_stack::kShards) * dli_stack::kLineWords, n,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of v over the 64 lanes of a full wave, in a scalar: DPP adds within each 16-lane row
// (quad swaps, then the half-row and row mirrors), then the four row sums. Every lane must be
// active.
template <int kCtrl>
__device__ __forceinline__ unsigned dppMove(unsigned x) {
  return static_cast<unsigned>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ unsigned waveSum(unsigned v) {
  v += dppMove<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dppMove<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dppMove<0x141>(v);  // row_half_mirror
  v += dppMove<0x140>(v);  // row_mirror
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// Polls a stage counter from one wave (lane i < kShards loads shard i with an agent-scope
// vector load) until the shards sum to at least target, the abort word is set, or kSpinLimit
// polls have passed (which sets the abort word). The loop condition is uniform over the wave.
// first (tracing, or NULL): receives the time the first poll returned (the wave's loads complete
// in issue order, so that is also when the loads it issued before the wait had arrived).
// The shards are summed with waveSum (DPP, a few cycles; cross-lane shuffles took six
// LDS-crossbar round trips, ~0.3 us per poll).
__device__ __forceinline__ void pollStage(const unsigned* stage, unsigned target,
                                          unsigned* abort_word,
                                          unsigned long long* first = nullptr) {
  const int lane = freshThreadIdx() % kWave;
  for (int spins = 0;; ++spins) {
    unsigned v = lane < dli_stack::kShards ? loadAgent(stage + lane * dli_stack::kLineWords) : 0u;
    v = waveSum(v);
    if (first != nullptr && spins == 0 && lane == 0) *first = __builtin_amdgcn_s_memrealtime();
    if (__builtin_amdgcn_readfirstlane(v) >= target) break;
    if (spins % kAbortPollEvery == 0 &&
        __builtin_amdgcn_readfirstlane(loadAgent(abort_word)) != 0u)
      break;
    if (spins >= kSpinLimit) {
      __hip_atomic_store(gp(abort_word), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Returns in every thread of the workgroup once the stage counter reaches target (wave 0 polls).
__device__ __forceinline__ void waitAtLeast(const unsigned* stage, unsigned target,
                                            unsigned* abort_word,
                                            unsigned long long* first = nullptr) {
  if (threadIdx.x < kWave) pollStage(stage, target, abort_word, first);
  __syncthreads();
}

// Stage timeline (Args::trace). Thread 0 keeps the stamps of the current layer in LDS (a
// global store would count against the wave's vmcnt and delay a later s_waitcnt) and writes
// them out when the workgroup enters the next layer and at the end: flushStamps.
__device__ __forceinline__ void stamp(const Args& a, int l, int e, unsigned long long* lds) {
  if (a.trace == nullptr || a.trace_base + l >= a.trace_layers) return;
  if (threadIdx.x == 0) lds[e] = __builtin_amdgcn_s_memrealtime();
}

// Stamps event e once every wave's outstanding loads have arrived (only while tracing: the
// stage waits for them soon after anyway, but the wait and barrier stay off the untraced path).
__device__ __forceinline__ void stampLoaded(const Args& a, int l, int e, unsigned long long* lds) {
  if (a.trace == nullptr || a.trace_base + l >= a.trace_layers) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // every wave's loads
  if (threadIdx.x == 0) lds[e] = __builtin_amdgcn_s_memrealtime();
}

// The LDS stamp slot of event e while tracing layer l, else NULL.
__device__ __forceinline__ unsigned long long* traceSlot(const Args& a, int l, int e,
                                                         unsigned long long* lds) {
  return a.trace == nullptr || a.trace_base + l >= a.trace_layers ? nullptr : lds + e;
}

__device__ __forceinline__ void flushStamps(const Args& a, int l, unsigned long long* lds) {
  unsigned long long* const t = a.trace;
  if (t == nullptr || a.trace_base + l >= a.trace_layers) return;
  if (threadIdx.x == 0) {
    unsigned long long* const row =
        t + (static_cast<int64_t>(a.trace_base + l) * gridDim.x + blockIdx.x) *
                dli_stack::kTraceEvents;
    for (int e = 0; e < dli_stack::kTraceEvents; ++e) {
      row[e] = lds[e];
      lds[e] = 0;
    }
  }
}

// Returns v unchanged through an empty asm statement, so the compiler cannot hoist what is
// computed from it out of the layer loop: per-stage addresses are then recomputed in each
// stage instead of being held in registers (or spilled) across all five stages.
template <typename T>
__device__ __forceinline__ T fresh(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

// LDS of a workgroup. Waves 0..kEarly-1 of an attention workgroup stage the third cache block
// of their next-layer unit in kv_early while o_proj, gate_up and down_proj run (those use only
// the union beside it); the rest of the stages use the union one at a time (each ends with a
// barrier): the tile reductions and RMSNorm row sums, the attention merge, and the last wave's
// staged block, which kv[kDecWaves - 1] overlays. The q|k|v stage parks its epilogue operands
// (two tiles' worth) in the union after its own tile reduction and row sums (qkvPark).
template <int MB>
struct StackLds {
  using GuCore = SkinnyCore<2, MB, kNormWaves, kNormUnroll>;
  using QkvCore = SkinnyCore<1, MB, kNormWaves, kNormUnroll>;
  using Epi = QkvEpilogue<MB, WriteThroughMem, true>;
  static constexpr int kQkvParkFloat = QkvCore::kLdsFloats + kNormLdsFloats<MB, kNormWaves>;
  union Shared {
    // the largest stage tile reduction (gate_up), then the RMSNorm row sums
    float gemm[GuCore::kLdsFloats + kNormLdsFloats<MB, kNormWaves>];
    DecodeAttnLds attn;
  };
  static_assert(kQkvParkFloat % 2 == 0 &&
                    kQkvParkFloat * sizeof(float) + 2 * Epi::kPairs * sizeof(QkvParked) <=
                        sizeof(Shared),
                "the q|k|v epilogue operands fit the union after the stage's own use");
  // as many early slots as fit in 160 KB beside the union (7 up to 32 rows, 5 at 64)
  static constexpr int kEarlyFit =
      static_cast<int>((163840 - 512 - sizeof(Shared)) / sizeof(KvBlockLds));
  static constexpr int kEarly = kEarlyFit < kDecWaves - 1 ? kEarlyFit : kDecWaves - 1;
  union {
    KvBlockLds kv[kDecWaves];
    struct {
      KvBlockLds kv_early[kEarly];
      Shared u;
    } p;
  };
  int is_last;
  unsigned long long trace[dli_stack::kTraceEvents];  // stamps of the current layer

  __device__ __forceinline__ QkvParked* qkvPark() {
    return reinterpret_cast<QkvParked*>(p.u.gemm + kQkvParkFloat);
  }
};

// Layout of the stack's activation slabs: MFMA fragment order (fragOffset) for the 32- and
// 64-row kernels, where every fragment load is one contiguous 1 KB read; row-major for the
// 16-row kernel, whose loads of rows past M fold onto row M - 1 (a batch of 1 would otherwise
// read 16 rows per fragment).
template <bool kFrag>
struct ActX;
template <>
struct ActX<true> {
  __device__ __forceinline__ static XFrag make(const uint16_t* p, int ld) {
    return XFrag{p, ld / 64};
  }
  __device__ __forceinline__ static int steps(int ld) { return ld / 64; }
};
template <>
struct ActX<false> {
  __device__ __forceinline__ static XGlobal make(const uint16_t* p, int ld) {
    return XGlobal{p, ld};
  }
  __device__ __forceinline__ static int steps(int) { return 0; }
};

template <int MB>
__device__ void decoderStack(const Args& a) {
  using AX = ActX<(MB >= 2)>;
  using OCore = SkinnyCore<1, MB, kResWaves, (MB >= 4 ? 2 : 4)>;
  // down_proj splits: wave 0 (the poller of the act wait) takes no K step (kDownIdle)
  using DownCore = SkinnyCore<1, MB, kResWaves, 2, kDownIdle>;
  using Mem = WriteThroughMem;
  constexpr int kTileElems = 16 * 16 * MB;
  static_assert(SkinnyCore<1, MB, kNormWaves, kNormUnroll>::kLdsFloats <=
                    StackLds<MB>::GuCore::kLdsFloats,
                "lds");
  static_assert(OCore::kLdsFloats <= StackLds<MB>::GuCore::kLdsFloats, "lds");
  __shared__ StackLds<MB> smem;
  float* lds = smem.p.u.gemm;

  const int G = gridDim.x, bid = blockIdx.x;
  const int qkv_tiles = (a.Hq + 2 * a.Hkv) * a.D / 16, o_tiles = a.H / 16;
  const int gu_tiles = a.F / 16, down_tiles = a.H / 16;
  const int pairs = a.M * a.Hkv, splits = a.attn_splits, down_splits = a.down_splits;
  const int attn_units = pairs * splits, down_units = down_tiles * down_splits;
  const int q_tiles = a.Hq * a.D / 16, kv_tiles = qkv_tiles - q_tiles;
  const int qkv_wgs = dli_stack::qkvWorkgroups(q_tiles, kv_tiles, G);  // S1 workgroups
  const int jb = bid - (G - qkv_wgs);  // index among the q|k|v workgroups, < 0 for the others
  // o_proj tile of this workgroup (then every G-th): jb on the q|k|v workgroups if they cover
  // the tiles, else bid
  const int o_first = o_tiles <= qkv_wgs ? (jb >= 0 ? jb : o_tiles) : bid;
  const bool has_o = o_first < o_tiles;

  if (threadIdx.x == 0)
    for (int e = 0; e < dli_stack::kTraceEvents; ++e) smem.trace[e] = 0;
  // launch epoch (advanced only by the last workgroup out, after every workgroup has read it)
  const unsigned epoch = __builtin_amdgcn_readfirstlane(loadAgent(a.sync + dli_stack::kEpochWord));
  // Prologue: x_in (row-major), or the embedding rows of token_ids (embedding/kernel.py:6-23:
  // a zero row for an id out of range), into x0 in fragment order, one 16-column tile per
  // workgroup like a down_proj tile, counted on kDownDone as the output of "layer -1" (so every
  // layer's q|k|v waits for (l + 1) x down_tiles arrivals and reads its x in fragment order).
  for (int t = bid; t < down_tiles; t += G) {
    const int m = threadIdx.x / 2;  // thread item: 8 columns of one row
    const int64_t n = static_cast<int64_t>(t) * 16 + 8 * (threadIdx.x % 2);
    if (m < a.M) {  // the host checks 16-byte alignment and H % 64 == 0
      U128 v;
      if (a.token_ids != nullptr) {
        const int64_t id = a.ids64 ? static_cast<const int64_t*>(a.token_ids)[m]
                                   : static_cast<const int32_t*>(a.token_ids)[m];
        v = id >= 0 && id < a.vocab ? gload16(a.embed + id * a.H + n) : zero16();
      } else {
        v = gload16(a.x_in + m * a.H + n);
      }
      Mem::store16(a.x0 + actOffset(m, n, a.H, AX::steps(a.H)), v);
    }
    arrive(a.sync + dli_stack::stageWord(dli_stack::kDownDone), 1);
  }
  for (int l = 0; l < a.layers; ++l) {
    if (l > 0) flushStamps(a, l - 1, smem.trace);
    const Layer& L = a.layer[l];
    const unsigned gen = static_cast<unsigned>(l + 1);
    const unsigned tag = dli_stack::partialTag(epoch, l);
    // This layer's activation slab and the residual stream entering it. Every pointer and size
    // below passes through fresh() so that no address is computed once for all layers.
    uint16_t* const slab = fresh(a.slabs) + l * fresh(a.slab_elems);
    uint16_t* const q = slab;
    uint16_t* const attn = slab + a.off_attn;
    uint16_t* const h_mid = slab + a.off_h_mid;
    uint16_t* const act = slab + a.off_act;
    uint16_t* const h = l == a.layers - 1 ? fresh(a.h_out) : slab + a.off_h;
    const uint16_t* const h_prev =
        l == 0 ? fresh(a.x0) : static_cast<const uint16_t*>(slab - a.slab_elems + a.off_h);
    unsigned* const sync = fresh(a.sync);
    unsigned* const abort_word = sync + dli_stack::kAbortWord;
    stamp(a, l, dli_stack::kTrLayerStart, smem.trace);

    // S1: q|k|v tiles of the residual stream the previous layer finished, on the last qkv_wgs
    // workgroups (the ones without down_proj work, which reach this stage first). q tiles come
    // one per workgroup and k/v tiles two per workgroup when the grid has room (qkvWorkgroups),
    // so q, which attention needs first, is ready after one tile.
    if (jb >= 0) {
      const int H = fresh(a.H), M = fresh(a.M);
      // built where used (prefetch, then each tile's epilogue) from fresh copies, so that none
      // of it is held, or spilled, across the tile's GEMM
      auto qkvParams = [&] {
        const Layer& Lf = a.layer[l];
        uint16_t* const qs = fresh(a.slabs) + l * fresh(a.slab_elems);
        return QkvParams{fresh(Lf.b_qkv),
                         fresh(a.cos_t),
                         fresh(a.sin_t),
                         fresh(a.max_pos),
                         fresh(a.positions),
                         fresh(a.pos64),
                         qs,
                         KvCacheArgs{fresh(Lf.k_pool), fresh(Lf.v_pool), fresh(Lf.block_table),
                                     fresh(a.block_size), fresh(a.max_blocks)},
                         fresh(a.M),
                         fresh(a.Hq),
                         fresh(a.Hkv),
                         fresh(a.D),
                         reinterpret_cast<uint64_t*>(qs),
                         fresh(tag)};
      };
      const int j = jb;
      // this workgroup's tiles: t0, then t0 + t_stride while below t_end
      int t0, t_stride, t_end;
      if (qkv_wgs == q_tiles + (kv_tiles + 1) / 2) {
        const bool q_wg = j < q_tiles;
        t0 = q_wg ? j : q_tiles + 2 * (j - q_tiles);
        t_stride = 1;
        t_end = q_wg ? j + 1 : (t0 + 2 < qkv_tiles ? t0 + 2 : qkv_tiles);
      } else {
        t0 = j;
        t_stride = qkv_wgs;
        t_end = qkv_tiles;
      }
      // operands of this workgroup's (at most) two tiles, parked in LDS
      using Epi = QkvEpilogue<MB, Mem, true>;
      Epi epi0, epi1;
      epi0.park = smem.qkvPark();
      epi1.park = epi0.park + Epi::kPairs;
      epi0.prefetch(qkvParams(), static_cast<int64_t>(t0) * 16);
      if (t0 + t_stride < t_end)
        epi1.prefetch(qkvParams(), static_cast<int64_t>(t0 + t_stride) * 16);
      unsigned kv_written = 0;
      auto finish = [&](int64_t t) {
        Epi e;  // the operands parked for tile t
        e.park = smem.qkvPark() + (t == t0 ? 0 : Epi::kPairs);
        if (t < q_tiles) {  // q: tagged words, which attention polls directly
          e.template apply<kQkvQ>(qkvParams(), t * 16, lds);
          stamp(a, l, dli_stack::kTrQPublished, smem.trace);
        } else {  // k/v into the cache: attention needs it only for the newest-token block
          e.template apply<kQkvCache>(qkvParams(), t * 16, lds);
          ++kv_written;
        }
      };
      tileLoop<1, MB, kNormWaves, kNormUnroll, Mem, true>(
          L.w_qkv, AX::make(h_prev, H), qkv_tiles * 16, H, M, lds, L.input_norm, a.eps, t0,
          t_stride, t_end,
          [&] {
            // h of the previous layer (for the first layer: the prologue's copy of x_in)
            waitAtLeast(sync + dli_stack::stageWord(dli_stack::kDownDone), gen * down_tiles,
                        abort_word, traceSlot(a, l, dli_stack::kTrQkvPoll, smem.trace));
            stamp(a, l, dli_stack::kTrQkvWait, smem.trace);
          },
          [&](int64_t t) { finish(t); },
          [&](int p) {
            if (p == 2)
              stampLoaded(a, l, dli_stack::kTrQkvX, smem.trace);
            else
              stamp(a, l, dli_stack::kTrQkvNorm + p, smem.trace);
          });
      if (kv_written > 0) {
        arrive(sync + dli_stack::stageWord(dli_stack::kKvDone), kv_written);
        stamp(a, l, dli_stack::kTrKvPublished, smem.trace);
      }
    }

    // S2: attention units. A workgroup with one unit per layer stages the third cache blocks of
    // its next-layer unit (waves 0..kEarly-1) after this one, or after its o_proj tile if it
    // has one, so that part of the K/V stream runs under o_proj, gate_up and down_proj.
    const bool early = attn_units <= G && bid < attn_units && !has_o;
    auto stageNext = [&] {
      const Layer& N = a.layer[l + 1];
      const DecodeAttnArgs dn{q,
                              N.k_pool,
                              N.v_pool,
                              N.block_table,
                              fresh(a.positions),
                              a.pos64,
                              0,
                              nullptr,
                              nullptr,
                              nullptr,
                              nullptr,
                              a.Hq,
                              a.Hkv,
                              a.max_blocks,
                              splits,
                              a.scale_log2};
      stageThirdKvBlocks(dn, bid % splits, bid / splits, smem.kv, StackLds<MB>::kEarly);
    };
    if (bid < attn_units) {
      // split partials as tagged words: the last active split merges them as they arrive, no
      // pair counter
      const DecodeAttnArgs da{q,
                              L.k_pool,
                              L.v_pool,
                              L.block_table,
                              fresh(a.positions),
                              a.pos64,
                              0,
                              nullptr,
                              nullptr,
                              nullptr,
                              attn,
                              a.Hq,
                              a.Hkv,
                              a.max_blocks,
                              splits,
                              a.scale_log2,
                              fresh(a.attn_tag),
                              tag,
                              abort_word,
                              AX::steps(a.Hq * a.D),
                              reinterpret_cast<const uint64_t*>(q)};
      for (int u = bid; u < attn_units; u += G) {
        const bool merged = decodeAttentionUnit<Mem, true, MB == 1>(
            da, u % splits, u / splits, gen * splits, false, smem.p.u.attn, smem.kv,
            early && l > 0 ? StackLds<MB>::kEarly : 0,
            [] {},  // q is polled as tagged words
            [&] {
              pollStage(sync + dli_stack::stageWord(dli_stack::kKvDone), gen * kv_tiles,
                        abort_word);
            },
            [&](int point) {
              stamp(a, l, point == 5 ? dli_stack::kTrAttnWait : dli_stack::kTrAttnWave0 + point,
                    smem.trace);
            });
        stamp(a, l, dli_stack::kTrAttnUnit, smem.trace);
        if (merged) {
          arrive(sync + dli_stack::stageWord(dli_stack::kAttnDone), 1);
          stamp(a, l, dli_stack::kTrAttnMerged, smem.trace);
        }
      }
      if (early && l + 1 < a.layers) {
        stageNext();
        stamp(a, l, dli_stack::kTrStagedNext, smem.trace);
      }
    }

    // S3: o_proj + attention residual, on the q|k|v workgroups when they are enough (idle
    // through attention, so they request the o_proj weights meanwhile).
    for (int t = o_first; t < o_tiles; t += G) {
      const int H = fresh(a.H), M = fresh(a.M), qd = fresh(a.Hq * a.D);
      const int64_t n0 = static_cast<int64_t>(t) * 16;
      ResidualTile<MB, kResThreads, Mem> rt;
      OCore::template runGated<Mem>(
          L.w_o, AX::make(attn, qd), H, qd, M, n0, 0, qd / 64, lds,
          [&] {
            waitAtLeast(sync + dli_stack::stageWord(dli_stack::kAttnDone), gen * pairs,
                        abort_word, traceSlot(a, l, dli_stack::kTrOPoll, smem.trace));
            stamp(a, l, dli_stack::kTrOWait, smem.trace);
            rt.load(h_prev, nullptr, n0, M, H, AX::steps(H));
          },
          [&](int p) {
            if (p == 1) stampLoaded(a, l, dli_stack::kTrOX, smem.trace);
          });
      rt.store(h_mid, n0, M, H, [&](int e) { return lds[e]; }, AX::steps(H));
      arrive(sync + dli_stack::stageWord(dli_stack::kODone), 1);
      stamp(a, l, dli_stack::kTrODone, smem.trace);
    }

    // S4: gate_up + SwiGLU, RMSNorm of h_mid in registers. When o_proj ran on the q|k|v
    // workgroups, tiles bid, bid + a_wgs, ... on each of the other a_wgs workgroups (which
    // request their weights while o_proj runs). Otherwise tile bid on each workgroup without
    // q|k|v work and the tiles beyond those in contiguous runs on the q|k|v workgroups, which
    // are idle through attention and o_proj and request their tiles' weights meanwhile.
    const int a_wgs = G - qkv_wgs;
    int gu_first = bid, gu_stride = 1, gu_end = bid + 1;
    if (o_tiles <= qkv_wgs && a_wgs > 0) {
      gu_stride = a_wgs;
      gu_end = jb < 0 ? gu_tiles : 0;
    } else if (jb >= 0) {
      const int rest = gu_tiles > a_wgs ? gu_tiles - a_wgs : 0;
      const int per = (rest + qkv_wgs - 1) / qkv_wgs;
      gu_first = a_wgs + jb * per;
      gu_end = gu_first + per;
    }
    if (gu_end > gu_tiles) gu_end = gu_tiles;
    if (gu_first < gu_end) {
      const int H = fresh(a.H), M = fresh(a.M), F = fresh(a.F);
      tileLoop<2, MB, kNormWaves, kNormUnroll, Mem, true, (MB >= 2)>(
          L.w_gate_up, AX::make(h_mid, H), 2 * static_cast<int64_t>(F), H, M, lds,
          L.post_norm,
          a.eps, gu_first, gu_stride, gu_end,
          [&] {
            waitAtLeast(sync + dli_stack::stageWord(dli_stack::kODone), gen * o_tiles,
                        abort_word, traceSlot(a, l, dli_stack::kTrGuPoll, smem.trace));
            stamp(a, l, dli_stack::kTrGuWait, smem.trace);
          },
          [&](int64_t t) { gateUpEpilogue<MB, Mem, (MB >= 2)>(lds, act, M, F, t, AX::steps(F)); },
          [&](int p) {
            if (p == 2)
              stampLoaded(a, l, dli_stack::kTrGuX, smem.trace);
            else
              stamp(a, l, dli_stack::kTrGuNorm + p, smem.trace);
          });
      arrive(sync + dli_stack::stageWord(dli_stack::kGateUpDone),
             static_cast<unsigned>((gu_end - gu_first + gu_stride - 1) / gu_stride));
      stamp(a, l, dli_stack::kTrGuDone, smem.trace);
    }

    // S5: down_proj + MLP residual. With one split a tile is reduced over the full K; with
    // several, split 0 of a tile adds the other splits' tagged partials as they arrive and
    // writes h.
    // Unit of workgroup w < down_units: with the units a multiple of the 8 XCDs (workgroups
    // are dealt to them round-robin, w on XCD w % 8), unit (w % 8) * (down_units / 8) + w / 8,
    // so that each XCD holds the units of one or two splits and its L2 fetches those splits'
    // share of act rather than all of it.
    const bool xcd_order = down_units % 8 == 0 && down_units <= G;
    for (int w = bid; w < down_units; w += G) {
      const int u = xcd_order ? (w % 8) * (down_units / 8) + w / 8 : w;
      const int H = fresh(a.H), M = fresh(a.M), F = fresh(a.F);
      const int tile = u % down_tiles, split = u / down_tiles;
      const int64_t n0 = static_cast<int64_t>(tile) * 16;
      ResidualTile<MB, kResThreads, Mem> rt;
      auto gate = [&] {
        waitAtLeast(sync + dli_stack::stageWord(dli_stack::kGateUpDone), gen * gu_tiles,
                    abort_word, traceSlot(a, l, dli_stack::kTrDownPoll, smem.trace));
        stamp(a, l, dli_stack::kTrDownWait, smem.trace);
        rt.load(h_mid, nullptr, n0, M, H, AX::steps(H));
      };
      const int h_frag = l == a.layers - 1 ? 0 : AX::steps(H);  // the last layer writes h_out
      if (down_splits == 1) {
        OCore::template runGated<Mem>(L.w_down, AX::make(act, F), H, F, M, n0, 0, F / 64,
                                      lds,
                                      gate, [&](int p) {
                                        if (p == 1)
                                          stampLoaded(a, l, dli_stack::kTrDownX, smem.trace);
                                        else
                                          stamp(a, l, dli_stack::kTrDownReduced, smem.trace);
                                      });
        rt.store(h, n0, M, H, [&](int e) { return lds[e]; }, h_frag);
        arrive(sync + dli_stack::stageWord(dli_stack::kDownDone), 1);
        stamp(a, l, dli_stack::kTrDownDone, smem.trace);
        continue;
      }
      int sb, se;
      splitRange(F / 64, split, down_splits, sb, se);
      DownCore::template runGated<Mem>(
          L.w_down, AX::make(act, F), H, F, M, n0, sb, se, lds, gate, [&](int p) {
            if (p == 1)
              stampLoaded(a, l, dli_stack::kTrDownX, smem.trace);
            else
              stamp(a, l, dli_stack::kTrDownReduced, smem.trace);
          });
      if (splitKTagged<MB, kResThreads, Mem>(
              lds, fresh(a.down_tag) + static_cast<int64_t>(tile) * down_splits * kTileElems,
              split, down_splits, tag, abort_word, rt, h, n0, M, H, h_frag))
        arrive(sync + dli_stack::stageWord(dli_stack::kDownDone), 1);
      stamp(a, l, dli_stack::kTrDownDone, smem.trace);
    }
  }

  flushStamps(a, a.layers - 1, smem.trace);

  // Leave: the last workgroup out resets every counter but the abort word and advances the
  // epoch.
  unsigned* const sync = a.sync;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(gp(sync) + dli_stack::kExitWord, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    smem.is_last = old + 1 == static_cast<unsigned>(G);
  }
  __syncthreads();
  if (!smem.is_last) return;
  for (int i = threadIdx.x; i < dli_stack::kStages * dli_stack::kShards; i += kStackThreads)
    __hip_atomic_store(gp(sync) + i * dli_stack::kLineWords, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) {
    if (a.status != nullptr) {
      // every other workgroup arrived after its last wait, so a give-up is visible here
      const unsigned aborted = loadAgent(sync + dli_stack::kAbortWord);
      if (aborted != 0u) {
        __hip_atomic_fetch_or(gp(a.status), aborted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gp(sync) + dli_stack::kAbortWord, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __hip_atomic_store(gp(sync) + dli_stack::kExitWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gp(sync) + dli_stack::kEpochWord, epoch + 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

#define DK_STACK_KERNEL(MB)                                                                \
  extern "C" __global__ void __launch_bounds__(kStackThreads, 1)                           \
      decoder_stack_m##MB(const Args a) {                                                  \
    decoderStack<MB>(a);                                                                   \
  }

DK_STACK_KERNEL(1)
DK_STACK_KERNEL(2)
DK_STACK_KERNEL(4)
