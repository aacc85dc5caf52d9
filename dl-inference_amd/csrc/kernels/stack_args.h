#pragma once

// Kernel argument block of the persistent decoder-stack kernel (stack.hip), shared by the HIP
// kernel and the host launcher (csrc/hip/stack_ops.cc) so both see one layout. Plain C types
// only: it is passed by value as the kernel's single argument.
#include <stdint.h>

namespace dli_stack {

constexpr int kMaxLayers = 32;  // layers per launch (more are run as several launches)

// Device pointers of one decoder layer (bf16 unless noted).
struct Layer {
  const uint16_t* input_norm;  // [H]
  const uint16_t* w_qkv;       // [(Hq + 2 Hkv) D, H]  rows q | k | v
  const uint16_t* b_qkv;       // [(Hq + 2 Hkv) D] or NULL
  const uint16_t* w_o;         // [H, Hq D]
  const uint16_t* post_norm;   // [H]
  const uint16_t* w_gate_up;   // [2 F, H]  16-row blocks: gate 16i.., then up 16i..
  const uint16_t* w_down;      // [H, F]
  uint16_t* k_pool;            // [blocks, Hkv, block_size, D]
  uint16_t* v_pool;            // [blocks, Hkv, D, block_size]
  const int32_t* block_table;  // int32 [M, max_blocks]
};

struct Args {
  Layer layer[kMaxLayers];
  const uint16_t* x_in;  // [M, H] residual stream entering the first layer
  // When non-NULL, the first layer's input rows are instead rows token_ids[m] of embed
  // ([vocab, H]; a zero row for an id outside [0, vocab)), gathered by the prologue; x_in is
  // then not read.
  const void* token_ids;  // [M] int32/int64 (ids64)
  const uint16_t* embed;
  int64_t vocab;
  int ids64;
  uint16_t* h_out;       // [M, H] residual stream after the last layer
  uint16_t* x0;          // x_in in fragment order (written by the launch's prologue)
  // Activations of layer l live in their own slab at slabs + l * slab_elems (never reused within
  // a launch): q as [M, Hq, D / 2] tagged 8-byte words (bf16 pair, tag) at offset 0; in MFMA
  // fragment order (fragOffset in
  // skinny.h, rows padded to the tile's 16 MB) attn [M, Hq D] at off_attn, h_mid [M, H]
  // (residual stream after attention) at off_h_mid, act [M, F] at off_act and h [M, H] (after
  // the layer) at off_h; the last layer writes h_out (row-major) instead, and the first reads
  // x0, the prologue's fragment-order copy of x_in (or of the embedding rows).
  uint16_t* slabs;
  int64_t slab_elems, off_attn, off_h_mid, off_act, off_h;
  const float* cos_t;  // [max_pos, D / 2]
  const float* sin_t;
  const void* positions;  // [M] int32/int64: slot of each row's new token
  uint64_t* attn_tag;     // attention unit partials, tagged words [M Hq][splits][O, m, l]
  uint64_t* down_tag;     // down_proj split partial tiles, tagged words [tiles][splits][tile]
  unsigned* sync;         // arrival counters (zero before the first launch; left at zero)
  // Launch status, or NULL. When set, the last workgroup out ORs the abort word into *status
  // (non-zero: a wait of this launch gave up, its outputs are invalid) and clears the abort word,
  // so the next launch starts clean; the caller reads and zeroes *status. When NULL the abort word
  // stays set for dli_hip_decoder_stack_status.
  unsigned* status;
  // Stage timeline, or NULL: stamp (s_memrealtime, 100 MHz) of event e of workgroup w in layer
  // trace_base + l at trace[((trace_base + l) * grid + w) * kTraceEvents + e] while
  // trace_base + l < trace_layers.
  unsigned long long* trace;
  int trace_base, trace_layers;
  int64_t max_pos, block_size, max_blocks;
  int layers, M, H, Hq, Hkv, D, F, pos64, attn_splits, down_splits;
  float eps, scale_log2;
};

// Events of the stage timeline (Args::trace), per layer and workgroup; 0 = not reached.
enum : int {
  kTrLayerStart = 0,  // the workgroup enters the layer
  kTrQkvWait,         // S1: the previous layer's h is complete
  kTrQPublished,      // S1: this workgroup's q tile is published
  kTrKvPublished,     // S1: this workgroup's k/v tiles are in the cache
  kTrAttnWait,        // S2: every wave has q (tagged words polled by wave 0)
  kTrAttnUnit,        // S2: the unit's partial (or output) is written
  kTrAttnMerged,      // S2: this workgroup merged a pair and published it
  kTrOWait,           // S3: attention complete
  kTrODone,           // S3: o_proj tile published
  kTrGuWait,          // S4: h_mid complete
  kTrGuDone,          // S4: gate_up tiles published
  kTrDownWait,        // S5: act complete
  kTrDownDone,        // S5: down_proj unit done (tile published if it merged)
  kTrStagedNext,      // early staging of the next layer's cache blocks issued
  kTrAttnWave0,       // S2: wave 0 has attended its cache blocks
  kTrAttnWaves,       // S2: every wave has attended its cache blocks
  kTrAttnArrived,     // S2: the unit's partial is stored and counted
  kTrAttnBlock1,      // S2: wave 0 has attended its first cache block
  kTrAttnBlock2,      // S2: wave 0 has attended its second cache block
  kTrQkvNorm,         // S1: x loaded and normalized
  kTrQkvReduced,      // S1: first tile reduced
  kTrGuNorm,          // S4: h_mid loaded and normalized
  kTrGuReduced,       // S4: first tile reduced
  kTrDownReduced,     // S5: tile (or split partial) reduced
  kTrQkvX,            // S1: x (and every load issued before it) arrived
  kTrGuX,             // S4: h_mid arrived
  kTrOX,              // S3: the attention rows arrived
  kTrDownX,           // S5: act arrived
  kTrQkvPoll,         // S1: the first poll of the wait returned
  kTrOPoll,           // S3: the first poll of the wait returned
  kTrGuPoll,          // S4: the first poll of the wait returned
  kTrDownPoll,        // S5: the first poll of the wait returned
  kTraceEvents = 32
};

// Layout of `sync` in 32-bit words. A stage counter is split into kShards sub-counters, each on
// its own 256-byte line: a workgroup adds to sub-counter blockIdx.x % kShards, so arrivals do
// not all serialize on one address, and a waiting workgroup sums the shards. Then the exit
// counter, the abort word and the launch epoch (own lines). The epoch, read by every workgroup
// at the start and advanced by the last one out, goes into the tags of the tagged partials, so
// a word left by an earlier launch or layer never carries the tag a reader expects.
enum : int {
  kKvDone = 0,   // every k/v tile written into the cache (q travels as tagged words)
  kAttnDone,     // attention output of every pair written
  kODone,        // every o_proj tile (h_mid) written
  kGateUpDone,   // every gate_up tile (act) written
  kDownDone,     // every down_proj tile (h) written
  kStages
};
constexpr int kShards = 64;
static_assert(kShards <= 64 && (kShards & (kShards - 1)) == 0, "one lane per shard");
constexpr int kLineWords = 64;
constexpr int stageWord(int stage) { return stage * kShards * kLineWords; }
constexpr int kExitWord = kStages * kShards * kLineWords;
constexpr int kAbortWord = kExitWord + kLineWords;
constexpr int kEpochWord = kAbortWord + kLineWords;

// Tag of the tagged partials of layer l (l < 256) in the launch of `epoch`; never 0, the value
// of a zero-filled workspace.
constexpr unsigned partialTag(unsigned epoch, int l) {
  return ((epoch & 0xFFFFFFu) << 8) | static_cast<unsigned>(l + 1);
}

// Workgroups of the q|k|v stage (the last ones of the grid): one per q tile plus one per two k/v
// tiles when the grid has room for that and at least as many others, else two tiles of any kind
// per workgroup. The host sizes the attention split count from what this leaves free.
constexpr int qkvWorkgroups(int q_tiles, int kv_tiles, int grid) {
  return 2 * (q_tiles + (kv_tiles + 1) / 2) <= grid ? q_tiles + (kv_tiles + 1) / 2
                                                    : (q_tiles + kv_tiles + 1) / 2;
}

inline int64_t syncWords() { return kEpochWord + 1; }

}  // namespace dli_stack
