// Entry points of the persistent decoder-stack kernel (csrc/kernels/stack.hip). Declared in
// include/dli_hip.h.
#include <cstdlib>
#include <cstring>
#include <string>

#include "../kernels/stack_args.h"
#include "runtime.h"

static_assert(dli_stack::kTraceEvents == DLI_STACK_TRACE_EVENTS, "trace layout of include/dli_hip.h");

namespace dli::hip {
namespace {

constexpr int kStackThreads = 512;
constexpr int64_t kMaxHidden = 1024;  // x of a norm-prologue tile stays in registers
constexpr int kDecWaves = 8;
constexpr int kMaxStackSplits = 8;    // split-K partials summed by the last arriver
constexpr int kMemcpyDeviceToHost = 2;
constexpr int kMemcpyHostToDevice = 1;

DeviceKernel k_stack_m1("stack", "decoder_stack_m1");
DeviceKernel k_stack_m2("stack", "decoder_stack_m2");
DeviceKernel k_stack_m4("stack", "decoder_stack_m4");

int bad(const std::string& what) {
  return fail(DLI_HIP_EINVAL, "decoder_stack: " + what);
}

size_t alignUp(size_t v, size_t a) { return (v + a - 1) / a * a; }

int tileRows(int64_t m) { return m <= 16 ? 16 : (m <= 32 ? 32 : 64); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Workspace regions, each 256-byte aligned: arrival counters, attention partials, down_proj
// partials, x0 (the launch input in fragment order), then one activation slab per layer of a
// launch (q, attn, h_mid, act, h; bf16 elements, offsets relative to the slab). attn, h_mid, act and h are in MFMA fragment order
// with rows padded to the kernel's tile (tileRows).
struct StackLayout {
  size_t sync, attn_tag, down_tag, x0, slabs, total;
  int64_t slab_elems, off_attn, off_h_mid, off_act, off_h;
};

StackLayout layoutFor(int64_t m, int64_t hidden, int64_t q_heads, int64_t kv_heads,
                      int64_t head_dim, int64_t ffn, int attn_splits, int down_splits,
                      int num_layers) {
  const int64_t down_tiles = hidden / 16, rows = m * q_heads;
  StackLayout l{};
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t here = at;
    at += alignUp(bytes, 256);
    return here;
  };
  l.sync = take(static_cast<size_t>(dli_stack::syncWords()) * sizeof(unsigned));
  // tagged words (8 bytes): attention partials O, m, l per (row, split); down_proj partial tiles
  l.attn_tag = take(static_cast<size_t>(rows) * attn_splits * (head_dim + 2) * sizeof(uint64_t));
  l.down_tag =
      take(static_cast<size_t>(down_tiles) * down_splits * 16 * tileRows(m) * sizeof(uint64_t));
  const int64_t mp = tileRows(m);  // fragment-order activations hold whole 16-row blocks
  l.x0 = take(static_cast<size_t>(mp * hidden) * 2);  // x_in in fragment order
  int64_t e = 0;  // slab elements, each part 256-byte aligned (128 bf16)
  auto part = [&](int64_t elems) {
    const int64_t here = e;
    e += (elems + 127) / 128 * 128;
    return here;
  };
  part(rows * head_dim * 2);  // q at 0: [rows, head_dim / 2] tagged 8-byte words
  l.off_attn = part(mp * q_heads * head_dim);
  l.off_h_mid = part(mp * hidden);
  l.off_act = part(mp * ffn);
  l.off_h = part(mp * hidden);
  l.slab_elems = e;
  const int per_launch = num_layers < dli_stack::kMaxLayers ? num_layers : dli_stack::kMaxLayers;
  l.slabs = take(static_cast<size_t>(e) * 2 * static_cast<size_t>(per_launch));
  l.total = at;
  return l;
}

// One workgroup per CU (every workgroup resident at once); DLI_STACK_GRID=<n> lowers it.
int stackGrid(unsigned* grid) {
  int cus = 0;
  if (int rc = computeUnits(&cus)) return rc;
  static const int forced = [] {
    const char* v = std::getenv("DLI_STACK_GRID");
    return v ? std::atoi(v) : 0;
  }();
  *grid = static_cast<unsigned>(forced > 0 && forced < cus ? forced : cus);
  return 0;
}

// Attention units go to the workgroups that do no q|k|v work (dli_stack::qkvWorkgroups, the
// last ones of the grid), so splits ~ (grid - those) / pairs, unless the caller requests a count.
int attnSplits(int64_t pairs, int64_t max_blocks, int64_t q_tiles, int64_t kv_tiles,
               int requested, int* splits) {
  unsigned grid = 0;
  if (int rc = stackGrid(&grid)) return rc;
  const int64_t qkv_wgs = dli_stack::qkvWorkgroups(static_cast<int>(q_tiles),
                                                   static_cast<int>(kv_tiles),
                                                   static_cast<int>(grid));
  const int64_t free_wgs = static_cast<int64_t>(grid) > qkv_wgs ? grid - qkv_wgs : grid;
  *splits = decodeAttentionSplits(pairs, max_blocks, static_cast<int>(free_wgs), kDecWaves,
                                  requested);
  return 0;
}

}  // namespace
}  // namespace dli::hip

using namespace dli::hip;

extern "C" {

size_t dli_hip_decoder_stack_workspace(int num_layers, int64_t batch, int64_t hidden_size,
                                       int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                       int64_t ffn, int64_t max_blocks, int down_splits,
                                       int attention_splits) {
  if (num_layers <= 0 || batch <= 0 || hidden_size <= 0 || q_heads <= 0 || kv_heads <= 0 ||
      head_dim <= 0 || ffn <= 0 || max_blocks <= 0 || down_splits < 1 || attention_splits < 0 ||
      attention_splits > kMaxDecodeSplits)
    return 0;
  int splits = 0;
  if (attnSplits(batch * kv_heads, max_blocks, q_heads * head_dim / 16,
                 2 * kv_heads * head_dim / 16, attention_splits, &splits) != 0)
    return 0;
  return layoutFor(batch, hidden_size, q_heads, kv_heads, head_dim, ffn, splits, down_splits,
                   num_layers)
      .total;
}

int dli_hip_decoder_stack(const DliDecoderLayer* layers, int num_layers, const void* hidden_in,
                          void* hidden_out, const void* positions, int positions_dtype,
                          const float* cos_table, const float* sin_table, int64_t max_pos,
                          int64_t block_size, int64_t max_blocks, int64_t batch,
                          int64_t hidden_size, int64_t q_heads, int64_t kv_heads,
                          int64_t head_dim, int64_t ffn, float eps, int down_splits,
                          void* workspace, size_t workspace_bytes, unsigned* status,
                          const DliStackOptions* options, void* stream) {
  if (layers == nullptr || num_layers < 0) return bad("layers is NULL");
  if (num_layers == 0) return 0;
  const DliStackOptions opt = options != nullptr ? *options : DliStackOptions{};
  if (opt.attention_splits < 0 || opt.attention_splits > kMaxDecodeSplits)
    return bad("attention_splits must be in [0, 32]");
  if (opt.trace != nullptr && opt.trace_layers <= 0)
    return bad("trace_layers must be positive with a trace buffer");
  if (batch <= 0 || batch > 64) return bad("batch must be in [1, 64]");
  if (hidden_size <= 0 || hidden_size % 64 != 0 || hidden_size > kMaxHidden)
    return bad("hidden_size must be a multiple of 64 in [64, 1024]");
  if (head_dim != 64) return bad("head_dim must be 64");
  if (block_size != 64) return bad("block_size must be 64");
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || q_heads / kv_heads > 16)
    return bad("q_heads must be a multiple of kv_heads, at most 16 per kv head");
  if ((q_heads * head_dim) % 64 != 0) return bad("q_heads * head_dim must be a multiple of 64");
  if (ffn <= 0 || ffn % 64 != 0) return bad("ffn must be a positive multiple of 64");
  if (down_splits < 1 || down_splits > kMaxStackSplits || down_splits > ffn / 64)
    return bad("down_splits must be in [1, min(8, ffn / 64)]");
  if (positions == nullptr || (positions_dtype != DLI_I64 && positions_dtype != DLI_I32))
    return bad("positions (int64/int32 [batch]) are required");
  if (cos_table == nullptr || sin_table == nullptr || max_pos <= 0)
    return bad("rotary tables are required");
  if (max_blocks <= 0) return bad("empty cache geometry");
  const bool from_ids = opt.token_ids != nullptr;
  if (from_ids) {
    if (opt.token_ids_dtype != DLI_I64 && opt.token_ids_dtype != DLI_I32)
      return bad("token_ids must be int64 or int32");
    if (opt.embedding == nullptr || !aligned16(opt.embedding) || opt.vocab <= 0)
      return bad("token_ids need a 16-byte aligned embedding table and vocab > 0");
  } else if (hidden_in == nullptr || !aligned16(hidden_in)) {
    return bad("hidden_in is NULL or not 16-byte aligned");
  }
  if (hidden_out == nullptr || !aligned16(hidden_out))
    return bad("hidden_out is NULL or not 16-byte aligned");
  for (int i = 0; i < num_layers; ++i) {
    const DliDecoderLayer& L = layers[i];
    if (L.input_norm == nullptr || L.w_qkv == nullptr || L.w_o == nullptr ||
        L.post_norm == nullptr || L.w_gate_up == nullptr || L.w_down == nullptr ||
        L.key_pool == nullptr || L.value_pool == nullptr || L.block_table == nullptr)
      return bad("layer " + std::to_string(i) + " has a NULL pointer");
    if (!aligned16(L.input_norm) || !aligned16(L.w_qkv) || !aligned16(L.w_o) ||
        !aligned16(L.post_norm) || !aligned16(L.w_gate_up) || !aligned16(L.w_down))
      return bad("layer " + std::to_string(i) + " weights must be 16-byte aligned");
  }
  int splits = 0;
  if (int rc = attnSplits(batch * kv_heads, max_blocks, q_heads * head_dim / 16,
                          2 * kv_heads * head_dim / 16, opt.attention_splits, &splits))
    return rc;
  if (max_blocks > static_cast<int64_t>(splits) * kDecWaves * 64)
    return bad("max_blocks exceeds what the attention splits can index");
  const StackLayout lay = layoutFor(batch, hidden_size, q_heads, kv_heads, head_dim, ffn, splits,
                                   down_splits, num_layers);
  if (workspace == nullptr || workspace_bytes < lay.total) return bad("workspace too small");
  unsigned grid = 0;
  if (int rc = stackGrid(&grid)) return rc;
  if ((q_heads + 2 * kv_heads) * head_dim / 16 > 2 * static_cast<int64_t>(grid))
    return bad("more than two q|k|v tiles per workgroup");
  DeviceKernel* kernel = batch <= 16 ? &k_stack_m1 : (batch <= 32 ? &k_stack_m2 : &k_stack_m4);

  char* ws = static_cast<char*>(workspace);
  dli_stack::Args a;
  std::memset(&a, 0, sizeof(a));
  a.h_out = static_cast<uint16_t*>(hidden_out);
  a.slabs = reinterpret_cast<uint16_t*>(ws + lay.slabs);
  a.x0 = reinterpret_cast<uint16_t*>(ws + lay.x0);
  a.slab_elems = lay.slab_elems;
  a.off_attn = lay.off_attn;
  a.off_h_mid = lay.off_h_mid;
  a.off_act = lay.off_act;
  a.off_h = lay.off_h;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.positions = positions;
  a.attn_tag = reinterpret_cast<uint64_t*>(ws + lay.attn_tag);
  a.down_tag = reinterpret_cast<uint64_t*>(ws + lay.down_tag);
  a.sync = reinterpret_cast<unsigned*>(ws + lay.sync);
  a.status = status;
  a.max_pos = max_pos;
  a.block_size = block_size;
  a.max_blocks = max_blocks;
  a.M = static_cast<int>(batch);
  a.H = static_cast<int>(hidden_size);
  a.Hq = static_cast<int>(q_heads);
  a.Hkv = static_cast<int>(kv_heads);
  a.D = static_cast<int>(head_dim);
  a.F = static_cast<int>(ffn);
  a.pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  a.attn_splits = splits;
  a.down_splits = down_splits;
  a.eps = eps;
  a.scale_log2 = static_cast<float>(1.4426950408889634 / 8.0);  // log2(e) / sqrt(64)
  a.trace = opt.trace;
  a.trace_layers = opt.trace != nullptr ? opt.trace_layers : 0;
  // Layers run in launches of at most kMaxLayers; later launches continue from hidden_out.
  for (int first = 0; first < num_layers; first += dli_stack::kMaxLayers) {
    const int count = num_layers - first < dli_stack::kMaxLayers ? num_layers - first
                                                                  : dli_stack::kMaxLayers;
    a.layers = count;
    a.trace_base = first;
    a.x_in = static_cast<const uint16_t*>(first == 0 ? hidden_in : hidden_out);
    // the first launch gathers the embedding rows of token_ids; later ones continue from h_out
    a.token_ids = first == 0 && from_ids ? opt.token_ids : nullptr;
    a.ids64 = opt.token_ids_dtype == DLI_I64 ? 1 : 0;
    a.embed = static_cast<const uint16_t*>(opt.embedding);
    a.vocab = opt.vocab;
    for (int i = 0; i < dli_stack::kMaxLayers; ++i) {
      dli_stack::Layer& d = a.layer[i];
      if (i >= count) {
        d = dli_stack::Layer{};
        continue;
      }
      const DliDecoderLayer& L = layers[first + i];
      d.input_norm = static_cast<const uint16_t*>(L.input_norm);
      d.w_qkv = static_cast<const uint16_t*>(L.w_qkv);
      d.b_qkv = static_cast<const uint16_t*>(L.b_qkv);
      d.w_o = static_cast<const uint16_t*>(L.w_o);
      d.post_norm = static_cast<const uint16_t*>(L.post_norm);
      d.w_gate_up = static_cast<const uint16_t*>(L.w_gate_up);
      d.w_down = static_cast<const uint16_t*>(L.w_down);
      d.k_pool = static_cast<uint16_t*>(L.key_pool);
      d.v_pool = static_cast<uint16_t*>(L.value_pool);
      d.block_table = L.block_table;
    }
    if (int rc = launchResident(*kernel, {grid}, {kStackThreads}, 0, stream, a)) return rc;
  }
  return 0;
}

int dli_hip_decoder_stack_status(void* workspace, int* aborted, void* stream) {
  if (workspace == nullptr || aborted == nullptr) return bad("workspace and aborted are required");
  if (int rc = dli_hip_stream_synchronize(stream)) return rc;
  unsigned* word = static_cast<unsigned*>(workspace) + dli_stack::kAbortWord;
  unsigned value = 0;
  if (int rc = dli_hip_memcpy(&value, word, sizeof(value), kMemcpyDeviceToHost)) return rc;
  *aborted = value != 0 ? 1 : 0;
  if (value != 0) {
    const unsigned zero = 0;
    if (int rc = dli_hip_memcpy(word, &zero, sizeof(zero), kMemcpyHostToDevice)) return rc;
  }
  return 0;
}

}  // extern "C"
