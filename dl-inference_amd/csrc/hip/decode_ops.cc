// Entry points of the fused decode kernels (csrc/kernels/decode.hip) and the MFMA decode
// attention (csrc/kernels/attention.hip). Declared in include/dli_hip.h.
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <string>

#include "../kernels/scratch.h"
#include "runtime.h"

namespace dli::hip {
namespace {

constexpr int kThreads = 256;
constexpr int kNormThreads = 512;    // qkv_rope_append and gate_up_silu workgroups
constexpr int kTileN = 32;           // weight rows per workgroup of gate_up / lm_head (NF = 2)
constexpr int kRowTile = 16;         // weight rows per workgroup of qkv / linear_residual / partial
constexpr int kResWaves = 8;         // waves per linear_residual workgroup
constexpr int64_t kMaxNormN = 1024;  // residual_rms_norm: 256 threads x 4 columns
constexpr int kMaxNormSplits = 8;    // residual_rms_norm sums at most 8 split-K partials
constexpr int64_t kMaxLmK = 1024;    // tile loops keep x for K / 64 <= 16 steps in registers

struct MbKernels {
  DeviceKernel m1, m2, m4;
  MbKernels(const char* module, const char* base)
      : m1(module, make(base, "_m1")), m2(module, make(base, "_m2")), m4(module, make(base, "_m4")) {}
  DeviceKernel* pick(int64_t m) { return m <= 16 ? &m1 : (m <= 32 ? &m2 : (m <= 64 ? &m4 : nullptr)); }

 private:
  static const char* make(const char* base, const char* suffix) {
    return (new std::string(std::string(base) + suffix))->c_str();
  }
};

MbKernels k_qkv("decode", "qkv_rope_append");
MbKernels k_linres("decode", "linear_residual");
MbKernels k_linres_splitk("decode", "linear_residual_splitk");
MbKernels k_partial("decode", "linear_partial");
MbKernels k_gate_up("decode", "gate_up_silu");
MbKernels k_lm_head("decode", "lm_head_argmax");
DeviceKernel k_res_norm("decode", "residual_rms_norm");
DeviceKernel k_argmax_final("decode", "argmax_finalize");
// many-row (prefill) forms of linear_residual and gate_up_silu: tiled MFMA GEMMs with the same
// epilogues (mfma_gemm.hip)
DeviceKernel k_mfma_linres64("mfma_gemm", "mfma_linear_residual_bf16_t64");
DeviceKernel k_mfma_linres128("mfma_gemm", "mfma_linear_residual_bf16_t128");
DeviceKernel k_mfma_gu64("mfma_gemm", "mfma_gate_up_silu_bf16_t64");
DeviceKernel k_mfma_gu128("mfma_gemm", "mfma_gate_up_silu_bf16_t128");
DeviceKernel k_mfma_gu_stream("mfma_gemm", "mfma_gate_up_silu_bf16_stream_t64");
DeviceKernel k_mfma_qkvh64("mfma_gemm", "mfma_qkv_heads_bf16_t64");
DeviceKernel k_mfma_qkvh128("mfma_gemm", "mfma_qkv_heads_bf16_t128");

// Tiled launch of those: 128 x 128 tiles once they alone give every CU a workgroup, else 64 x 64;
// grid (column tiles, row tiles).
bool tiledGrid(int64_t rows, int64_t cols, bool* big, unsigned (&grid)[2]) {
  // 128 x 128 tiles once there are enough of them to fill most of the 256 CUs (measured at
  // 896 columns: 2048 rows / 112 tiles ran faster in 64 x 64 tiles, 4096 rows / 224 tiles in
  // 128 x 128 tiles)
  *big = ((rows + 127) / 128) * ((cols + 127) / 128) >= 168;
  const int64_t tile = *big ? 128 : 64;
  const int64_t gx = (cols + tile - 1) / tile, gy = (rows + tile - 1) / tile;
  if (gy > 65535 || gx > (int64_t{1} << 31)) return false;
  grid[0] = static_cast<unsigned>(gx);
  grid[1] = static_cast<unsigned>(gy);
  return true;
}
DeviceKernel k_dec_attn("attention", "decode_attention_d64");
DeviceKernel k_dec_attn128("attention", "decode_attention_d128");

int bad(const char* op, const std::string& what) {
  return fail(DLI_HIP_EINVAL, std::string(op) + ": " + what);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t alignUp(size_t v, size_t a) { return (v + a - 1) / a * a; }

int tileRows(int64_t m) { return m <= 16 ? 16 : (m <= 32 ? 32 : 64); }

// Split-K partials: [splits, m, n] (linear_residual_norm) or [tiles][splits][16 x tileRows(m)]
// (linear_residual), whichever is larger; arrival counters (one per 16-row tile) follow.
size_t splitPartialBytes(int64_t n, int64_t m, int splits) {
  const int64_t tiles = (n + kRowTile - 1) / kRowTile;
  const int64_t a = static_cast<int64_t>(splits) * m * n;
  const int64_t b = tiles * splits * kRowTile * tileRows(m);
  return alignUp(static_cast<size_t>(a > b ? a : b) * sizeof(float), 256);
}

// Workgroups of a grid-strided tile loop: one per tile, at most as many as are resident at once
// (two 256-thread workgroups per CU fit below 256 VGPRs; the 64-row variants use more). The
// 512-thread RMSNorm-prologue kernels fit one per CU.
int tileGrid(int64_t tiles, int64_t m, unsigned* grid, bool prologue = false) {
  int cus = 0;
  if (int rc = computeUnits(&cus)) return rc;
  const int64_t resident = static_cast<int64_t>(cus) * (m <= 32 && !prologue ? 2 : 1);
  *grid = static_cast<unsigned>(tiles < resident ? tiles : resident);
  return 0;
}

int checkSkinny(const char* op, int64_t m, int64_t k) {
  if (m <= 0 || m > 64) return bad(op, "batch rows must be in [1, 64]");
  if (k <= 0 || k % 64 != 0) return bad(op, "reduction size must be a positive multiple of 64");
  return 0;
}

// Partial GEMM over `splits` K ranges into workspace [splits, m, n] fp32, then the residual
// (+ RMSNorm) kernel. n <= kMaxNormN.
int partialThenResidual(const char* op, const void* x, const void* w, const void* bias,
                        const void* residual, const void* norm_weight, void* h_out, void* xn_out,
                        int64_t m, int64_t n, int64_t k, float eps, int splits, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (n <= 0 || n > kMaxNormN) return bad(op, "n must be in [1, 1024]");
  if (splits < 1 || splits > k / 64 || splits > kMaxNormSplits)
    return bad(op, "splits must be in [1, min(8, k / 64)]");
  if (workspace == nullptr || workspace_bytes < dli_hip_splitk_workspace(n, m, splits))
    return bad(op, "workspace too small");
  if (!aligned16(x) || !aligned16(w)) return bad(op, "x and w must be 16-byte aligned");
  float* partials = static_cast<float*>(workspace);  // [splits, m, n]
  const unsigned tiles = static_cast<unsigned>((n + kRowTile - 1) / kRowTile);
  if (int rc = launch(*k_partial.pick(m), {tiles, static_cast<unsigned>(splits)}, {kThreads}, 0,
                      stream, x, w, partials, static_cast<int>(m), n, static_cast<int>(k), splits))
    return rc;
  return launch(k_res_norm, {static_cast<unsigned>(m)}, {kThreads}, 0, stream,
                static_cast<const float*>(partials), splits, bias, residual, norm_weight, h_out,
                xn_out, static_cast<int>(m), static_cast<int>(n), eps);
}

}  // namespace

// ops.cc: the tiled bf16 GEMM for decode-sized m (K split into a workspace)
bool tiledDecodeLinear(int64_t m, int64_t n);
int64_t bf16Splits(int64_t m, int64_t n, int64_t k);
int tiledBf16(const void* x, const void* w, const void* bias, const void* residual, void* out,
              int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
              void* stream);
int tiledBf16Parts(const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                   void* workspace, size_t workspace_bytes, void* stream, int* parts_out);

namespace {

// Reduces of the large-hidden decode projections (mfma_gemm.hip): they read the fp32 parts
// [parts, m, n] that decodeParts writes.
DeviceKernel k_reduce_qkv("mfma_gemm", "splitk_reduce_qkv_rope_append");
DeviceKernel k_reduce_res_norm2("mfma_gemm", "splitk_reduce_residual_norm_p2");
DeviceKernel k_reduce_res_norm4("mfma_gemm", "splitk_reduce_residual_norm_p4");
DeviceKernel k_reduce_res_norm8("mfma_gemm", "splitk_reduce_residual_norm_p8");
constexpr int64_t kResNormMaxN = 4096;  // splitk_reduce_residual_norm: 256 threads x 2 x 8
constexpr int kResNormMaxSplits = 8;

// Parts of a decode-sized projection whose output is wider than the fused kernels hold: the
// tiled MFMA GEMM where it runs faster (tiledDecodeLinear), else the skinny partial kernel with
// `splits` K ranges (at most 8 and k / 64, fewer if the workspace holds fewer). The parts go to
// workspace [parts, m, n] fp32, summed by the caller's reduce in part order.
int64_t skinnyParts(int64_t k, int64_t splits) {
  int64_t s = splits < 1 ? 1 : splits;
  if (s > kMaxNormSplits) s = kMaxNormSplits;
  if (s > k / 64) s = k / 64 > 0 ? k / 64 : 1;
  return s;
}

// Workspace bytes of decodeParts: every part it would write, at most 8 (what the reduces sum;
// the tiled path halves its split count until the parts fit).
size_t decodePartsBytes(int64_t m, int64_t n, int64_t k, int64_t splits) {
  int64_t parts = tiledDecodeLinear(m, n) ? bf16Splits(m, n, k) : skinnyParts(k, splits);
  if (parts > kResNormMaxSplits) parts = kResNormMaxSplits;
  return static_cast<size_t>(parts * m * n) * sizeof(float);
}

int decodeParts(const char* op, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                int64_t splits, void* workspace, size_t workspace_bytes, void* stream,
                int* parts_out) {
  if (!aligned16(x) || !aligned16(w)) return bad(op, "x and w must be 16-byte aligned");
  if (tiledDecodeLinear(m, n)) {
    if (k <= 0 || k % 8 != 0) return bad(op, "reduction size must be a positive multiple of 8");
    return tiledBf16Parts(x, w, m, n, k, workspace, workspace_bytes, stream, parts_out);
  }
  if (int rc = checkSkinny(op, m, k)) return rc;
  int64_t parts = skinnyParts(k, splits);
  const size_t part = static_cast<size_t>(m * n) * sizeof(float);
  while (parts > 1 && workspace_bytes < part * parts) --parts;
  if (workspace == nullptr || workspace_bytes < part) return bad(op, "workspace too small");
  *parts_out = static_cast<int>(parts);
  const unsigned tiles = static_cast<unsigned>((n + kRowTile - 1) / kRowTile);
  return launch(*k_partial.pick(m), {tiles, static_cast<unsigned>(parts)}, {kThreads}, 0, stream,
                x, w, static_cast<float*>(workspace), static_cast<int>(m), n, static_cast<int>(k),
                static_cast<int>(parts));
}

// q|k|v parts for the skinny path: enough K ranges for about two workgroups per CU.
int64_t qkvSkinnySplits(int64_t n, int64_t k) {
  const int64_t tiles = (n + kRowTile - 1) / kRowTile;
  return skinnyParts(k, (512 + tiles - 1) / tiles);
}

}  // namespace
}  // namespace dli::hip

using namespace dli::hip;

extern "C" {

size_t dli_hip_splitk_workspace(int64_t n, int64_t m, int splits) {
  if (n <= 0 || m <= 0 || splits < 1) return 0;
  return splitPartialBytes(n, m, splits) +
         alignUp(static_cast<size_t>((n + kRowTile - 1) / kRowTile) * sizeof(unsigned), 256);
}

int dli_hip_qkv_rope_append(const void* hidden, const void* norm_weight, const void* w_qkv,
                            const void* b_qkv, const float* cos_table, const float* sin_table,
                            int64_t max_pos, const void* positions, int positions_dtype,
                            void* q_out, void* key_pool, void* value_pool,
                            const int32_t* block_table, int64_t block_size, int64_t max_blocks,
                            int64_t batch, int64_t hidden_size, int64_t q_heads, int64_t kv_heads,
                            int64_t head_dim, float eps, void* stream) {
  const char* op = "qkv_rope_append";
  if (int rc = checkSkinny(op, batch, hidden_size)) return rc;
  if (hidden_size > kMaxLmK) return bad(op, "hidden_size above 1024 is not supported");
  if (positions == nullptr || (positions_dtype != DLI_I64 && positions_dtype != DLI_I32))
    return bad(op, "positions (int64/int32 [batch]) are required");
  if (head_dim <= 0 || head_dim % 2 != 0) return bad(op, "head_dim must be even");
  if (kv_heads <= 0 || q_heads <= 0) return bad(op, "head counts must be positive");
  if ((q_heads * head_dim) % kRowTile != 0 || (kv_heads * head_dim) % kRowTile != 0)
    return bad(op, "q and kv widths must be multiples of 16");
  if (block_size <= 0 || max_blocks <= 0) return bad(op, "empty cache geometry");
  if (!aligned16(hidden) || !aligned16(w_qkv) || (norm_weight != nullptr && !aligned16(norm_weight)))
    return bad(op, "hidden, norm_weight and w_qkv must be 16-byte aligned");
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  const int64_t tiles = (n + kRowTile - 1) / kRowTile;
  if (tiles > 65535) return bad(op, "too many q|k|v rows");
  const int pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  // one tile per workgroup: the kernel prefetches the epilogue operands of tile blockIdx.x
  return launch(*k_qkv.pick(batch), {static_cast<unsigned>(tiles)}, {kNormThreads}, 0, stream,
                hidden,
                norm_weight, eps, w_qkv, b_qkv, cos_table, sin_table, max_pos, positions, pos64,
                q_out, key_pool, value_pool, block_table, block_size, max_blocks,
                static_cast<int>(batch), static_cast<int>(hidden_size),
                static_cast<int>(q_heads), static_cast<int>(kv_heads),
                static_cast<int>(head_dim));
}

size_t dli_hip_qkv_rope_append_workspace(int64_t batch, int64_t hidden_size, int64_t q_heads,
                                         int64_t kv_heads, int64_t head_dim) {
  if (batch <= 0 || batch > 64 || hidden_size <= kMaxLmK || q_heads <= 0 || kv_heads <= 0 ||
      head_dim <= 0)
    return 0;
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  return decodePartsBytes(batch, n, hidden_size, qkvSkinnySplits(n, hidden_size));
}

int dli_hip_qkv_rope_append_ws(const void* hidden, const void* norm_weight, const void* w_qkv,
                               const void* b_qkv, const float* cos_table, const float* sin_table,
                               int64_t max_pos, const void* positions, int positions_dtype,
                               void* q_out, void* key_pool, void* value_pool,
                               const int32_t* block_table, int64_t block_size,
                               int64_t max_blocks, int64_t batch, int64_t hidden_size,
                               int64_t q_heads, int64_t kv_heads, int64_t head_dim, float eps,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (hidden_size <= kMaxLmK)
    return dli_hip_qkv_rope_append(hidden, norm_weight, w_qkv, b_qkv, cos_table, sin_table,
                                   max_pos, positions, positions_dtype, q_out, key_pool,
                                   value_pool, block_table, block_size, max_blocks, batch,
                                   hidden_size, q_heads, kv_heads, head_dim, eps, stream);
  // a hidden size the fused kernel does not hold in registers: GEMM parts, then one reduce that
  // adds the bias, rotates q and k and writes q and the cache
  const char* op = "qkv_rope_append";
  if (batch <= 0 || batch > 64) return bad(op, "batch rows must be in [1, 64]");
  if (norm_weight != nullptr)
    return bad(op, "the RMSNorm prologue needs hidden_size <= 1024 (normalize first)");
  if (positions == nullptr || (positions_dtype != DLI_I64 && positions_dtype != DLI_I32))
    return bad(op, "positions (int64/int32 [batch]) are required");
  if (head_dim <= 0 || head_dim % 2 != 0) return bad(op, "head_dim must be even");
  if (kv_heads <= 0 || q_heads <= 0 || q_heads > 4096 || kv_heads > 4096)
    return bad(op, "head counts must be in [1, 4096]");
  if (block_size <= 0 || max_blocks <= 0) return bad(op, "empty cache geometry");
  if (max_pos < 0) return bad(op, "negative max_pos");
  if (w_qkv == nullptr || cos_table == nullptr || sin_table == nullptr || q_out == nullptr ||
      key_pool == nullptr || value_pool == nullptr || block_table == nullptr)
    return bad(op, "NULL pointer");
  if (!aligned16(q_out) || !aligned16(key_pool) || !aligned16(value_pool))
    return bad(op, "q_out and the cache pools must be 16-byte aligned");
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  const size_t need = dli_hip_qkv_rope_append_workspace(batch, hidden_size, q_heads, kv_heads,
                                                        head_dim);
  if (workspace == nullptr || workspace_bytes < need) return bad(op, "workspace too small");
  int parts = 0;
  if (int rc = decodeParts(op, hidden, w_qkv, batch, n, hidden_size,
                           qkvSkinnySplits(n, hidden_size), workspace, need, stream, &parts))
    return rc;
  const int64_t pairs = batch * n / 2;
  const int64_t blocks = (pairs + 255) / 256;
  return launch(k_reduce_qkv, {static_cast<unsigned>(blocks < 4096 ? blocks : 4096)}, {256}, 0,
                stream, static_cast<const float*>(workspace), parts, b_qkv, cos_table, sin_table,
                max_pos, positions, positions_dtype == DLI_I64 ? 1 : 0, q_out, key_pool,
                value_pool, block_table, block_size, max_blocks, static_cast<int>(batch),
                static_cast<int>(q_heads), static_cast<int>(kv_heads),
                static_cast<int>(head_dim));
}

int dli_hip_linear_residual(const void* x, const void* w, const void* bias, const void* residual,
                            void* out, int64_t m, int64_t n, int64_t k, int splits,
                            void* workspace, size_t workspace_bytes, void* stream) {
  const char* op = "linear_residual";
  // outputs wider than the fused decode kernels hold (n > 1024, a large hidden size) with more
  // than 8 rows: the tiled GEMM, K split into the workspace as far as it holds (the splits
  // argument sizes the workspace only)
  if (m > 8 && m <= 64 && n > 1024 && k % 8 == 0 && aligned16(x) && aligned16(w) &&
      tiledDecodeLinear(m, n)) {
    if (splits < 1) return bad(op, "splits must be positive");
    return tiledBf16(x, w, bias, residual, out, m, n, k, workspace, workspace_bytes, stream);
  }
  if (m > 64) {  // many rows (a prompt): one tiled MFMA GEMM, no split
    if (n <= 0) return bad(op, "n must be positive");
    if (k <= 0 || k % 8 != 0) return bad(op, "k must be a positive multiple of 8");
    if (!aligned16(x) || !aligned16(w)) return bad(op, "x and w must be 16-byte aligned");
    bool big = false;
    unsigned grid[2];
    if (!tiledGrid(m, n, &big, grid)) return bad(op, "too many rows");
    return launch(big ? k_mfma_linres128 : k_mfma_linres64, {grid[0], grid[1]}, {256}, 0,
                  stream, x, w, bias, residual, out, m, n, k);
  }
  if (int rc = checkSkinny(op, m, k)) return rc;
  if (n <= 0) return bad(op, "n must be positive");
  if (splits < 1 || splits > k / 64 || splits > kMaxNormSplits)
    return bad(op, "splits must be in [1, min(8, k / 64)]");
  if (!aligned16(x) || !aligned16(w)) return bad(op, "x and w must be 16-byte aligned");
  const int64_t tiles = (n + kRowTile - 1) / kRowTile;
  if (splits == 1)
    return launch(*k_linres.pick(m), {static_cast<unsigned>(tiles)}, {kResWaves * 64}, 0, stream,
                  x, w, bias, residual, out, static_cast<int>(m), n, static_cast<int>(k));
  if (workspace == nullptr || workspace_bytes < dli_hip_splitk_workspace(n, m, splits))
    return bad(op, "workspace too small");
  float* partials = static_cast<float*>(workspace);
  unsigned* counters = reinterpret_cast<unsigned*>(static_cast<char*>(workspace) +
                                                   splitPartialBytes(n, m, splits));
  return launch(*k_linres_splitk.pick(m),
                {static_cast<unsigned>(tiles), static_cast<unsigned>(splits)}, {kResWaves * 64},
                0, stream, x, w, bias, residual, out, static_cast<int>(m), n,
                static_cast<int>(k), splits, partials, counters);
}

int dli_hip_linear_residual_norm(const void* x, const void* w, const void* bias,
                                 const void* residual, const void* norm_weight, void* h_out,
                                 void* xn_out, int64_t m, int64_t n, int64_t k, float eps,
                                 int splits, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const char* op = "linear_residual_norm";
  if (norm_weight == nullptr || xn_out == nullptr) return bad(op, "norm_weight and xn_out are required");
  if (n > kMaxNormN) {
    // wider than the fused residual kernel holds (a large hidden size): GEMM parts, then one
    // workgroup per row sums them with the residual and normalizes
    if (m <= 0 || m > 64) return bad(op, "batch rows must be in [1, 64]");
    if (n > kResNormMaxN || n % 8 != 0) return bad(op, "n above 1024 must be a multiple of 8, at most 4096");
    if (splits < 1) return bad(op, "splits must be positive");
    if (residual == nullptr || h_out == nullptr) return bad(op, "residual and h_out are required");
    if (!aligned16(residual) || !aligned16(norm_weight) || !aligned16(h_out) ||
        !aligned16(xn_out) || (bias != nullptr && !aligned16(bias)))
      return bad(op, "residual, bias, norm_weight, h_out and xn_out must be 16-byte aligned");
    const size_t need = decodePartsBytes(m, n, k, splits);
    int parts = 0;
    if (int rc = decodeParts(op, x, w, m, n, k, splits, workspace,
                             workspace_bytes < need ? workspace_bytes : need, stream, &parts))
      return rc;
    if (parts > kResNormMaxSplits) return bad(op, "too many K parts");
    DeviceKernel& k = parts <= 2 ? k_reduce_res_norm2 : (parts <= 4 ? k_reduce_res_norm4 : k_reduce_res_norm8);
    return launch(k, {static_cast<unsigned>(m)}, {256}, 0, stream,
                  static_cast<const float*>(workspace), parts, bias, residual, norm_weight, h_out,
                  xn_out, static_cast<int>(m), static_cast<int>(n), eps);
  }
  if (int rc = checkSkinny(op, m, k)) return rc;
  return partialThenResidual(op, x, w, bias, residual, norm_weight, h_out, xn_out, m, n, k, eps,
                             splits, workspace, workspace_bytes, stream);
}

int dli_hip_gate_up_silu(const void* hidden, const void* norm_weight, const void* w_gate_up,
                         void* out, int64_t m, int64_t ffn, int64_t hidden_size, float eps,
                         void* stream) {
  const char* op = "gate_up_silu";
  if (m > 64 || (m > 0 && hidden_size > kMaxLmK && norm_weight == nullptr)) {
    // many rows (a prompt), or a hidden size the skinny kernels do not hold: one tiled MFMA
    // GEMM over the interleaved weight, SwiGLU in its epilogue
    if (ffn <= 0 || ffn % 16 != 0) return bad(op, "ffn must be a positive multiple of 16");
    if (hidden_size <= 0 || hidden_size % 8 != 0)
      return bad(op, "hidden_size must be a positive multiple of 8");
    if (norm_weight != nullptr)
      return bad(op, "the RMSNorm prologue is for at most 64 rows (normalize first)");
    if (!aligned16(hidden) || !aligned16(w_gate_up))
      return bad(op, "hidden and w_gate_up must be 16-byte aligned");
    if (m <= 64)  // decode-sized rows: 64 x 64 tiles, 128-wide K slices
      return launch(k_mfma_gu_stream, {static_cast<unsigned>((2 * ffn + 63) / 64), 1}, {256}, 0,
                    stream, hidden, w_gate_up, out, m, ffn, hidden_size);
    bool big = false;
    unsigned grid[2];
    if (!tiledGrid(m, 2 * ffn, &big, grid)) return bad(op, "too many rows");
    return launch(big ? k_mfma_gu128 : k_mfma_gu64, {grid[0], grid[1]}, {256}, 0, stream, hidden,
                  w_gate_up, out, m, ffn, hidden_size);
  }
  if (int rc = checkSkinny(op, m, hidden_size)) return rc;
  if (ffn <= 0 || ffn % 16 != 0) return bad(op, "ffn must be a positive multiple of 16");
  if (hidden_size > kMaxLmK) return bad(op, "hidden_size above 1024 is not supported");
  if (!aligned16(hidden) || !aligned16(w_gate_up) ||
      (norm_weight != nullptr && !aligned16(norm_weight)))
    return bad(op, "hidden, norm_weight and w_gate_up must be 16-byte aligned");
  unsigned grid = 0;
  if (int rc = tileGrid(ffn / 16, m, &grid, norm_weight != nullptr)) return rc;
  return launch(*k_gate_up.pick(m), {grid}, {kNormThreads}, 0, stream, hidden, norm_weight, eps,
                w_gate_up, out, static_cast<int>(m), ffn, static_cast<int>(hidden_size));
}

int dli_hip_qkv_rope_heads(const void* x, const void* w_qkv, const void* b_qkv, const float* cos,
                           const float* sin, int64_t max_pos, void* q_out, void* k_out,
                           void* v_out, int64_t batch, int64_t seq, int64_t hidden_size,
                           int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t start_pos,
                           void* stream) {
  const char* op = "qkv_rope_heads";
  if (batch < 0 || seq < 0) return bad(op, "negative size");
  const int64_t m = batch * seq;
  if (m == 0) return 0;
  if (hidden_size <= 0 || hidden_size % 8 != 0)
    return bad(op, "hidden_size must be a positive multiple of 8");
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 1024)
    return bad(op, "head_dim must be a multiple of 8 in [8, 1024]");
  if (q_heads <= 0 || kv_heads <= 0 || q_heads > 4096 || kv_heads > 4096)
    return bad(op, "q_heads and kv_heads must be in [1, 4096]");
  if (max_pos < 0) return bad(op, "negative max_pos");
  if (x == nullptr || w_qkv == nullptr || b_qkv == nullptr || cos == nullptr || sin == nullptr ||
      q_out == nullptr || k_out == nullptr || v_out == nullptr)
    return bad(op, "NULL pointer");
  if (!aligned16(x) || !aligned16(w_qkv) || !aligned16(b_qkv) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(q_out) || !aligned16(k_out) || !aligned16(v_out))
    return bad(op, "x, w_qkv, b_qkv, cos, sin and the outputs must be 16-byte aligned");
  const int64_t n = (q_heads + 2 * kv_heads) * head_dim;
  if (m >= (int64_t{1} << 31) || n >= (int64_t{1} << 31))
    return bad(op, "batch * seq and the q|k|v width must be below 2^31");
  bool big = false;
  unsigned grid[2];
  if (!tiledGrid(m, n, &big, grid)) return bad(op, "too many rows");
  return launch(big ? k_mfma_qkvh128 : k_mfma_qkvh64, {grid[0], grid[1]}, {256}, 0, stream, x,
                w_qkv, b_qkv, cos, sin, max_pos, q_out, k_out, v_out, m, hidden_size, seq,
                start_pos, static_cast<int>(q_heads), static_cast<int>(kv_heads),
                static_cast<int>(head_dim));
}

size_t dli_hip_lm_head_argmax_workspace(int64_t m, int64_t vocab) {
  const int64_t tiles = (vocab + kTileN - 1) / kTileN;
  return static_cast<size_t>(tiles) * m * (sizeof(float) + sizeof(int32_t));
}

int dli_hip_lm_head_argmax(const void* xn, const void* w, void* logits, int logits_dtype,
                           int64_t* ids, int64_t m, int64_t vocab, int64_t hidden_size,
                           void* workspace, size_t workspace_bytes, void* stream) {
  return dli_hip_lm_head_argmax_norm(xn, nullptr, 0.f, w, logits, logits_dtype, ids, m, vocab,
                                     hidden_size, workspace, workspace_bytes, stream);
}

int dli_hip_lm_head_argmax_norm(const void* x, const void* norm_weight, float eps, const void* w,
                                void* logits, int logits_dtype, int64_t* ids, int64_t m,
                                int64_t vocab, int64_t hidden_size, void* workspace,
                                size_t workspace_bytes, void* stream) {
  const char* op = "lm_head_argmax";
  const void* xn = x;
  if (norm_weight != nullptr && (hidden_size % 64 != 0 || !aligned16(norm_weight)))
    return bad(op, "norm weight needs hidden_size % 64 == 0 and 16-byte alignment");
  if (int rc = checkSkinny(op, m, hidden_size)) return rc;
  if (hidden_size > kMaxLmK) return bad(op, "hidden_size above 1024 is not supported");
  if (vocab <= 0 || vocab >= (int64_t{1} << 31)) return bad(op, "vocab must be in [1, 2^31)");
  if (logits != nullptr && logits_dtype != DLI_F32 && logits_dtype != DLI_BF16)
    return bad(op, "logits dtype must be float32 or bfloat16");
  if (ids == nullptr) return bad(op, "ids is NULL");
  if (workspace == nullptr || workspace_bytes < dli_hip_lm_head_argmax_workspace(m, vocab))
    return bad(op, "workspace too small");
  if (!aligned16(xn) || !aligned16(w)) return bad(op, "xn and w must be 16-byte aligned");
  const int64_t tiles = (vocab + kTileN - 1) / kTileN;
  unsigned blocks = 0;
  if (int rc = tileGrid(tiles, m, &blocks)) return rc;
  float* part_val = static_cast<float*>(workspace);
  int32_t* part_idx = reinterpret_cast<int32_t*>(part_val + tiles * m);
  const int logits_f32 = logits_dtype == DLI_F32 ? 1 : 0;
  if (int rc = launch(*k_lm_head.pick(m), {blocks}, {kThreads}, 0, stream,
                      xn, w, logits, logits_f32, part_val, part_idx, static_cast<int>(m), vocab,
                      static_cast<int>(hidden_size), norm_weight, eps))
    return rc;
  // one partial per row from each lm_head workgroup (blocks <= tiles: the workspace holds them)
  return launch(k_argmax_final, {static_cast<unsigned>(m)}, {kThreads}, 0, stream,
                static_cast<const float*>(part_val), static_cast<const int32_t*>(part_idx),
                static_cast<int>(blocks), ids);
}

}  // extern "C"

namespace dli::hip {
namespace {

// Device address of the decode module's static `scratch` array on the current device, looked
// up once per device (with that device current) by name on the loaded module, which also loads
// the module and the two lm_head kernels there, so later calls load and allocate nothing. Each
// device holds its own copy at its own address.
int lmHeadScratch(void** out) {
  static std::array<std::atomic<void*>, 64> per_device{};
  static std::mutex mutex;
  int device = 0;
  if (int rc = dli_hip_get_device(&device)) return rc;
  if (device < 0 || device >= 64) return fail(DLI_HIP_EINVAL, "device index out of range");
  void* p = per_device[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(mutex);
    p = per_device[device].load(std::memory_order_relaxed);
    if (p == nullptr) {
      size_t bytes = 0;
      if (int rc = moduleGlobal("decode", "scratch", &p, &bytes)) return rc;
      if (p == nullptr || bytes != dli_scratch::kLmHeadBytes)
        return fail(DLI_HIP_ENODEV, "decode module scratch has an unexpected size");
      void* fn = nullptr;
      for (DeviceKernel* k : {&k_lm_head.m1, &k_lm_head.m2, &k_lm_head.m4, &k_argmax_final})
        if (int rc = k->resolve(&fn)) return rc;
      per_device[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

}  // namespace
}  // namespace dli::hip

extern "C" int dli_hip_lm_head_argmax_norm_noalloc(const void* x, const void* norm_weight,
                                                   float eps, const void* w, void* logits,
                                                   int logits_dtype, int64_t* ids, int64_t m,
                                                   int64_t vocab, int64_t hidden_size,
                                                   void* stream) {
  const char* op = "lm_head_argmax_noalloc";
  if (int rc = checkSkinny(op, m, hidden_size)) return rc;
  if (vocab <= 0 || vocab >= (int64_t{1} << 31)) return bad(op, "vocab must be in [1, 2^31)");
  const size_t need = dli_hip_lm_head_argmax_workspace(m, vocab);
  if (need > dli_scratch::kLmHeadBytes)
    return bad(op, "m = " + std::to_string(m) + " rows over vocab " + std::to_string(vocab) +
                       " need " + std::to_string(need) + " bytes of scratch, above its " +
                       std::to_string(dli_scratch::kLmHeadBytes) + "-byte maximum");
  void* scratch = nullptr;
  if (int rc = lmHeadScratch(&scratch)) return rc;
  // the same kernels as dli_hip_lm_head_argmax_norm, with the static scratch as the workspace
  return dli_hip_lm_head_argmax_norm(x, norm_weight, eps, w, logits, logits_dtype, ids, m, vocab,
                                     hidden_size, scratch, dli_scratch::kLmHeadBytes, stream);
}

namespace dli::hip {

// MFMA decode attention (one query per sequence, bf16, head_dim 64, 64-key cache blocks); used
// by dli_hip_paged_attention when the case fits. Returns 1 when it does not apply.
//
// Splits along the keys: at most one (sequence, kv head, split) workgroup per CU, so the whole
// grid runs in one round (the kernel fits one 8-wave workgroup per CU); the blocks of a
// sequence are dealt round-robin over all waves of its splits. The last split of a (sequence,
// kv head) to finish merges the partials (agent-scope stores and loads plus a per-(sequence,
// kv head) counter in the workspace, which it leaves at zero). A caller's split count
// (`requested` > 0) replaces the per-CU choice.
namespace {
constexpr int kDecWaves = 8;
constexpr int kDecBlock = 64;

// Workspace: partials [ml: rows x splits x 2][o: rows x splits x head_dim] fp32 inside a region
// sized for kMaxDecodeSplits and the largest head_dim (128), then per-(sequence, kv head)
// arrival counters (rows of them, which is at least batch * kv_heads), 256-B aligned. The
// counters sit at the same offset for every head_dim, so one workspace may serve calls of both
// head sizes: no call's partials overlap another's counters.
constexpr int64_t kMaxDecodeHeadDim = 128;
size_t partialBytes(int64_t rows) {
  return alignUp(static_cast<size_t>(rows) * kMaxDecodeSplits * (2 + kMaxDecodeHeadDim) *
                     sizeof(float),
                 256);
}

}  // namespace

// Splits of `units` workgroup units whose blocks are dealt over `wph` waves per head: about one
// workgroup per CU, no more splits than groups of wph blocks, never fewer than the per-lane
// block ids of a wave (64) allow.
int decodeAttentionSplits(int64_t units, int64_t max_blocks, int cus, int wph, int requested) {
  int64_t splits = requested > 0 ? requested : (units > 0 ? cus / units : 1);
  const int64_t useful = (max_blocks + wph - 1) / wph;
  if (splits > useful) splits = useful;
  const int64_t needed = (max_blocks + wph * 64 - 1) / (wph * 64);
  if (splits < needed) splits = needed;
  if (splits < 1) splits = 1;
  return static_cast<int>(splits);
}

int decodeAttentionFast(int dtype, const void* q, const void* key_pool, const void* value_pool,
                        const int32_t* block_table, void* out, int64_t batch, int64_t q_heads,
                        int64_t kv_heads, int64_t seq_q, int64_t head_dim, int64_t block_size,
                        int64_t max_blocks, int64_t past, const void* positions,
                        int positions_dtype, float scale, int requested_splits, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (dtype != DLI_BF16 || seq_q != 1 || (head_dim != 64 && head_dim != 128) ||
      q_heads / kv_heads > 16 || block_size != kDecBlock || !aligned16(q))
    return 1;
  if (batch * kv_heads > 65535) return 1;
  int cus = 0;
  if (int rc = computeUnits(&cus)) return rc;
  // head_dim 128: every kv head of a sequence in one workgroup when they divide its 8 waves (the
  // workgroup then reads whole cache blocks of the pools)
  const int hpw = head_dim == 128 && kDecWaves % kv_heads == 0 ? static_cast<int>(kv_heads) : 1;
  const int splits =
      decodeAttentionSplits(batch * kv_heads / hpw, max_blocks, cus, kDecWaves / hpw,
                            requested_splits);
  if (splits > kMaxDecodeSplits) return 1;
  const int64_t rows = batch * q_heads;
  const size_t need = partialBytes(rows) + static_cast<size_t>(rows) * sizeof(unsigned);
  if (splits > 1 && (workspace == nullptr || workspace_bytes < need)) return 1;
  float* ws_ml = static_cast<float*>(workspace);
  float* ws_o = splits > 1 ? ws_ml + rows * splits * 2 : nullptr;
  unsigned* counters =
      splits > 1 ? reinterpret_cast<unsigned*>(static_cast<char*>(workspace) +
                                               partialBytes(rows))
                 : nullptr;
  const int pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  const float scale_log2 = scale * 1.4426950408889634f;
  if (head_dim == 128)
    return launch(k_dec_attn128,
                  {static_cast<unsigned>(splits), static_cast<unsigned>(batch * kv_heads / hpw)},
                  {kDecWaves * 64}, 0, stream, static_cast<const uint16_t*>(q),
                  static_cast<const uint16_t*>(key_pool), static_cast<const uint16_t*>(value_pool),
                  block_table, positions, pos64, past, ws_ml, ws_o, counters,
                  static_cast<uint16_t*>(out), static_cast<int>(q_heads),
                  static_cast<int>(kv_heads), max_blocks, splits, scale_log2, hpw);
  return launch(k_dec_attn, {static_cast<unsigned>(splits), static_cast<unsigned>(batch * kv_heads)},
                {kDecWaves * 64}, 0, stream, static_cast<const uint16_t*>(q),
                static_cast<const uint16_t*>(key_pool), static_cast<const uint16_t*>(value_pool),
                block_table, positions, pos64, past, ws_ml, ws_o, counters,
                static_cast<uint16_t*>(out), static_cast<int>(q_heads), static_cast<int>(kv_heads),
                max_blocks, splits, scale_log2);
}

size_t decodeAttentionWorkspace(int64_t batch, int64_t q_heads, int64_t seq_q, int64_t head_dim,
                                int64_t max_tokens) {
  if (seq_q != 1 || (head_dim != 64 && head_dim != 128)) return 0;
  const int64_t rows = batch * q_heads;
  return partialBytes(rows) + static_cast<size_t>(rows) * sizeof(unsigned);
}

}  // namespace dli::hip
